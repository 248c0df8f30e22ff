// ceiling.hip -- measurement kernels for bench.py's ceiling leg (gfx950),
// and the seeded generator of bench.py's synthetic inputs.
//
// Built into its own library (libluxgpu_ceiling.so), not into the plugin.
// They bound what any single launch of the decode GEMV can show on this
// hardware, timed exactly as the GEMV is:
//   * an empty kernel: the fixed cost of one launch (dispatch and
//     completion), with no memory traffic;
//   * a plain read of `bytes` bytes: every lane issues eight 128-bit loads at
//     once (each wave instruction reads 1 KB contiguous, whole 128-byte
//     lines) with the non-temporal cache policy, the fastest single-launch
//     read pattern measured for 33 MB; the words are folded and stored only
//     if they equal a value random data does not produce, so the loads stay.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace {

typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}

constexpr int kLoads = 8;          // 128-bit loads per lane
constexpr int kThreads = 256;
constexpr int kBlockBytes = kThreads * kLoads * 16;

__global__ __launch_bounds__(kThreads) void ceiling_empty_kernel(uint32_t* sink, int never) {
    if (never == 0x7fffffff) sink[blockIdx.x] = threadIdx.x;
}

__global__ __launch_bounds__(kThreads) void ceiling_read_kernel(const uint8_t* base, uint32_t bytes, uint32_t* sink) {
    // offsets past `bytes` read zeros
    const auto r = rsrc(base, bytes);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t wbase = ((uint32_t)blockIdx.x * (kThreads / 64) + wave) * kLoads * 1024u;
    v4u32 v[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; i++) v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, wbase + i * 1024 + lane * 16, 0, 2);
    v4u32 acc = v[0];
#pragma unroll
    for (int i = 1; i < kLoads; i++) acc = (acc ^ v[i]) + (v[i] << 1);
    if (acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u && acc.z == 0x85ebca6bu) sink[blockIdx.x] = acc.w;
}

}  // namespace

extern "C" {

// One launch of the empty kernel with `blocks` blocks of 256 threads on
// `stream`; sink: any device buffer of >= 4 * blocks bytes (never written).
// Returns the hipError_t of the launch.
__attribute__((visibility("default"))) int lux_ceiling_empty(int blocks, void* sink, void* stream) {
    if (blocks <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(ceiling_empty_kernel, dim3(blocks), dim3(kThreads), 0, (hipStream_t)stream,
                       static_cast<uint32_t*>(sink), 0);
    return (int)hipGetLastError();
}

// One launch of the plain read of `bytes` bytes at `buf` (< 2^31) on
// `stream`; sink: a device buffer of >= 4 * ceil(bytes / 32 KiB) bytes (never
// written in practice).  Returns the hipError_t of the launch.
__attribute__((visibility("default"))) int lux_ceiling_read(const void* buf, uint64_t bytes, void* sink,
                                                            void* stream) {
    if (buf == nullptr || bytes == 0 || bytes >= (1ull << 31)) return (int)hipErrorInvalidValue;
    const int blocks = (int)((bytes + kBlockBytes - 1) / kBlockBytes);
    hipLaunchKernelGGL(ceiling_read_kernel, dim3(blocks), dim3(kThreads), 0, (hipStream_t)stream,
                       static_cast<const uint8_t*>(buf), (uint32_t)bytes, static_cast<uint32_t*>(sink));
    return (int)hipGetLastError();
}

// Launches i = first .. first + n - 1 of the plain read, launch i reading
// the `bytes` bytes at base + (i % copies) * stride, from this C loop (the
// way bench.py issues the timed quantized-matmul launches).  Returns the
// first hipError_t met.
__attribute__((visibility("default"))) int lux_ceiling_read_loop(const void* base, uint64_t stride, int copies,
                                                                 uint64_t bytes, void* sink, void* stream, int first,
                                                                 int n) {
    if (copies <= 0 || n < 0 || first < 0) return (int)hipErrorInvalidValue;
    for (int i = first; i < first + n; i++) {
        const int rc = lux_ceiling_read(static_cast<const uint8_t*>(base) + (uint64_t)(i % copies) * stride, bytes,
                                        sink, stream);
        if (rc != 0) return rc;
    }
    return 0;
}

// `n` launches of the empty kernel (`blocks` blocks) issued back to back
// from this C loop, between two events on `stream`: the per-launch floor
// without a Python call per launch.  *ms_out: the events' elapsed time.
// Returns the first hipError_t met.
__attribute__((visibility("default"))) int lux_ceiling_empty_loop(int n, int blocks, void* sink, void* stream,
                                                                  float* ms_out) {
    if (n <= 0 || blocks <= 0 || ms_out == nullptr) return (int)hipErrorInvalidValue;
    const hipStream_t st = (hipStream_t)stream;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipEventRecord(e0, st);
    for (int i = 0; i < n && e == hipSuccess; i++) {
        hipLaunchKernelGGL(ceiling_empty_kernel, dim3(blocks), dim3(kThreads), 0, st, static_cast<uint32_t*>(sink), 0);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipEventRecord(e1, st);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(ms_out, e0, e1);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    return (int)e;
}

// The plugin's op_quantized_matmul_ex (lux_gpu_quant_backend.h), called
// through the pointer the quant table holds: opaque context and buffer
// handles, then the shape, the dtypes and the kernel choice as ints.
typedef int (*LuxQmmExFn)(void* ctx, void* x, void* w_q, void* scales, void* biases, void* out, int M, int K,
                          int N, int group_size, int bits, int x_dtype, int sb_dtype, int out_dtype, int kernel);

// Calls i = first .. first + n - 1 of the op from this C loop, call i on
// weight set i % copies (w_q[], scales[], biases[] hold `copies` handles),
// the way a C caller drives the op, with no Python call per launch: what
// bench.py times.  Returns the op's first non-zero status, else 0.
__attribute__((visibility("default"))) int lux_bench_qmm_loop(void* fn, void* ctx, void* x, void* const* w_q,
                                                              void* const* scales, void* const* biases,
                                                              int copies, void* out, int M, int K, int N,
                                                              int group_size, int bits, int x_dtype, int sb_dtype,
                                                              int out_dtype, int kernel, int first, int n) {
    if (fn == nullptr || copies <= 0 || n < 0 || first < 0) return (int)hipErrorInvalidValue;
    const LuxQmmExFn op = reinterpret_cast<LuxQmmExFn>(fn);
    for (int i = first; i < first + n; i++) {
        const int c = i % copies;
        const int rc = op(ctx, x, w_q[c], scales[c], biases[c], out, M, K, N, group_size, bits, x_dtype, sb_dtype,
                          out_dtype, kernel);
        if (rc != 0) return rc;
    }
    return 0;
}

}  // extern "C"

// ---- synthetic inputs ------------------------------------------------------
// The portable generator the test fixtures are made with (their SHA-256
// digests are committed), so that bench.py times the same tensors:
// xoshiro256** seeded through splitmix64; normals by Box-Muller on 53-bit
// uniforms u1 in (0, 1], u2 in [0, 1), two per pair of draws.

namespace {
uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
struct Xoshiro {
    uint64_t s[4];
    explicit Xoshiro(uint64_t seed) {
        uint64_t sm = seed;
        for (int i = 0; i < 4; i++) s[i] = splitmix64(&sm);
    }
    static uint64_t rotl(uint64_t v, int k) { return (v << k) | (v >> (64 - k)); }
    uint64_t next() {
        const uint64_t r = rotl(s[1] * 5, 7) * 9, t = s[1] << 17;
        s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }
};
}  // namespace

extern "C" {

// n normals of mean `mean` and deviation `stddev` into out (host memory)
__attribute__((visibility("default"))) void lux_bench_rng_normal_f32(float* out, size_t n, uint64_t seed, float mean,
                                                                     float stddev) {
    Xoshiro x(seed);
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = (double)((x.next() >> 11) + 1) * 0x1.0p-53;
        const double u2 = (double)(x.next() >> 11) * 0x1.0p-53;
        const double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + stddev * (r * cos(two_pi * u2)));
        if (i + 1 < n) out[i + 1] = (float)(mean + stddev * (r * sin(two_pi * u2)));
    }
}

// n uniform 32-bit words (the high halves of the draws) into out
__attribute__((visibility("default"))) void lux_bench_rng_u32(uint32_t* out, size_t n, uint64_t seed) {
    Xoshiro x(seed);
    for (size_t i = 0; i < n; i++) out[i] = (uint32_t)(x.next() >> 32);
}

}  // extern "C"
