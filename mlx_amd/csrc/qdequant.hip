// qdequant.hip -- format kernels: dequantize, quantize, and the generic
// one-thread-per-output matmul used for shapes the tiled kernels reject.
#include "kernels.h"
#include "qcommon.h"

namespace lxq {

namespace {

// code k of a row, runtime bit width
__device__ __forceinline__ uint32_t row_code(const uint32_t* __restrict__ row, int k, int bits) {
    const uint32_t bit = (uint32_t)k * (uint32_t)bits, wi = bit >> 5, sh = bit & 31u;
    uint64_t pair = row[wi];
    if (sh + (uint32_t)bits > 32u) pair |= (uint64_t)row[wi + 1] << 32;
    return (uint32_t)(pair >> sh) & ((1u << bits) - 1u);
}

__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ wq,
                                                      const void* __restrict__ sc,
                                                      const void* __restrict__ bi,
                                                      void* __restrict__ out, int N, int K,
                                                      int gsize, int bits, int sb_dt, int out_dt) {
    const size_t total = (size_t)N * K;
    const int G = K / gsize, rw = (K * bits) >> 5;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int n = (int)(i / K), k = (int)(i - (size_t)n * K);
        const uint32_t q = row_code(wq + (size_t)n * rw, k, bits);
        const size_t gi = (size_t)n * G + k / gsize;
        store_f(out, i, out_dt, fmaf(load_f(sc, gi, sb_dt), (float)q, load_f(bi, gi, sb_dt)));
    }
}

// Quantizer.  Lane t takes the 8 consecutive weights 8t .. 8t+7 of the
// row-major [N, K] matrix (one 16- or 32-byte load; a wave reads 512
// consecutive weights), so a group of GS weights spans GS/8 adjacent lanes
// and 8 codes of BITS bits are exactly BITS bytes at byte 8t*BITS/8 of the
// packed stream (rows are contiguous in both).  Per group, following the
// CPU quantizer's sequential scan (oracle/lux_cpu_quant.c, lux_cpu_quantize):
// mn/mx start at the group's first weight and take a later weight only if
// strictly smaller/larger, so a NaN first weight poisons the group and later
// NaNs are skipped, and ties keep the first occurrence.  The lanes of a group
// combine their partial results in index order (the lower segment wins
// ties); lanes other than the group's first start from +inf / -inf.
template <int WDT>
__device__ __forceinline__ void load8(const void* w, size_t e, float (&v)[8]) {
    if constexpr (WDT == DT_F32) {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(w) + e);
        const float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w) + e);
        const uint32_t d[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[2 * i] = WDT == DT_F16 ? f16_to_f32(d[i] & 0xffffu) : bf16_to_f32(d[i] & 0xffffu);
            v[2 * i + 1] = WDT == DT_F16 ? f16_to_f32(d[i] >> 16) : bf16_to_f32(d[i] >> 16);
        }
    }
}

template <int BITS, int WDT>
__global__ __launch_bounds__(256) void quantize_kernel(const void* __restrict__ w, uint32_t* __restrict__ wq,
                                                       void* __restrict__ sc, void* __restrict__ bi,
                                                       size_t chunks, int gsize, int sb_dt) {
    __shared__ __attribute__((aligned(16))) uint8_t pk[4][64 * 8];  // per wave: 64 lanes x BITS bytes
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t t0 = ((size_t)blockIdx.x * 4 + wave) * 64;  // first chunk of this wave
    const size_t t = t0 + lane;
    const bool act = t < chunks;
    const int L = gsize >> 3;    // lanes per group (4, 8 or 16; groups start at lane multiples of L)
    const int lig = lane & (L - 1);
    float v[8];
    if (act) {
        load8<WDT>(w, 8 * t, v);
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = 0.f;
    }
    float mn = lig == 0 ? v[0] : __builtin_inff(), mx = lig == 0 ? v[0] : -__builtin_inff();
#pragma unroll
    for (int i = 0; i < 8; i++) {
        mn = v[i] < mn ? v[i] : mn;
        mx = v[i] > mx ? v[i] : mx;
    }
    for (int d = 1; d < L; d <<= 1) {
        const float omn = __shfl_xor(mn, d), omx = __shfl_xor(mx, d);
        const bool up = lane & d;  // this lane holds the upper (later) segment
        const float lmn = up ? omn : mn, umn = up ? mn : omn;
        const float lmx = up ? omx : mx, umx = up ? mx : omx;
        mn = umn < lmn ? umn : lmn;
        mx = umx > lmx ? umx : lmx;
    }
    const float levels = (float)((1u << BITS) - 1u);
    // the codes are computed from the stored (rounded) scale and bias
    const float s = round_dt((mx - mn) / levels, sb_dt), b = round_dt(mn, sb_dt);
    if (act && lig == 0) {
        const size_t gi = 8 * t / (size_t)gsize;
        store_f(sc, gi, sb_dt, s);
        store_f(bi, gi, sb_dt, b);
    }
    uint64_t chunk = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint32_t q = 0;
        if (s != 0.0f) {
            float r = rintf((v[i] - b) / s);
            r = (r >= 0.0f) ? r : 0.0f;  // NaN -> 0
            r = r > levels ? levels : r;
            q = (uint32_t)r;
        }
        chunk |= (uint64_t)q << (i * BITS);
    }
    // the wave's packed bytes are contiguous: stage them in LDS, store whole dwords
#pragma unroll
    for (int y = 0; y < BITS; y++) pk[wave][lane * BITS + y] = (uint8_t)(chunk >> (8 * y));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // this wave's bytes [t0 BITS, min(t0 + 64, chunks) BITS): whole dwords, since
    // both ends are multiples of 4 (64 BITS, and N K BITS / 8 with K % 32 == 0)
    if (t0 < chunks) {
        const int nwords = (int)((chunks - t0 < 64) ? (chunks - t0) : 64) * BITS / 4;  // up to 16 BITS
        for (int i = lane; i < nwords; i += 64)
            wq[t0 * BITS / 4 + i] = reinterpret_cast<const uint32_t*>(pk[wave])[i];
    }
}

// y[m, n] = sum_k x * fmaf(s, q, b): fp32, ascending k, separate multiply and
// add (no contraction), the same order as the CPU oracle
__global__ __launch_bounds__(256) void qmm_generic_kernel(const void* __restrict__ x,
                                                          const uint32_t* __restrict__ wq,
                                                          const void* __restrict__ sc,
                                                          const void* __restrict__ bi,
                                                          void* __restrict__ y, int M, int K,
                                                          int N, int gsize, int bits, int x_dt,
                                                          int sb_dt, Epilogue ep) {
#pragma clang fp contract(off)
    const size_t total = (size_t)M * N;
    const int G = K / gsize, rw = (K * bits) >> 5;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int n = (int)(i % N), m = (int)(i / N);
        const uint32_t* row = wq + (size_t)n * rw;
        float acc = 0.f;
        for (int k = 0; k < K; k++) {
            const size_t gi = (size_t)n * G + k / gsize;
            const float wv = fmaf(load_f(sc, gi, sb_dt), (float)row_code(row, k, bits),
                                  load_f(bi, gi, sb_dt));
            acc = acc + load_f(x, (size_t)m * K + k, x_dt) * wv;
        }
        store_out<true>(y, i, n, ep, acc);
    }
}

unsigned grid_for(size_t total) {
    size_t b = (total + 255) / 256;
    return (unsigned)(b < 65536 ? (b ? b : 1) : 65536);
}

}  // namespace

LuxStatus launch_dequantize(const uint32_t* wq, const void* scales, const void* biases, void* out,
                            int N, int K, int group_size, int bits, int sb_dtype, int out_dtype,
                            hipStream_t st) {
    if ((size_t)N * K == 0) return LuxStatus::Ok;
    hipLaunchKernelGGL(dequant_kernel, dim3(grid_for((size_t)N * K)), dim3(256), 0, st, wq, scales,
                       biases, out, N, K, group_size, bits, sb_dtype, out_dtype);
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

namespace {
template <int BITS, int WDT>
void launch_quantize_t(const void* w, uint32_t* wq, void* scales, void* biases, size_t chunks, int group_size,
                       int sb_dtype, hipStream_t st) {
    const size_t blocks = (chunks + 255) / 256;
    hipLaunchKernelGGL((quantize_kernel<BITS, WDT>), dim3((unsigned)blocks), dim3(256), 0, st, w, wq, scales, biases,
                       chunks, group_size, sb_dtype);
}
template <int WDT>
LuxStatus launch_quantize_w(const void* w, uint32_t* wq, void* sc, void* bi, size_t chunks, int gs, int bits,
                            int sb, hipStream_t st) {
    switch (bits) {
    case 2: launch_quantize_t<2, WDT>(w, wq, sc, bi, chunks, gs, sb, st); break;
    case 3: launch_quantize_t<3, WDT>(w, wq, sc, bi, chunks, gs, sb, st); break;
    case 4: launch_quantize_t<4, WDT>(w, wq, sc, bi, chunks, gs, sb, st); break;
    case 5: launch_quantize_t<5, WDT>(w, wq, sc, bi, chunks, gs, sb, st); break;
    case 6: launch_quantize_t<6, WDT>(w, wq, sc, bi, chunks, gs, sb, st); break;
    case 8: launch_quantize_t<8, WDT>(w, wq, sc, bi, chunks, gs, sb, st); break;
    default: return LuxStatus::NotSupported;
    }
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}
}  // namespace

LuxStatus launch_quantize(const void* w, uint32_t* wq, void* scales, void* biases, int N, int K,
                          int group_size, int bits, int w_dtype, int sb_dtype, hipStream_t st) {
    const size_t chunks = (size_t)N * K / 8;  // 8 weights per lane; group sizes are 32, 64, 128
    if (chunks == 0) return LuxStatus::Ok;
    if (group_size != 32 && group_size != 64 && group_size != 128) return LuxStatus::NotSupported;
    // one block per 256 lanes: the grid's x dimension holds up to 2^31 - 1 blocks
    if ((chunks + 255) / 256 >= (1ull << 31)) return LuxStatus::NotSupported;
    switch (w_dtype) {
    case DT_F32: return launch_quantize_w<DT_F32>(w, wq, scales, biases, chunks, group_size, bits, sb_dtype, st);
    case DT_F16: return launch_quantize_w<DT_F16>(w, wq, scales, biases, chunks, group_size, bits, sb_dtype, st);
    default: return launch_quantize_w<DT_BF16>(w, wq, scales, biases, chunks, group_size, bits, sb_dtype, st);
    }
}

LuxStatus launch_qmm_generic(const QmmArgs& a, hipStream_t st) {
    const size_t total = (size_t)a.M * a.N;
    if (total == 0) return LuxStatus::Ok;
    if (planned(a, "qmm_generic_kernel")) return LuxStatus::Ok;
    hipLaunchKernelGGL(qmm_generic_kernel, dim3(grid_for(total)), dim3(256), 0, st, a.x, a.wq,
                       a.scales, a.biases, a.y, a.M, a.K, a.N, a.group_size, a.bits, a.x_dtype,
                       a.sb_dtype, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

}  // namespace lxq
