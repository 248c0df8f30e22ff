// qnoalloc.hip -- the allocation-free quantized matmul entry point.
//
// lux_gpu_quantized_matmul_noalloc runs op_quantized_matmul_ex's kernels on
// caller-owned device pointers and a caller stream, with no context: it
// calls no allocating routine, for callers that cannot (code under graph
// capture, serving loops that forbid allocation).  The kernels that need
// device memory beyond their operands -- the split-K small-M GEMM and the
// large GEMM's split last round (partial sums, tile counters and flags) --
// take it from `scratch` below: a static device array that each GPU holds
// from module load until the process ends.  Its size is the context
// workspace's, so a shape takes the same K split, and gives the same bits,
// on both entry points.
#include <hip/hip_runtime.h>

#include <mutex>

#include "qdispatch.h"

static __device__ __align__(256) uint8_t scratch[lxq::kSplitWorkspaceBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
// device address of this device's `scratch` (the array's name in host code
// is a host-side stand-in, not a device address); null until set up
void* g_scratch[kMaxDevices] = {nullptr};
// launches on each device's scratch so far (the GEMMs' split tiles meet by
// this launch number, never 0)
uint32_t g_epoch[kMaxDevices] = {0};

__global__ void clear_words(uint32_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

// once per device, with that device current: look up the array's device
// address and clear it (a kernel on `st`, ordered before this call's work;
// the GEMMs return their counters and flags to zero after every launch).
// That first call must not be under stream capture: the clear would become
// a node of the caller's graph and run on every replay, after later calls
// have relied on the array being clear once.  It is refused instead.
LuxBackendError scratch_on(int dev, hipStream_t st, void** out, uint32_t* epoch) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_scratch[dev] == nullptr) {
        if (!lux_hip_is_gfx950(dev)) return LUX_BACKEND_ERROR_NOT_SUPPORTED;
        // (a stream the query rejects is left to the launch below to report)
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cap) != hipSuccess) {
            (void)hipGetLastError();
            cap = hipStreamCaptureStatusNone;
        }
        if (cap != hipStreamCaptureStatusNone) return LUX_BACKEND_ERROR_NOT_SUPPORTED;
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            return LUX_BACKEND_ERROR_INTERNAL;
        }
        hipLaunchKernelGGL(clear_words, dim3(1024), dim3(256), 0, st, static_cast<uint32_t*>(p),
                           lxq::kSplitWorkspaceBytes / 4);
        if (hipGetLastError() != hipSuccess) return LUX_BACKEND_ERROR_INTERNAL;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    if (++g_epoch[dev] == 0u) g_epoch[dev] = 1u;
    *epoch = g_epoch[dev];
    return LUX_BACKEND_OK;
}

}  // namespace

extern "C" __attribute__((visibility("default"))) LuxBackendError lux_gpu_quantized_matmul_noalloc(
    const void* x, const void* w_q, const void* scales, const void* biases, void* out, int M, int K, int N,
    int group_size, int bits, LuxBackendDtype x_dtype, LuxBackendDtype sb_dtype, LuxBackendDtype out_dtype,
    LuxQuantKernel kernel, void* stream) {
    if (!x || !w_q || !scales || !biases || !out) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    LuxBackendError e = lux_hip_qmm_validate(M, K, N, group_size, bits, x_dtype, sb_dtype, out_dtype, kernel);
    if (e != LUX_BACKEND_OK) return e;
    if (M == 0 || N == 0) return LUX_BACKEND_OK;
    // the scratch bounds the K split; a shape whose split would need more
    // is refused (the split rule lowers the split to fit, so none does)
    if (lxq::qgemm_sk_workspace(M, K, N, bits, x_dtype, lxq::kSplitWorkspaceBytes) > lxq::kSplitWorkspaceBytes)
        return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return LUX_BACKEND_ERROR_DEVICE_LOST;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    void* ws = nullptr;
    uint32_t epoch = 0;
    e = scratch_on(dev, st, &ws, &epoch);
    if (e != LUX_BACKEND_OK) return e;

    lxq::QmmArgs a;
    a.x = x;
    a.wq = static_cast<const uint32_t*>(w_q);
    a.scales = scales;
    a.biases = biases;
    a.y = out;
    a.M = M; a.K = K; a.N = N; a.group_size = group_size; a.bits = bits;
    a.x_dtype = x_dtype; a.sb_dtype = sb_dtype; a.out_dtype = out_dtype;
    a.ws = ws;
    a.ws_bytes = lxq::kSplitWorkspaceBytes;
    a.epoch = epoch;
    return lux_hip_qmm_dispatch(a, kernel, st);
}
