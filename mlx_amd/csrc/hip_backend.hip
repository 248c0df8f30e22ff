// hip_backend.hip -- host side of libluxgpu_backend_hip.so.
//
// Implements the Lux GPU backend plugin ABI v2 (include/lux_gpu_backend_abi.h,
// layout-identical to reference include/lux/gpu/backend_plugin.h) over HIP:
//   context = one gfx950 device + one non-blocking stream,
//   buffer  = one hipMalloc allocation with kTailPad zeroed bytes of slack
//             past its end (kernels may read whole 16-byte chunks there),
// and the additive quantized-matmul extension (include/lux_gpu_quant_backend.h).
//
// Semantics follow the reference's built-in CPU backend where the ABI leaves
// them open (reference src/cpu_backend.cpp:121-165): buffer_alloc zero-fills,
// copies move min(bytes, buffer size) bytes and succeed, copy-to-host blocks
// and is ordered after all work queued on the context (the reference core
// reads results without calling sync first, src/gpu_core.cpp:399-403).
// No C++ exception crosses the C ABI.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <new>

#include "../../include/lux_gpu_backend_abi.h"
#include "../../include/lux_gpu_quant_backend.h"
#include "kernels.h"
#include "qdispatch.h"
#include "qweights.h"

namespace {

struct HipContext {
    int device = 0;
    hipStream_t stream = nullptr;
    char name[256] = {0};
    int compute_units = 0;
    int max_wg = 0;
    // kernel workspace (partial sums and self-resetting tile counters and
    // flags of the split-K small-M GEMM and of the large GEMM's split last
    // round), allocated and zeroed once here so that no launch
    // allocates; used only by work on `stream`, which orders its users
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // launches on ws so far: each GEMM launch gets the next number as its
    // epoch (the split tiles meet by it; never 0)
    uint32_t epoch = 0;
};


struct HipBuffer {
    void* ptr = nullptr;
    size_t size = 0;
};

HipContext* C(LuxBackendContext* c) { return reinterpret_cast<HipContext*>(c); }
HipBuffer* B(LuxBackendBuffer* b) { return reinterpret_cast<HipBuffer*>(b); }

LuxBackendError map_err(hipError_t e) {
    switch (e) {
    case hipSuccess: return LUX_BACKEND_OK;
    case hipErrorOutOfMemory: return LUX_BACKEND_ERROR_OUT_OF_MEMORY;
    case hipErrorInvalidValue: return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    case hipErrorNoDevice:
    case hipErrorInvalidDevice: return LUX_BACKEND_ERROR_DEVICE_LOST;
    default: return LUX_BACKEND_ERROR_INTERNAL;
    }
}

LuxBackendError map_status(lxq::LuxStatus s) {
    switch (s) {
    case lxq::LuxStatus::Ok: return LUX_BACKEND_OK;
    case lxq::LuxStatus::Invalid: return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    case lxq::LuxStatus::OutOfMemory: return LUX_BACKEND_ERROR_OUT_OF_MEMORY;
    case lxq::LuxStatus::NotSupported: return LUX_BACKEND_ERROR_NOT_SUPPORTED;
    default: return LUX_BACKEND_ERROR_INTERNAL;
    }
}

bool is_gfx950(int dev) { return lux_hip_is_gfx950(dev); }

// ---------------------------------------------------------------------------
// lifecycle, device info, sync
// ---------------------------------------------------------------------------

LuxBackendContext* hip_create_context(int device_index) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device_index < 0 || device_index >= count)
        return nullptr;
    if (!is_gfx950(device_index)) return nullptr;
    if (hipSetDevice(device_index) != hipSuccess) return nullptr;
    HipContext* ctx = new (std::nothrow) HipContext();
    if (!ctx) return nullptr;
    ctx->device = device_index;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device_index) != hipSuccess ||
        hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return nullptr;
    }
    std::snprintf(ctx->name, sizeof(ctx->name), "%s (%s)", p.name, p.gcnArchName);
    ctx->compute_units = p.multiProcessorCount;
    ctx->max_wg = p.maxThreadsPerBlock;
    // without a workspace the kernels that need one are skipped
    if (hipMalloc(&ctx->ws, lxq::kSplitWorkspaceBytes) == hipSuccess) {
        if (hipMemset(ctx->ws, 0, lxq::kSplitWorkspaceBytes) == hipSuccess) {
            ctx->ws_bytes = lxq::kSplitWorkspaceBytes;
        } else {
            hipFree(ctx->ws);
            ctx->ws = nullptr;
        }
    } else {
        (void)hipGetLastError();
        ctx->ws = nullptr;
    }
    return reinterpret_cast<LuxBackendContext*>(ctx);
}

void hip_destroy_context(LuxBackendContext* c) {
    HipContext* ctx = C(c);
    if (!ctx) return;
    hipSetDevice(ctx->device);
    if (ctx->stream) {
        hipStreamSynchronize(ctx->stream);
        hipStreamDestroy(ctx->stream);
    }
    if (ctx->ws) hipFree(ctx->ws);
    delete ctx;
}

LuxBackendError hip_get_device_count(int* count) {
    if (!count) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    int ok = 0;
    for (int d = 0; d < n; d++) ok += is_gfx950(d) ? 1 : 0;
    *count = ok;
    return LUX_BACKEND_OK;
}

LuxBackendError hip_get_device_info(LuxBackendContext* c, LuxBackendDeviceInfo* info) {
    HipContext* ctx = C(c);
    if (!ctx || !info) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    hipSetDevice(ctx->device);
    size_t free_b = 0, total_b = 0;
    hipError_t e = hipMemGetInfo(&free_b, &total_b);
    if (e != hipSuccess) return map_err(e);
    info->name = ctx->name;
    info->vendor = "AMD";
    info->memory_total = total_b;
    info->memory_available = free_b;
    info->compute_units = ctx->compute_units;
    info->max_workgroup_size = ctx->max_wg;
    info->is_discrete = true;
    info->is_unified_memory = false;
    return LUX_BACKEND_OK;
}

LuxBackendError hip_sync(LuxBackendContext* c) {
    HipContext* ctx = C(c);
    if (!ctx) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    return map_err(hipStreamSynchronize(ctx->stream));
}

// ---------------------------------------------------------------------------
// buffers
// ---------------------------------------------------------------------------

LuxBackendBuffer* hip_buffer_alloc(LuxBackendContext* c, size_t bytes) {
    HipContext* ctx = C(c);
    if (!ctx) return nullptr;
    hipSetDevice(ctx->device);
    HipBuffer* b = new (std::nothrow) HipBuffer();
    if (!b) return nullptr;
    b->size = bytes;
    if (bytes) {
        if (hipMalloc(&b->ptr, bytes + lxq::kTailPad) != hipSuccess) {
            delete b;
            return nullptr;
        }
        // zero-filled like the reference CPU backend (src/cpu_backend.cpp:129),
        // tail slack included; ordered before any later work on the context stream
        if (hipMemsetAsync(b->ptr, 0, bytes + lxq::kTailPad, ctx->stream) != hipSuccess) {
            hipFree(b->ptr);
            delete b;
            return nullptr;
        }
    }
    return reinterpret_cast<LuxBackendBuffer*>(b);
}

LuxBackendBuffer* hip_buffer_alloc_with_data(LuxBackendContext* c, const void* data, size_t bytes) {
    HipContext* ctx = C(c);
    if (!ctx || (bytes && !data)) return nullptr;
    hipSetDevice(ctx->device);
    HipBuffer* b = new (std::nothrow) HipBuffer();
    if (!b) return nullptr;
    b->size = bytes;
    if (bytes) {
        if (hipMalloc(&b->ptr, bytes + lxq::kTailPad) != hipSuccess) {
            delete b;
            return nullptr;
        }
        // the caller may free `data` on return: copy synchronously
        if (hipMemsetAsync(static_cast<uint8_t*>(b->ptr) + bytes, 0, lxq::kTailPad, ctx->stream) != hipSuccess ||
            hipMemcpyAsync(b->ptr, data, bytes, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
            hipStreamSynchronize(ctx->stream) != hipSuccess) {
            hipFree(b->ptr);
            delete b;
            return nullptr;
        }
    }
    return reinterpret_cast<LuxBackendBuffer*>(b);
}

void hip_buffer_free(LuxBackendContext* c, LuxBackendBuffer* buf) {
    HipBuffer* b = B(buf);
    if (!b) return;
    if (HipContext* ctx = C(c)) {
        hipSetDevice(ctx->device);
        // queued kernels may still read the buffer
        hipStreamSynchronize(ctx->stream);
    }
    if (b->ptr) hipFree(b->ptr);
    delete b;
}

LuxBackendError hip_buffer_copy_to_host(LuxBackendContext* c, LuxBackendBuffer* buf, void* dst,
                                        size_t bytes) {
    HipContext* ctx = C(c);
    HipBuffer* b = B(buf);
    if (!ctx || !b || !dst) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    const size_t n = std::min(bytes, b->size);
    if (!n) return LUX_BACKEND_OK;
    hipSetDevice(ctx->device);
    hipError_t e = hipMemcpyAsync(dst, b->ptr, n, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return map_err(e);
}

LuxBackendError hip_buffer_copy_from_host(LuxBackendContext* c, LuxBackendBuffer* buf,
                                          const void* src, size_t bytes) {
    HipContext* ctx = C(c);
    HipBuffer* b = B(buf);
    if (!ctx || !b || !src) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    const size_t n = std::min(bytes, b->size);
    if (!n) return LUX_BACKEND_OK;
    hipSetDevice(ctx->device);
    hipError_t e = hipMemcpyAsync(b->ptr, src, n, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return map_err(e);
}

void* hip_buffer_get_host_ptr(LuxBackendContext*, LuxBackendBuffer*) {
    return nullptr;  // discrete device memory: no host view
}

// ---------------------------------------------------------------------------
// quantized matmul extension
// ---------------------------------------------------------------------------

size_t dtype_size(int dt) { return dt == LUX_DTYPE_FLOAT32 ? 4 : 2; }
bool dtype_ok(int dt) {
    return dt == LUX_DTYPE_FLOAT32 || dt == LUX_DTYPE_FLOAT16 || dt == LUX_DTYPE_BFLOAT16;
}
bool bits_ok(int b) { return b == 2 || b == 3 || b == 4 || b == 5 || b == 6 || b == 8; }

// shared shape/format validation: OK, INVALID_ARGUMENT or NOT_SUPPORTED
LuxBackendError check_format(int K, int N, int group_size, int bits) {
    if (K <= 0 || N < 0) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (!bits_ok(bits)) return LUX_BACKEND_ERROR_NOT_SUPPORTED;
    if (group_size != 32 && group_size != 64 && group_size != 128)
        return LUX_BACKEND_ERROR_NOT_SUPPORTED;
    if (K % group_size) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    return LUX_BACKEND_OK;
}

bool fits(HipBuffer* b, size_t need) { return b && (need == 0 || (b->ptr && b->size >= need)); }

// M up to this value goes to the GEMV: LUX_HIP_GEMV_MAX_M when set, else 8,
// or 16 where the GEMV family's MFMA kernels take the shape (16-bit x, 4- or
// 8-bit codes, K % 1024 == 0).  There they measured faster than the small-M
// GEMM (graph replays): 4-bit K = 4096, N = 14336, M = 9 / 12 / 16 15.2 /
// 15.7 / 16.3 us against 21.0-21.2, N = 28672, M = 16 29.3 against 39.8;
// 8-bit K = 4096, N = 14336, M = 12 / 16 23.7 against 26.0 / 26.3, K = N =
// 8192 20.9 / 21.3 against 22.8 / 23.2.  3- and 6-bit codes at M = 16 run
// 2.2x slower on the GEMV side, so their crossover stays at 8.
int gemv_max_m(int K, int bits, LuxBackendDtype x_dtype) {
    static const int env = [] {
        const char* e = std::getenv("LUX_HIP_GEMV_MAX_M");
        if (!e || !*e) return -1;
        const int d = std::atoi(e);
        return d < 0 ? 0 : d;
    }();
    if (env >= 0) return env;
    const bool mfma_gemv = x_dtype != LUX_DTYPE_FLOAT32 && (bits == 4 || bits == 8) && K % 1024 == 0;
    return mfma_gemv ? 16 : 8;
}

// shapes the MFMA GEMMs take: 16-bit activations, and
//  * 8 < M <= 64 with K a multiple of 128 (split-K small-M kernel: its
//    super-steps are 128 codes of K; it runs unsplit without a workspace),
//    x, W and f32 scales below 2 GiB; or
//  * K a multiple of 256 (the large kernel's scale windows span 4 K steps of
//    64), x and W below 4 GiB (32-bit offsets), and its LDS buffers within
//    one CU's 160 KB (f32 scales at group size 32 with 6-bit codes, and with
//    8-bit codes where K % 1024 != 0, do
//    not fit)
bool gemm_ok(int M, int K, int N, int group_size, int bits, LuxBackendDtype x_dtype,
             LuxBackendDtype sb_dtype) {
    if (x_dtype == LUX_DTYPE_FLOAT32) return false;
    if (M > 8 && M <= 64 && K % 128 == 0 && (size_t)M * K * 2 < (1ull << 31) &&
        (size_t)N * K * bits / 8 < (1ull << 31) && (size_t)N * (K / 32) * 4 < (1ull << 31))
        return true;
    // (the register-W kernel, 4/8-bit codes with K % 1024 == 0, fits them all)
    if (sb_dtype == LUX_DTYPE_FLOAT32 && group_size == 32 && bits >= 6 && !(bits == 8 && K % 1024 == 0))
        return false;
    return K % 256 == 0 && (size_t)M * K * 2 < (1ull << 32) && (size_t)N * K * bits / 8 < (1ull << 32);
}

LuxQuantKernel select_kernel_impl(int M, int K, int N, int group_size, int bits,
                                  LuxBackendDtype x_dtype, LuxBackendDtype sb_dtype) {
    if (M <= gemv_max_m(K, bits, x_dtype) || !gemm_ok(M, K, N, group_size, bits, x_dtype, sb_dtype))
        return LUX_QMM_KERNEL_GEMV;
    return LUX_QMM_KERNEL_GEMM;
}

}  // namespace

bool lux_hip_is_gfx950(int dev) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) return false;
    return std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
}

LuxBackendError lux_hip_qmm_validate(int M, int K, int N, int group_size, int bits, int x_dtype, int sb_dtype,
                                     int out_dtype, int kernel) {
    if (M < 0) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    LuxBackendError e = check_format(K, N, group_size, bits);
    if (e != LUX_BACKEND_OK) return e;
    if (!dtype_ok(x_dtype) || !dtype_ok(sb_dtype) || !dtype_ok(out_dtype)) return LUX_BACKEND_ERROR_NOT_SUPPORTED;
    if (kernel != LUX_QMM_KERNEL_AUTO && kernel != LUX_QMM_KERNEL_GEMV && kernel != LUX_QMM_KERNEL_GEMM)
        return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    return LUX_BACKEND_OK;
}

LuxBackendError lux_hip_qmm_dispatch(const lxq::QmmArgs& a, int kernel, hipStream_t st) {
    const LuxBackendDtype xd = (LuxBackendDtype)a.x_dtype, sd = (LuxBackendDtype)a.sb_dtype;
    if (kernel == LUX_QMM_KERNEL_AUTO) kernel = select_kernel_impl(a.M, a.K, a.N, a.group_size, a.bits, xd, sd);
    if (kernel == LUX_QMM_KERNEL_GEMM) {
        // an explicit GEMM request runs the GEMM or fails: its numerics
        // (weights rounded to the activation type) differ from the GEMV's
        if (!gemm_ok(a.M, a.K, a.N, a.group_size, a.bits, xd, sd)) return LUX_BACKEND_ERROR_NOT_SUPPORTED;
        return map_status(lxq::launch_qgemm(a, st));
    }
    if (a.K % 64 == 0) {
        lxq::LuxStatus s = lxq::launch_qgemv(a, st);
        if (s != lxq::LuxStatus::NotSupported) return map_status(s);
    }
    return map_status(lxq::launch_qmm_generic(a, st));
}

namespace {

LuxBackendError qmm_impl(LuxBackendContext* c, LuxBackendBuffer* x, LuxBackendBuffer* w_q,
                         LuxBackendBuffer* scales, LuxBackendBuffer* biases,
                         LuxBackendBuffer* out, int M, int K, int N, int group_size, int bits,
                         LuxBackendDtype x_dtype, LuxBackendDtype sb_dtype,
                         LuxBackendDtype out_dtype, LuxQuantKernel kernel,
                         LuxBackendBuffer* bias = nullptr, LuxBackendDtype bias_dtype = LUX_DTYPE_FLOAT32,
                         int act = LUX_QMM_ACT_NONE) {
    HipContext* ctx = C(c);
    if (!ctx || !x || !w_q || !scales || !biases || !out) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (act < LUX_QMM_ACT_NONE || act > LUX_QMM_ACT_GELU) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    LuxBackendError e = lux_hip_qmm_validate(M, K, N, group_size, bits, x_dtype, sb_dtype, out_dtype, kernel);
    if (e != LUX_BACKEND_OK) return e;
    if (bias && !dtype_ok(bias_dtype)) return LUX_BACKEND_ERROR_NOT_SUPPORTED;
    const size_t G = (size_t)(K / group_size);
    if (!fits(B(x), (size_t)M * K * dtype_size(x_dtype)) ||
        !fits(B(w_q), (size_t)N * K * bits / 8) || !fits(B(scales), (size_t)N * G * dtype_size(sb_dtype)) ||
        !fits(B(biases), (size_t)N * G * dtype_size(sb_dtype)) ||
        !fits(B(out), (size_t)M * N * dtype_size(out_dtype)) ||
        (bias && !fits(B(bias), (size_t)N * dtype_size(bias_dtype))))
        return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (M == 0 || N == 0) return LUX_BACKEND_OK;

    lxq::QmmArgs a;
    a.x = B(x)->ptr;
    a.wq = static_cast<const uint32_t*>(B(w_q)->ptr);
    a.scales = B(scales)->ptr;
    a.biases = B(biases)->ptr;
    a.y = B(out)->ptr;
    a.M = M; a.K = K; a.N = N; a.group_size = group_size; a.bits = bits;
    a.x_dtype = x_dtype; a.sb_dtype = sb_dtype; a.out_dtype = out_dtype;
    a.bias = bias ? B(bias)->ptr : nullptr;
    a.bias_dtype = bias_dtype;
    a.act = act;
    a.ws = ctx->ws;
    a.ws_bytes = ctx->ws_bytes;
    if (++ctx->epoch == 0u) ctx->epoch = 1u;
    a.epoch = ctx->epoch;

    if (hipSetDevice(ctx->device) != hipSuccess) return LUX_BACKEND_ERROR_DEVICE_LOST;
    return lux_hip_qmm_dispatch(a, kernel, ctx->stream);
}

LuxBackendError hip_op_quantized_matmul(LuxBackendContext* c, LuxBackendBuffer* x,
                                        LuxBackendBuffer* w_q, LuxBackendBuffer* scales,
                                        LuxBackendBuffer* biases, LuxBackendBuffer* out, int M,
                                        int K, int N, int group_size, int bits,
                                        LuxBackendDtype x_dtype, LuxBackendDtype sb_dtype,
                                        LuxBackendDtype out_dtype) {
    return qmm_impl(c, x, w_q, scales, biases, out, M, K, N, group_size, bits, x_dtype, sb_dtype,
                    out_dtype, LUX_QMM_KERNEL_AUTO);
}

LuxBackendError hip_op_quantized_matmul_ex(LuxBackendContext* c, LuxBackendBuffer* x,
                                           LuxBackendBuffer* w_q, LuxBackendBuffer* scales,
                                           LuxBackendBuffer* biases, LuxBackendBuffer* out,
                                           int M, int K, int N, int group_size, int bits,
                                           LuxBackendDtype x_dtype, LuxBackendDtype sb_dtype,
                                           LuxBackendDtype out_dtype, LuxQuantKernel kernel) {
    return qmm_impl(c, x, w_q, scales, biases, out, M, K, N, group_size, bits, x_dtype, sb_dtype,
                    out_dtype, kernel);
}

LuxBackendError hip_op_quantized_matmul_fused(LuxBackendContext* c, LuxBackendBuffer* x,
                                              LuxBackendBuffer* w_q, LuxBackendBuffer* scales,
                                              LuxBackendBuffer* biases, LuxBackendBuffer* bias,
                                              LuxBackendBuffer* out, int M, int K, int N,
                                              int group_size, int bits, LuxBackendDtype x_dtype,
                                              LuxBackendDtype sb_dtype, LuxBackendDtype bias_dtype,
                                              LuxBackendDtype out_dtype, LuxQuantAct act) {
    return qmm_impl(c, x, w_q, scales, biases, out, M, K, N, group_size, bits, x_dtype, sb_dtype,
                    out_dtype, LUX_QMM_KERNEL_AUTO, bias, bias_dtype, (int)act);
}

LuxBackendError hip_op_dequantize(LuxBackendContext* c, LuxBackendBuffer* w_q,
                                  LuxBackendBuffer* scales, LuxBackendBuffer* biases,
                                  LuxBackendBuffer* out, int N, int K, int group_size, int bits,
                                  LuxBackendDtype sb_dtype, LuxBackendDtype out_dtype) {
    HipContext* ctx = C(c);
    if (!ctx || !w_q || !scales || !biases || !out) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    LuxBackendError e = check_format(K, N, group_size, bits);
    if (e != LUX_BACKEND_OK) return e;
    if (!dtype_ok(sb_dtype) || !dtype_ok(out_dtype)) return LUX_BACKEND_ERROR_NOT_SUPPORTED;
    const size_t G = (size_t)(K / group_size);
    if (!fits(B(w_q), (size_t)N * K * bits / 8) || !fits(B(scales), (size_t)N * G * dtype_size(sb_dtype)) ||
        !fits(B(biases), (size_t)N * G * dtype_size(sb_dtype)) ||
        !fits(B(out), (size_t)N * K * dtype_size(out_dtype)))
        return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (N == 0) return LUX_BACKEND_OK;
    if (hipSetDevice(ctx->device) != hipSuccess) return LUX_BACKEND_ERROR_DEVICE_LOST;
    return map_status(lxq::launch_dequantize(static_cast<const uint32_t*>(B(w_q)->ptr), B(scales)->ptr,
                                             B(biases)->ptr, B(out)->ptr, N, K, group_size, bits,
                                             sb_dtype, out_dtype, ctx->stream));
}

LuxBackendError hip_op_quantize(LuxBackendContext* c, LuxBackendBuffer* w, LuxBackendBuffer* w_q,
                                LuxBackendBuffer* scales, LuxBackendBuffer* biases, int N, int K,
                                int group_size, int bits, LuxBackendDtype w_dtype,
                                LuxBackendDtype sb_dtype) {
    HipContext* ctx = C(c);
    if (!ctx || !w || !w_q || !scales || !biases) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    LuxBackendError e = check_format(K, N, group_size, bits);
    if (e != LUX_BACKEND_OK) return e;
    if (!dtype_ok(w_dtype) || !dtype_ok(sb_dtype)) return LUX_BACKEND_ERROR_NOT_SUPPORTED;
    const size_t G = (size_t)(K / group_size);
    if (!fits(B(w), (size_t)N * K * dtype_size(w_dtype)) || !fits(B(w_q), (size_t)N * K * bits / 8) ||
        !fits(B(scales), (size_t)N * G * dtype_size(sb_dtype)) ||
        !fits(B(biases), (size_t)N * G * dtype_size(sb_dtype)))
        return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (N == 0) return LUX_BACKEND_OK;
    if (hipSetDevice(ctx->device) != hipSuccess) return LUX_BACKEND_ERROR_DEVICE_LOST;
    return map_status(lxq::launch_quantize(B(w)->ptr, static_cast<uint32_t*>(B(w_q)->ptr),
                                           B(scales)->ptr, B(biases)->ptr, N, K, group_size, bits,
                                           w_dtype, sb_dtype, ctx->stream));
}

// ---------------------------------------------------------------------------
// base tensor ops (f32): the slots the reference CPU backend fills
// (src/cpu_backend.cpp:360-364), plus div and transpose.  Unlike the CPU
// backend, the element counts are checked against the buffer sizes: a GPU
// kernel must not read or write past an allocation.
// ---------------------------------------------------------------------------

bool fits(LuxBackendBuffer* b, size_t floats) { return B(b) && floats <= B(b)->size / 4; }

LuxBackendError elementwise(int op, LuxBackendContext* c, LuxBackendBuffer* a, LuxBackendBuffer* b,
                            LuxBackendBuffer* out, size_t n) {
    HipContext* ctx = C(c);
    if (!ctx || !fits(a, n) || !fits(b, n) || !fits(out, n)) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (hipSetDevice(ctx->device) != hipSuccess) return LUX_BACKEND_ERROR_DEVICE_LOST;
    return map_status(lxq::launch_elementwise(op, static_cast<const float*>(B(a)->ptr),
                                              static_cast<const float*>(B(b)->ptr), static_cast<float*>(B(out)->ptr),
                                              n, ctx->stream));
}
LuxBackendError hip_op_add_f32(LuxBackendContext* c, LuxBackendBuffer* a, LuxBackendBuffer* b, LuxBackendBuffer* o,
                               size_t n) {
    return elementwise(0, c, a, b, o, n);
}
LuxBackendError hip_op_sub_f32(LuxBackendContext* c, LuxBackendBuffer* a, LuxBackendBuffer* b, LuxBackendBuffer* o,
                               size_t n) {
    return elementwise(1, c, a, b, o, n);
}
LuxBackendError hip_op_mul_f32(LuxBackendContext* c, LuxBackendBuffer* a, LuxBackendBuffer* b, LuxBackendBuffer* o,
                               size_t n) {
    return elementwise(2, c, a, b, o, n);
}
LuxBackendError hip_op_div_f32(LuxBackendContext* c, LuxBackendBuffer* a, LuxBackendBuffer* b, LuxBackendBuffer* o,
                               size_t n) {
    return elementwise(3, c, a, b, o, n);
}

LuxBackendError hip_op_matmul_f32(LuxBackendContext* c, LuxBackendBuffer* a, LuxBackendBuffer* b,
                                  LuxBackendBuffer* out, int M, int K, int N) {
    HipContext* ctx = C(c);
    if (!ctx || M < 0 || K < 0 || N < 0) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (!fits(a, (size_t)M * K) || !fits(b, (size_t)K * N) || !fits(out, (size_t)M * N))
        return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (hipSetDevice(ctx->device) != hipSuccess) return LUX_BACKEND_ERROR_DEVICE_LOST;
    return map_status(lxq::launch_matmul_f32(static_cast<const float*>(B(a)->ptr), static_cast<const float*>(B(b)->ptr),
                                             static_cast<float*>(B(out)->ptr), M, K, N, ctx->stream));
}

LuxBackendError hip_op_transpose_f32(LuxBackendContext* c, LuxBackendBuffer* in, LuxBackendBuffer* out, int rows,
                                     int cols) {
    HipContext* ctx = C(c);
    if (!ctx || rows < 0 || cols < 0) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (!fits(in, (size_t)rows * cols) || !fits(out, (size_t)rows * cols)) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (hipSetDevice(ctx->device) != hipSuccess) return LUX_BACKEND_ERROR_DEVICE_LOST;
    return map_status(lxq::launch_transpose_f32(static_cast<const float*>(B(in)->ptr), static_cast<float*>(B(out)->ptr),
                                                rows, cols, ctx->stream));
}

void* hip_get_native_stream(LuxBackendContext* c) {
    HipContext* ctx = C(c);
    return ctx ? reinterpret_cast<void*>(ctx->stream) : nullptr;
}

LuxQuantKernel hip_select_kernel(int M, int K, int N, int group_size, int bits,
                                 LuxBackendDtype x_dtype, LuxBackendDtype sb_dtype) {
    return select_kernel_impl(M, K, N, group_size, bits, x_dtype, sb_dtype);
}

// ---- quantized linear layers from safetensors files ----------------------

LuxBackendError hip_linear_describe(const char* path, const char* prefix, int group_size, int bits,
                                    lux_quant_linear_info* out) {
    return lxq::linear_describe(path, prefix, group_size, bits, out);
}

void hip_linear_free(LuxBackendContext* c, lux_quant_linear* l) {
    if (!l) return;
    for (LuxBackendBuffer* b : {l->w_q, l->scales, l->biases, l->bias})
        if (b) hip_buffer_free(c, b);
    std::memset(l, 0, sizeof(*l));
}

LuxBackendError hip_linear_load(LuxBackendContext* c, const char* path, const char* prefix, int group_size,
                                int bits, lux_quant_linear* out) {
    if (!out) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    std::memset(out, 0, sizeof(*out));
    if (!C(c)) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    lux_quant_linear_info info;
    LuxBackendError e = lxq::linear_describe(path, prefix, group_size, bits, &info);
    if (e != LUX_BACKEND_OK) return e;
    lxq::MappedFile f;
    if (!f.open(path)) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    // the file may have changed since it was described: re-check the ranges
    const uint64_t ranges[4][2] = {{info.weight_offset, info.weight_bytes}, {info.scales_offset, info.scales_bytes},
                                   {info.biases_offset, info.biases_bytes}, {info.bias_offset, info.bias_bytes}};
    for (const auto& r : ranges)
        if (r[0] > f.size || r[1] > f.size - r[0]) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    LuxBackendBuffer** dst[4] = {&out->w_q, &out->scales, &out->biases, &out->bias};
    for (int i = 0; i < 4; i++) {
        if (i == 3 && !info.has_bias) break;
        *dst[i] = hip_buffer_alloc_with_data(c, f.data + ranges[i][0], ranges[i][1]);
        if (!*dst[i]) {
            hip_linear_free(c, out);
            return LUX_BACKEND_ERROR_OUT_OF_MEMORY;
        }
    }
    out->info = info;
    return LUX_BACKEND_OK;
}

// ---------------------------------------------------------------------------
// tables
// ---------------------------------------------------------------------------

lux_gpu_backend_vtbl make_vtbl() {
    lux_gpu_backend_vtbl v;
    std::memset(&v, 0, sizeof(v));  // every slot not set below is NOT_SUPPORTED
    v.create_context = hip_create_context;
    v.destroy_context = hip_destroy_context;
    v.get_device_count = hip_get_device_count;
    v.get_device_info = hip_get_device_info;
    v.sync = hip_sync;
    v.buffer_alloc = hip_buffer_alloc;
    v.buffer_alloc_with_data = hip_buffer_alloc_with_data;
    v.buffer_free = hip_buffer_free;
    v.buffer_copy_to_host = hip_buffer_copy_to_host;
    v.buffer_copy_from_host = hip_buffer_copy_from_host;
    v.buffer_get_host_ptr = hip_buffer_get_host_ptr;
    v.op_add_f32 = hip_op_add_f32;
    v.op_sub_f32 = hip_op_sub_f32;
    v.op_mul_f32 = hip_op_mul_f32;
    v.op_div_f32 = hip_op_div_f32;
    v.op_matmul_f32 = hip_op_matmul_f32;
    v.op_transpose_f32 = hip_op_transpose_f32;
    return v;
}

const lux_gpu_backend_vtbl g_vtbl = make_vtbl();

lux_gpu_quant_vtbl make_qvtbl() {
    lux_gpu_quant_vtbl q;
    std::memset(&q, 0, sizeof(q));
    q.ext_version = LUX_GPU_QUANT_EXT_VERSION;
    q.struct_size = sizeof(lux_gpu_quant_vtbl);
    q.op_quantized_matmul = hip_op_quantized_matmul;
    q.op_dequantize = hip_op_dequantize;
    q.op_quantize = hip_op_quantize;
    q.op_quantized_matmul_ex = hip_op_quantized_matmul_ex;
    q.get_native_stream = hip_get_native_stream;
    q.select_kernel = hip_select_kernel;
    q.op_quantized_matmul_fused = hip_op_quantized_matmul_fused;
    q.linear_describe = hip_linear_describe;
    q.linear_load = hip_linear_load;
    q.linear_free = hip_linear_free;
    return q;
}

const lux_gpu_quant_vtbl g_qvtbl = make_qvtbl();

}  // namespace

extern "C" __attribute__((visibility("default"))) bool lux_gpu_backend_init(lux_gpu_backend_desc* out) {
    if (!out) return false;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return false;
    bool any = false;
    for (int d = 0; d < n && !any; d++) any = is_gfx950(d);
    if (!any) return false;
    out->abi_version = LUX_GPU_BACKEND_ABI_VERSION;
    out->backend_name = "hip";
    out->backend_version = "0.1.0";
    // f32 elementwise ops and matmul are filled (never UNIFIED_MEMORY: a
    // discrete GPU); the quantized ops come through the extension table
    out->capabilities = LUX_CAP_TENSOR_OPS | LUX_CAP_MATMUL;
    out->vtbl = &g_vtbl;
    return true;
}

extern "C" __attribute__((visibility("default"))) bool lux_gpu_backend_quant_init(const lux_gpu_quant_vtbl** out) {
    if (!out) return false;
    *out = &g_qvtbl;
    return true;
}

// a dry run of the dispatch: every launcher records its kernel's name
// instead of launching (QmmArgs::plan), so no device call is made and the
// operand pointers, stand-ins here, are never read
extern "C" __attribute__((visibility("default"))) const char* lux_gpu_quantized_matmul_kernel_name(
    int M, int K, int N, int group_size, int bits, LuxBackendDtype x_dtype, LuxBackendDtype sb_dtype,
    LuxBackendDtype out_dtype, LuxQuantKernel kernel) {
    if (lux_hip_qmm_validate(M, K, N, group_size, bits, x_dtype, sb_dtype, out_dtype, kernel) != LUX_BACKEND_OK)
        return nullptr;
    if (M == 0 || N == 0) return "";
    // never read or written; aligned like a device allocation, so that a
    // launcher that chose by alignment would choose as for real buffers
    alignas(256) static uint8_t stand_in[256];
    const char* name = nullptr;
    lxq::QmmArgs a;
    a.x = a.scales = a.biases = stand_in;
    a.wq = nullptr;
    a.y = stand_in;
    a.M = M; a.K = K; a.N = N; a.group_size = group_size; a.bits = bits;
    a.x_dtype = x_dtype; a.sb_dtype = sb_dtype; a.out_dtype = out_dtype;
    // a context's workspace
    a.ws = stand_in;
    a.ws_bytes = lxq::kSplitWorkspaceBytes;
    a.epoch = 1u;
    a.plan = &name;
    if (lux_hip_qmm_dispatch(a, kernel, nullptr) != LUX_BACKEND_OK) return nullptr;
    return name;
}
