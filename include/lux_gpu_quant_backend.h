/*
 * lux_gpu_quant_backend.h -- additive quantized-matmul extension of the Lux
 * GPU backend plugin ABI (version 2, lux_gpu_backend_abi.h).
 *
 * The reference's 64-slot vtable has no quantized entry
 * (reference include/lux/gpu/backend_plugin.h:82-382), and its header stays
 * unchanged, so the plugin exports a SECOND, optional symbol that a loader
 * looks up with dlsym next to lux_gpu_backend_init.  A core that does not
 * know the symbol never sees it.  The ops take the same context and device
 * buffer handles as the base vtable's op_matmul_f32
 * (reference backend_plugin.h:129).
 *
 * Format (all ops)
 *   w_q     uint32[N, K*bits/32]: row n holds K codes of `bits` bits; code k
 *           occupies bits [k*bits, k*bits+bits) of the row's little-endian
 *           bitstream and may straddle two words (bits 3, 5, 6).
 *   scales, biases  T_sb[N, K/group_size].
 *   dequantized weight  w_hat[n,k] = fmaf(scale[n,g], q[n,k], bias[n,g]),
 *           g = k / group_size, in fp32.
 *   x [M, K] (T_x), out [M, N] (T_out): out = x . w_hat^T, fp32 accumulate.
 *   bits in {2,3,4,5,6,8}; group_size in {32,64,128}; K % group_size == 0;
 *   T_x, T_sb, T_out in {FLOAT32, FLOAT16, BFLOAT16}.
 *
 * Errors: NULL handle or bad shape -> INVALID_ARGUMENT; unsupported bits,
 * group size or dtype -> NOT_SUPPORTED; a buffer smaller than the shape
 * needs -> INVALID_ARGUMENT; HIP launch failure -> INTERNAL.  All ops are
 * asynchronous on the context's stream; buffer_copy_to_host and sync order
 * after them.
 */
#ifndef LUX_GPU_QUANT_BACKEND_H
#define LUX_GPU_QUANT_BACKEND_H

#include "lux_gpu_backend_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

#define LUX_GPU_QUANT_EXT_VERSION 1
#define LUX_GPU_QUANT_INIT_SYMBOL "lux_gpu_backend_quant_init"

/* kernel selection for op_quantized_matmul_ex */
typedef enum {
    LUX_QMM_KERNEL_AUTO = 0, /* GEMV for M <= threshold, else GEMM */
    LUX_QMM_KERNEL_GEMV = 1, /* bandwidth-bound dequant-GEMV (any M, built for M <= 8) */
    LUX_QMM_KERNEL_GEMM = 2, /* MFMA GEMM (16-bit activations only) */
} LuxQuantKernel;

typedef struct lux_gpu_quant_vtbl {
    uint32_t ext_version; /* LUX_GPU_QUANT_EXT_VERSION */
    uint32_t struct_size; /* sizeof(lux_gpu_quant_vtbl) of the plugin */

    /* out[M,N] = x[M,K] . dequant(w_q, scales, biases)^T */
    LuxBackendError (*op_quantized_matmul)(LuxBackendContext* ctx, LuxBackendBuffer* x,
                                           LuxBackendBuffer* w_q, LuxBackendBuffer* scales,
                                           LuxBackendBuffer* biases, LuxBackendBuffer* out,
                                           int M, int K, int N, int group_size, int bits,
                                           LuxBackendDtype x_dtype, LuxBackendDtype sb_dtype,
                                           LuxBackendDtype out_dtype);

    /* out[N,K] = dequant(w_q, scales, biases) rounded to out_dtype; bit-exact
     * with the format's fmaf definition for out_dtype FLOAT32 */
    LuxBackendError (*op_dequantize)(LuxBackendContext* ctx, LuxBackendBuffer* w_q,
                                     LuxBackendBuffer* scales, LuxBackendBuffer* biases,
                                     LuxBackendBuffer* out, int N, int K, int group_size,
                                     int bits, LuxBackendDtype sb_dtype,
                                     LuxBackendDtype out_dtype);

    /* w[N,K] (T_w) -> (w_q, scales, biases): per group min/max affine
     * quantizer, scale = (max-min)/(2^bits-1), bias = min, stored RNE in
     * T_sb, q = clamp(rint((w - bias_s)/scale_s), 0, 2^bits-1) with the
     * stored values, q = 0 where scale_s == 0 */
    LuxBackendError (*op_quantize)(LuxBackendContext* ctx, LuxBackendBuffer* w,
                                   LuxBackendBuffer* w_q, LuxBackendBuffer* scales,
                                   LuxBackendBuffer* biases, int N, int K, int group_size,
                                   int bits, LuxBackendDtype w_dtype, LuxBackendDtype sb_dtype);

    /* op_quantized_matmul with an explicit kernel choice (tests, tuning) */
    LuxBackendError (*op_quantized_matmul_ex)(LuxBackendContext* ctx, LuxBackendBuffer* x,
                                              LuxBackendBuffer* w_q, LuxBackendBuffer* scales,
                                              LuxBackendBuffer* biases, LuxBackendBuffer* out,
                                              int M, int K, int N, int group_size, int bits,
                                              LuxBackendDtype x_dtype, LuxBackendDtype sb_dtype,
                                              LuxBackendDtype out_dtype, LuxQuantKernel kernel);

    /* the context's hipStream_t, for callers that time or order work on it */
    void* (*get_native_stream)(LuxBackendContext* ctx);

    /* which kernel AUTO picks for this shape and these dtypes (no launch) */
    LuxQuantKernel (*select_kernel)(int M, int K, int N, int group_size, int bits,
                                    LuxBackendDtype x_dtype, LuxBackendDtype sb_dtype);

    void* _reserved[8];
} lux_gpu_quant_vtbl;

typedef bool (*lux_gpu_backend_quant_init_fn)(const lux_gpu_quant_vtbl** out);

/*
 * Exported by libluxgpu_backend_hip.so.  No counterpart in the reference:
 * it is the additive entry a loader dlsym()s after lux_gpu_backend_init
 * succeeded (the step after reference src/plugin_loader.hpp:209) to reach
 * the quantized ops that the reference vtable has no slot for.  Sets *out to
 * a static table and returns true.
 */
__attribute__((visibility("default"))) bool lux_gpu_backend_quant_init(const lux_gpu_quant_vtbl** out);

#ifdef __cplusplus
}
#endif

#endif /* LUX_GPU_QUANT_BACKEND_H */
