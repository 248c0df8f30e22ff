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
    LUX_QMM_KERNEL_GEMV = 1, /* bandwidth-bound dequant-GEMV (any M, built for M <= 16) */
    LUX_QMM_KERNEL_GEMM = 2, /* MFMA GEMM (16-bit activations only) */
} LuxQuantKernel;

/* fused output stage of op_quantized_matmul_fused, applied in fp32 */
typedef enum {
    LUX_QMM_ACT_NONE = 0,
    LUX_QMM_ACT_RELU = 1, /* v < 0 ? 0 : v (NaN passes through) */
    LUX_QMM_ACT_SILU = 2, /* v / (1 + exp(-v)) */
    LUX_QMM_ACT_GELU = 3, /* v/2 (1 + erf(v / sqrt(2))) */
} LuxQuantAct;

/*
 * Quantized linear layers on disk (safetensors).  The file is a 64-bit
 * little-endian header length H, H bytes of JSON, then the data; each JSON
 * entry maps a tensor name to {"dtype", "shape", "data_offsets": [begin,
 * end]} relative to the data.  A layer with name prefix P holds
 *   P.weight  U32 [N, K*bits/32]      packed codes (the format above)
 *   P.scales  F32|F16|BF16 [N, K/g]
 *   P.biases  same dtype and shape as P.scales
 *   P.bias    F32|F16|BF16 [N]        optional output bias (fused op)
 * bits and group_size come from the caller, else from the "__metadata__"
 * string entries "P.bits" / "P.group_size", else its "bits" / "group_size".
 * No counterpart in the reference (it has no weight files).
 */
typedef struct lux_quant_linear_info {
    int32_t N, K, group_size, bits;
    LuxBackendDtype sb_dtype;   /* scales and biases */
    LuxBackendDtype bias_dtype; /* P.bias, when has_bias */
    int32_t has_bias;
    int32_t _pad;
    uint64_t weight_offset, weight_bytes; /* absolute file offsets of the data */
    uint64_t scales_offset, scales_bytes;
    uint64_t biases_offset, biases_bytes;
    uint64_t bias_offset, bias_bytes;
} lux_quant_linear_info;

typedef struct lux_quant_linear {
    lux_quant_linear_info info;
    LuxBackendBuffer* w_q;
    LuxBackendBuffer* scales;
    LuxBackendBuffer* biases;
    LuxBackendBuffer* bias; /* NULL without P.bias */
} lux_quant_linear;

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

    /* out[m,n] = act(sum_k x[m,k] w_hat[n,k] + bias[n]): the bias (T_bias[N],
     * or NULL for none) and the activation are applied in fp32 to the
     * accumulator, before the one rounding to T_out, by the kernel that
     * computes out (no second pass over out).  Same kernels, selection and
     * errors as op_quantized_matmul; an unknown act is INVALID_ARGUMENT.
     * No counterpart in the reference (it has no quantized or fused op);
     * NULL in plugins that predate it. */
    LuxBackendError (*op_quantized_matmul_fused)(LuxBackendContext* ctx, LuxBackendBuffer* x,
                                                 LuxBackendBuffer* w_q, LuxBackendBuffer* scales,
                                                 LuxBackendBuffer* biases, LuxBackendBuffer* bias,
                                                 LuxBackendBuffer* out, int M, int K, int N,
                                                 int group_size, int bits, LuxBackendDtype x_dtype,
                                                 LuxBackendDtype sb_dtype, LuxBackendDtype bias_dtype,
                                                 LuxBackendDtype out_dtype, LuxQuantAct act);

    /* Parse the safetensors header of `path` and describe layer `prefix`
     * (host only, no device work).  group_size / bits 0 = from the file.
     * Unreadable or malformed file, missing tensor, shapes that disagree:
     * INVALID_ARGUMENT; bits, group size or dtype outside the format:
     * NOT_SUPPORTED. */
    LuxBackendError (*linear_describe)(const char* path, const char* prefix, int group_size,
                                       int bits, lux_quant_linear_info* out);

    /* linear_describe, then one device buffer per tensor on ctx, filled from
     * the memory-mapped file (synchronous: the data is on the device when it
     * returns).  On error nothing stays allocated and *out is zeroed. */
    LuxBackendError (*linear_load)(LuxBackendContext* ctx, const char* path, const char* prefix,
                                   int group_size, int bits, lux_quant_linear* out);

    /* frees the buffers linear_load allocated and zeroes *layer */
    void (*linear_free)(LuxBackendContext* ctx, lux_quant_linear* layer);

    void* _reserved[4];
} lux_gpu_quant_vtbl;

/* layout pins: LP64 */
#if defined(__LP64__)
#ifdef __cplusplus
static_assert(sizeof(lux_gpu_quant_vtbl) == 120, "quant table size");
static_assert(offsetof(lux_gpu_quant_vtbl, op_quantized_matmul_fused) == 56, "fused op slot");
static_assert(offsetof(lux_gpu_quant_vtbl, linear_free) == 80, "weight file slots");
static_assert(sizeof(lux_quant_linear_info) == 96, "linear info size");
#else
_Static_assert(sizeof(lux_gpu_quant_vtbl) == 120, "quant table size");
_Static_assert(offsetof(lux_gpu_quant_vtbl, op_quantized_matmul_fused) == 56, "fused op slot");
_Static_assert(offsetof(lux_gpu_quant_vtbl, linear_free) == 80, "weight file slots");
_Static_assert(sizeof(lux_quant_linear_info) == 96, "linear info size");
#endif
#endif

typedef bool (*lux_gpu_backend_quant_init_fn)(const lux_gpu_quant_vtbl** out);

/*
 * Exported by libluxgpu_backend_hip.so.  No counterpart in the reference:
 * it is the additive entry a loader dlsym()s after lux_gpu_backend_init
 * succeeded (the step after reference src/plugin_loader.hpp:209) to reach
 * the quantized ops that the reference vtable has no slot for.  Sets *out to
 * a static table and returns true.
 */
__attribute__((visibility("default"))) bool lux_gpu_backend_quant_init(const lux_gpu_quant_vtbl** out);

/*
 * op_quantized_matmul_ex without a context and without allocation: no
 * counterpart in the reference.  It is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops that forbid
 * hipMalloc).  x, w_q, scales, biases and out are device pointers of the
 * current device holding at least the bytes the shape needs (not checked:
 * there are no buffer sizes here), and each of x, w_q, scales and biases
 * must be followed by at least 256 readable bytes of device memory (not
 * used for the result: the kernels copy operand arrays in whole 16-byte
 * chunks and may read up to 255 bytes past an array's end; the plugin's own
 * buffers carry that slack, so an operand carved from the end of a larger
 * allocation needs 256 bytes left after it).  `stream` is a hipStream_t of
 * that device (NULL: the null stream).  Same kernels, selection, results and shape and
 * dtype errors as op_quantized_matmul_ex.  The partial sums, tile counters
 * and flags of the split-K small-M GEMM and of the large GEMM's split last
 * round live in a 16 MiB (+ 4 KiB) static device array that
 * each GPU holds until the process ends (shapes whose split would need more
 * are INVALID_ARGUMENT; the split rule keeps every shape within it).  All
 * calls on one GPU share that array: calls that overlap in time on one GPU
 * (concurrent streams, or threads) race and give wrong results.  The first
 * call on a device clears the array with a kernel on its stream, so that
 * call must not be made under stream capture: it returns NOT_SUPPORTED
 * there (make one eager call on the device first; later calls may be
 * captured and replayed).
 */
__attribute__((visibility("default"))) LuxBackendError lux_gpu_quantized_matmul_noalloc(
    const void* x, const void* w_q, const void* scales, const void* biases, void* out, int M, int K, int N,
    int group_size, int bits, LuxBackendDtype x_dtype, LuxBackendDtype sb_dtype, LuxBackendDtype out_dtype,
    LuxQuantKernel kernel, void* stream);

/*
 * The name of the gfx950 kernel that op_quantized_matmul_ex (with a
 * context) would launch for this shape and kernel choice: for example
 * "qgemv_line_kernel" or "qgemm_rw_kernel", the kernel names profilers
 * show.  NULL where the op would return an error for these arguments; ""
 * where it launches nothing (M or N zero).  The string is static.  No
 * counterpart in the reference: a host-only query for tests and tuning
 * tools that makes no device call, so it answers on a machine without a GPU.
 */
__attribute__((visibility("default"))) const char* lux_gpu_quantized_matmul_kernel_name(
    int M, int K, int N, int group_size, int bits, LuxBackendDtype x_dtype, LuxBackendDtype sb_dtype,
    LuxBackendDtype out_dtype, LuxQuantKernel kernel);

#ifdef __cplusplus
}
#endif

#endif /* LUX_GPU_QUANT_BACKEND_H */
