/*
 * lux_quant_core.h -- the core-side half of the quantized path: backend
 * selection and the public quantized-matmul op, as a small C library
 * (libluxgpu_quant_core.so) that a core links next to its plugin loader.
 *
 * Selection follows the reference loader (reference src/plugin_loader.hpp):
 * search paths /usr/lib/lux-gpu, /usr/local/lib/lux-gpu, then the directory
 * of this library, with each ':'-separated LUX_GPU_BACKEND_PATH entry
 * inserted in front (:112-146); a backend <name> is
 * libluxgpu_backend_<name>.so in the first path that has it (:165-182),
 * dlopen'ed RTLD_NOW | RTLD_LOCAL, its lux_gpu_backend_init called and the
 * ABI version checked (:184-232).  Added: LUX_BACKEND=<name> picks a
 * backend explicitly (documented by the reference, README.md:65, not
 * implemented there), "hip" joins the probe list and the priority order
 * metal, cuda, hip, webgpu (:154-156, :250-262), and the additive
 * quantized-matmul table (lux_gpu_quant_backend.h) is looked up after a
 * successful init.
 *
 * Tensors are 2-D device buffers with a dtype; packed weights use
 * LUX_QTENSOR_U32.  lux_tensor_quantized_matmul is the op the reference core
 * would add beside lux_tensor_matmul (reference src/gpu_core.cpp:450-474):
 * shape checks, a zero-filled output, one call through the plugin table.
 * No counterpart of these types exists in the reference's public header, so
 * they are this library's own (lux_qcore, lux_qtensor).
 */
#ifndef LUX_QUANT_CORE_H
#define LUX_QUANT_CORE_H

#include <stddef.h>
#include <stdint.h>

#include "lux_gpu_quant_backend.h"

#ifdef __cplusplus
extern "C" {
#endif

#define LUX_QTENSOR_U32 100 /* packed codes: uint32 words, no float dtype */

typedef struct lux_qcore lux_qcore;
typedef struct lux_qtensor lux_qtensor;

/* Load a backend and create a context on `device`.  name: a backend name,
 * or NULL / "auto": LUX_BACKEND if set (and not "auto"), else the first
 * available backend in priority order.  Returns NULL when the backend does
 * not load or is unavailable (e.g. no device), has no quantized-matmul
 * table, LUX_BACKEND is "cpu" (the core's own CPU backend), or the context
 * fails; *err (may be NULL) then points to a message in static storage. */
__attribute__((visibility("default"))) lux_qcore* lux_qcore_open(const char* name, int device, const char** err);
__attribute__((visibility("default"))) void lux_qcore_close(lux_qcore* core);
__attribute__((visibility("default"))) const char* lux_qcore_backend_name(const lux_qcore* core);
__attribute__((visibility("default"))) const lux_gpu_backend_vtbl* lux_qcore_vtbl(const lux_qcore* core);
__attribute__((visibility("default"))) const lux_gpu_quant_vtbl* lux_qcore_quant(const lux_qcore* core);
__attribute__((visibility("default"))) LuxBackendContext* lux_qcore_context(const lux_qcore* core);

/* A [rows, cols] tensor of `dtype` (LuxBackendDtype or LUX_QTENSOR_U32) on
 * the core's device, filled from `data` (NULL: zero-filled).  NULL on a bad
 * shape or dtype, or when the allocation fails. */
__attribute__((visibility("default"))) lux_qtensor* lux_qtensor_create(lux_qcore* core, const void* data, int64_t rows,
                                                                       int64_t cols, int dtype);
/* copies min(bytes, tensor bytes) to `dst` after the queued work */
__attribute__((visibility("default"))) LuxBackendError lux_qtensor_to_host(lux_qcore* core, const lux_qtensor* t,
                                                                           void* dst, size_t bytes);
__attribute__((visibility("default"))) void lux_qtensor_free(lux_qcore* core, lux_qtensor* t);
/* dimension i (0: rows, 1: cols) and dtype; -1 for a NULL tensor */
__attribute__((visibility("default"))) int64_t lux_qtensor_dim(const lux_qtensor* t, int i);
__attribute__((visibility("default"))) int lux_qtensor_dtype(const lux_qtensor* t);

/* y[M, N] = x[M, K] . dequant(w_q, scales, biases)^T, y in x's dtype.
 * Requires x [M, K] (f32/f16/bf16), w_q [N, K*bits/32] LUX_QTENSOR_U32,
 * scales and biases [N, K/group_size] of one float dtype.  Returns a new
 * tensor, or NULL on a shape or dtype mismatch or a backend error (the
 * backend's code in *err_code when err_code is not NULL). */
__attribute__((visibility("default"))) lux_qtensor* lux_tensor_quantized_matmul(lux_qcore* core, const lux_qtensor* x,
                                                                                const lux_qtensor* w_q,
                                                                                const lux_qtensor* scales,
                                                                                const lux_qtensor* biases,
                                                                                int group_size, int bits,
                                                                                LuxBackendError* err_code);

#ifdef __cplusplus
}
#endif

#endif /* LUX_QUANT_CORE_H */
