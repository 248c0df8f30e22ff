// qdispatch.h -- the quantized matmul's argument checks and kernel dispatch,
// shared by the context ops (hip_backend.hip) and any entry point that runs
// the op on caller pointers and streams.
#pragma once
#include "../../include/lux_gpu_quant_backend.h"
#include "kernels.h"

// the device is an MI355X-class gfx950 GPU (the only target of the kernels)
bool lux_hip_is_gfx950(int dev);

// format, dtype and kernel-choice checks of a quantized matmul (no buffers):
// OK, INVALID_ARGUMENT or NOT_SUPPORTED as the ops document
LuxBackendError lux_hip_qmm_validate(int M, int K, int N, int group_size, int bits, int x_dtype, int sb_dtype,
                                     int out_dtype, int kernel);

// kernel selection (AUTO, GEMV, GEMM) and launch of a validated quantized
// matmul on `st`, with the current device the stream's
LuxBackendError lux_hip_qmm_dispatch(const lxq::QmmArgs& a, int kernel, hipStream_t st);
