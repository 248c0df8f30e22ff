/*
 * lux_cpu_quant.h -- CPU restatement of group-wise affine quantized matmul.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the correctness oracle and the
 * timed CPU baseline for the HIP plugin.  Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load it; the plugin never does.
 *
 * The reference (Lux GPU Core v0.2.0) has no quantized matmul, so the format
 * below is this project's specification.  It follows the conventions of the
 * reference's CPU kernel library:
 *   - C ABI, `lux_cpu_` prefix, output argument first
 *     (reference kernels/cpu/tensor_ops.h:24-83),
 *   - fp32 accumulation in ascending k, `sum += a * b`
 *     (reference src/cpu_backend.cpp:256-264),
 *   - dtype codes of LuxBackendDtype
 *     (reference include/lux/gpu/backend_plugin.h:38-47).
 *
 * Format
 *   W is [N, K] (row n = output feature).  Each row holds K codes of `bits`
 *   bits.  Code k of a row occupies bits [k*bits, k*bits + bits) of the row's
 *   little-endian bitstream of uint32 words; a code may straddle two words
 *   (bits 3, 5, 6).  w_q is uint32[N, K*bits/32].
 *   scales, biases are T_sb[N, K/group_size] (T_sb in {f32, f16, bf16}).
 *   Dequantized weight: w_hat = fmaf(float(scale), float(q), float(bias)).
 *   Quantized matmul:   y[m, n] = sum_k x[m, k] * w_hat[n, k]   (y = x W^T).
 *
 * Quantizer (per group of group_size consecutive k of one row)
 *   mn = min, mx = max (fp32);  scale = (mx - mn) / (2^bits - 1)  (fp32);
 *   bias = mn;  both stored as T_sb with round-to-nearest-even;
 *   q = clamp(nearbyintf((w - bias_s) / scale_s), 0, 2^bits - 1) using the
 *   STORED values widened to fp32;  scale_s == 0  =>  q = 0.
 */
#ifndef LUX_CPU_QUANT_H
#define LUX_CPU_QUANT_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes, identical to LuxBackendDtype */
enum { LUX_CPU_F32 = 0, LUX_CPU_F16 = 1, LUX_CPU_BF16 = 2 };

/* return codes, identical to LuxBackendError */
enum { LUX_CPU_OK = 0, LUX_CPU_EINVAL = 1, LUX_CPU_ENOTSUP = 3 };

/* ---- scalar conversions (round to nearest even) ------------------------ */
uint16_t lux_cpu_f32_to_f16(float f);
float    lux_cpu_f16_to_f32(uint16_t h);
uint16_t lux_cpu_f32_to_bf16(float f);
float    lux_cpu_bf16_to_f32(uint16_t h);
void lux_cpu_convert(void* out, int out_dtype, const void* in, int in_dtype, size_t n);

/* ---- seeded portable PRNG: SplitMix64-seeded xoshiro256**, Box-Muller ---- */
void lux_cpu_rng_normal_f32(float* out, size_t n, uint64_t seed, float mean, float stddev);
void lux_cpu_rng_u32(uint32_t* out, size_t n, uint64_t seed);

/* ---- bitstream pack / unpack (codes are uint8, bits in 1..8) ------------ */
int lux_cpu_pack_bits(uint32_t* w_q, const uint8_t* codes, int N, int K, int bits);
int lux_cpu_unpack_bits(uint8_t* codes, const uint32_t* w_q, int N, int K, int bits);

/* ---- quantize / dequantize --------------------------------------------- */
int lux_cpu_quantize(uint32_t* w_q, void* scales, void* biases, const float* w,
                     int N, int K, int group_size, int bits, int sb_dtype);
int lux_cpu_dequantize(void* out, const uint32_t* w_q, const void* scales,
                       const void* biases, int N, int K, int group_size,
                       int bits, int sb_dtype, int out_dtype);

/* ---- quantized matmul ---------------------------------------------------
 * lux_cpu_quantized_matmul: the oracle.  Scalar, fp32 accumulate in
 *   ascending k without fused multiply-add, output rounded RNE to out_dtype.
 * lux_cpu_quantized_matmul_f64: diagnostic, fp64 accumulation, fp64 output.
 * lux_cpu_quantized_matmul_omp: the timed CPU baseline.  OpenMP over rows of
 *   W, factored per group:  sum_g s_g * sum_k x_k q_k + b_g * sum_k x_k.
 *   Same result within fp32 rounding, not bit-identical.                    */
int lux_cpu_quantized_matmul(void* y, const void* x, const uint32_t* w_q,
                             const void* scales, const void* biases,
                             int M, int K, int N, int group_size, int bits,
                             int x_dtype, int sb_dtype, int out_dtype);
int lux_cpu_quantized_matmul_f64(double* y, const void* x, const uint32_t* w_q,
                                 const void* scales, const void* biases,
                                 int M, int K, int N, int group_size, int bits,
                                 int x_dtype, int sb_dtype);
int lux_cpu_quantized_matmul_omp(void* y, const void* x, const uint32_t* w_q,
                                 const void* scales, const void* biases,
                                 int M, int K, int N, int group_size, int bits,
                                 int x_dtype, int sb_dtype, int out_dtype,
                                 int num_threads);

/* lux_cpu_quantized_matmul_wround: the same scalar oracle with the
 *   dequantized weight rounded (RNE) to w_dtype before the multiply:
 *   y = sum_k x_k * T(fmaf(s, q, b)).  w_dtype F32 is the exact form above;
 *   F16/BF16 is the "dequantize to the activation type, then matmul"
 *   semantics of a GEMM that stages dequantized tiles for 16-bit MFMA.    */
int lux_cpu_quantized_matmul_wround(void* y, const void* x, const uint32_t* w_q,
                                    const void* scales, const void* biases,
                                    int M, int K, int N, int group_size, int bits,
                                    int x_dtype, int sb_dtype, int out_dtype,
                                    int w_dtype);

int lux_cpu_quantized_matmul_wround_omp(void* y, const void* x, const uint32_t* w_q,
                                        const void* scales, const void* biases,
                                        int M, int K, int N, int group_size, int bits,
                                        int x_dtype, int sb_dtype, int out_dtype, int w_dtype,
                                        int num_threads);

/* argument validation shared by all entry points: returns LUX_CPU_OK,
 * LUX_CPU_EINVAL (bad shape) or LUX_CPU_ENOTSUP (unsupported bits/group/dtype) */
int lux_cpu_quant_check(int M, int K, int N, int group_size, int bits,
                        int x_dtype, int sb_dtype, int out_dtype);

#ifdef __cplusplus
}
#endif
#endif /* LUX_CPU_QUANT_H */
