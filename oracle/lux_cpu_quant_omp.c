/*
 * lux_cpu_quant_omp.c -- the timed CPU baseline for quantized matmul.
 * TEST INFRASTRUCTURE ONLY (see lux_cpu_quant.h).
 *
 * OpenMP over rows of W (the reference CPU backend parallelises its dense
 * matmul with OpenMP the same way, src/cpu_backend.cpp:253-255) and the
 * per-group factorisation
 *     y[m,n] = sum_g ( s[n,g] * sum_{k in g} x[m,k] q[n,k]
 *                    + b[n,g] * sum_{k in g} x[m,k] )
 * whose inner loops the compiler vectorises.  Built with -O3 -mavx2 -mfma,
 * so results agree with the scalar oracle to fp32 rounding, not bit for bit.
 */
#include "lux_cpu_quant.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float ld(const void* p, size_t i, int dt) {
    if (dt == LUX_CPU_F32) return ((const float*)p)[i];
    if (dt == LUX_CPU_F16) return lux_cpu_f16_to_f32(((const uint16_t*)p)[i]);
    return lux_cpu_bf16_to_f32(((const uint16_t*)p)[i]);
}

static inline void st(void* p, size_t i, int dt, float v) {
    if (dt == LUX_CPU_F32) ((float*)p)[i] = v;
    else if (dt == LUX_CPU_F16) ((uint16_t*)p)[i] = lux_cpu_f32_to_f16(v);
    else ((uint16_t*)p)[i] = lux_cpu_f32_to_bf16(v);
}

/* unpack one row of codes into floats */
static void unpack_row(float* q, const uint32_t* row, int K, int bits) {
    if (bits == 4) {
        for (int w = 0; w < K / 8; w++) {
            uint32_t v = row[w];
            for (int j = 0; j < 8; j++) q[8 * w + j] = (float)((v >> (4 * j)) & 15u);
        }
    } else if (bits == 8) {
        for (int w = 0; w < K / 4; w++) {
            uint32_t v = row[w];
            for (int j = 0; j < 4; j++) q[4 * w + j] = (float)((v >> (8 * j)) & 255u);
        }
    } else {
        const uint32_t mask = (1u << bits) - 1u;
        for (int k = 0; k < K; k++) {
            uint32_t bit = (uint32_t)k * (uint32_t)bits, wi = bit >> 5, sh = bit & 31u;
            uint64_t pair = row[wi];
            if (sh + (uint32_t)bits > 32u) pair |= (uint64_t)row[wi + 1] << 32;
            q[k] = (float)((uint32_t)(pair >> sh) & mask);
        }
    }
}

int lux_cpu_quantized_matmul_omp(void* y, const void* x, const uint32_t* w_q,
                                 const void* scales, const void* biases,
                                 int M, int K, int N, int group_size, int bits,
                                 int x_dtype, int sb_dtype, int out_dtype,
                                 int num_threads) {
    int rc = lux_cpu_quant_check(M, K, N, group_size, bits, x_dtype, sb_dtype, out_dtype);
    if (rc) return rc;
    if (M == 0 || N == 0) return LUX_CPU_OK;
    const int G = K / group_size, wpr = K * bits / 32;
    float* xf = (float*)malloc((size_t)M * K * sizeof(float));
    float* xs = (float*)malloc((size_t)M * G * sizeof(float));
    if (!xf || !xs) { free(xf); free(xs); return LUX_CPU_EINVAL; }
    for (size_t i = 0; i < (size_t)M * K; i++) xf[i] = ld(x, i, x_dtype);
    for (int m = 0; m < M; m++)
        for (int g = 0; g < G; g++) {
            float s = 0.f;
            for (int i = 0; i < group_size; i++) s += xf[(size_t)m * K + g * group_size + i];
            xs[(size_t)m * G + g] = s;
        }
#ifdef _OPENMP
    if (num_threads > 0) omp_set_num_threads(num_threads);
#pragma omp parallel
#endif
    {
        float* q = (float*)malloc((size_t)K * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int n = 0; n < N; n++) {
            unpack_row(q, w_q + (size_t)n * wpr, K, bits);
            for (int m = 0; m < M; m++) {
                const float* xr = xf + (size_t)m * K;
                float acc = 0.f;
                for (int g = 0; g < G; g++) {
                    const float* xg = xr + g * group_size;
                    const float* qg = q + g * group_size;
                    float d = 0.f;
#ifdef _OPENMP
#pragma omp simd reduction(+ : d)
#endif
                    for (int i = 0; i < group_size; i++) d += xg[i] * qg[i];
                    acc += ld(scales, (size_t)n * G + g, sb_dtype) * d
                         + ld(biases, (size_t)n * G + g, sb_dtype) * xs[(size_t)m * G + g];
                }
                st(y, (size_t)m * N + n, out_dtype, acc);
            }
        }
        free(q);
    }
    free(xf);
    free(xs);
    return LUX_CPU_OK;
}

/* OpenMP form of lux_cpu_quantized_matmul_wround (rows of W in parallel,
 * dequantized row rounded to w_dtype, fp32 accumulation): the checker for
 * large GEMM shapes.  Same values as the scalar form up to fp32 summation
 * order. */
int lux_cpu_quantized_matmul_wround_omp(void* y, const void* x, const uint32_t* w_q,
                                        const void* scales, const void* biases,
                                        int M, int K, int N, int group_size, int bits,
                                        int x_dtype, int sb_dtype, int out_dtype, int w_dtype,
                                        int num_threads) {
    int rc = lux_cpu_quant_check(M, K, N, group_size, bits, x_dtype, sb_dtype, out_dtype);
    if (rc) return rc;
    if (M == 0 || N == 0) return LUX_CPU_OK;
    const int G = K / group_size, wpr = K * bits / 32;
    float* xf = (float*)malloc((size_t)M * K * sizeof(float));
    if (!xf) return LUX_CPU_EINVAL;
    for (size_t i = 0; i < (size_t)M * K; i++) xf[i] = ld(x, i, x_dtype);
#ifdef _OPENMP
    if (num_threads > 0) omp_set_num_threads(num_threads);
#pragma omp parallel
#endif
    {
        float* q = (float*)malloc((size_t)K * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int n = 0; n < N; n++) {
            unpack_row(q, w_q + (size_t)n * wpr, K, bits);
            for (int k = 0; k < K; k++) {
                const int g = k / group_size;
                float v = fmaf(ld(scales, (size_t)n * G + g, sb_dtype), q[k],
                               ld(biases, (size_t)n * G + g, sb_dtype));
                if (w_dtype == LUX_CPU_F16) v = lux_cpu_f16_to_f32(lux_cpu_f32_to_f16(v));
                else if (w_dtype == LUX_CPU_BF16) v = lux_cpu_bf16_to_f32(lux_cpu_f32_to_bf16(v));
                q[k] = v;
            }
            for (int m = 0; m < M; m++) {
                const float* xr = xf + (size_t)m * K;
                float acc = 0.f;
#ifdef _OPENMP
#pragma omp simd reduction(+ : acc)
#endif
                for (int k = 0; k < K; k++) acc += xr[k] * q[k];
                st(y, (size_t)m * N + n, out_dtype, acc);
            }
        }
        free(q);
    }
    free(xf);
    return LUX_CPU_OK;
}
