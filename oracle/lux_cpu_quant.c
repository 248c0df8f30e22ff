/*
 * lux_cpu_quant.c -- CPU restatement (oracle) of group-wise affine quantized
 * matmul.  TEST INFRASTRUCTURE ONLY: see lux_cpu_quant.h for the format and
 * for who may load this library.
 *
 * Built with -ffp-contract=off and without -mfma so that `acc = acc + a * b`
 * is a separate fp32 multiply and add, exactly as the reference CPU backend's
 * dense matmul loop (reference src/cpu_backend.cpp:258-261) compiles on
 * x86-64.  Dequantization uses an explicit fmaf (correctly rounded in libm).
 */
#include "lux_cpu_quant.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* conversions                                                              */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t lux_cpu_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u)          /* NaN: keep it quiet */
        return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);              /* round half to even */
    return (uint16_t)(u >> 16);
}

float lux_cpu_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t lux_cpu_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u)                         /* inf / NaN */
        return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (a >= 0x47800000u)                         /* >= 65536: overflow */
        return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) {
        /* below the smallest normal half (2^-14): the result is a multiple
         * of 2^-24.  Adding 0.5 (= 2^23 * 2^-24) to |f| makes the fp32 adder
         * round |f| to a multiple of 2^-24 with ties to even; the low mantissa
         * bits of the sum are then the subnormal half's mantissa.           */
        float s = u2f(a) + 0.5f;
        return (uint16_t)(sign | (f2u(s) - 0x3f000000u));
    }
    /* normal half: rebias the exponent (127 -> 15) and round the 13 dropped
     * mantissa bits half to even; a carry into the exponent is correct,
     * including the carry to infinity for [65520, 65536).                   */
    uint32_t odd = (a >> 13) & 1u;
    a = a - ((uint32_t)(127 - 15) << 23) + 0x0fffu + odd;
    return (uint16_t)(sign | (a >> 13));
}

float lux_cpu_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {                                 /* zero / subnormal: m * 2^-24 */
        float v = (float)m * u2f(0x33800000u);    /* 2^-24, exact */
        return u2f(sign | f2u(v));
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

static inline float load_el(const void* p, size_t i, int dt) {
    switch (dt) {
    case LUX_CPU_F32:  return ((const float*)p)[i];
    case LUX_CPU_F16:  return lux_cpu_f16_to_f32(((const uint16_t*)p)[i]);
    default:           return lux_cpu_bf16_to_f32(((const uint16_t*)p)[i]);
    }
}

static inline void store_el(void* p, size_t i, int dt, float v) {
    switch (dt) {
    case LUX_CPU_F32:  ((float*)p)[i] = v; break;
    case LUX_CPU_F16:  ((uint16_t*)p)[i] = lux_cpu_f32_to_f16(v); break;
    default:           ((uint16_t*)p)[i] = lux_cpu_f32_to_bf16(v); break;
    }
}

void lux_cpu_convert(void* out, int out_dtype, const void* in, int in_dtype, size_t n) {
    for (size_t i = 0; i < n; i++) store_el(out, i, out_dtype, load_el(in, i, in_dtype));
}

/* ------------------------------------------------------------------------ */
/* PRNG                                                                     */
/* ------------------------------------------------------------------------ */

static uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

typedef struct { uint64_t s[4]; } xoshiro;

static void xo_seed(xoshiro* x, uint64_t seed) {
    uint64_t sm = seed;
    for (int i = 0; i < 4; i++) x->s[i] = splitmix64(&sm);
}

static inline uint64_t rotl(uint64_t v, int k) { return (v << k) | (v >> (64 - k)); }

static uint64_t xo_next(xoshiro* x) {          /* xoshiro256** */
    uint64_t* s = x->s;
    uint64_t r = rotl(s[1] * 5, 7) * 9;
    uint64_t t = s[1] << 17;
    s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return r;
}

void lux_cpu_rng_normal_f32(float* out, size_t n, uint64_t seed, float mean, float stddev) {
    xoshiro x;
    xo_seed(&x, seed);
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        /* u1 in (0, 1], u2 in [0, 1), 53-bit resolution */
        double u1 = (double)((xo_next(&x) >> 11) + 1) * 0x1.0p-53;
        double u2 = (double)(xo_next(&x) >> 11) * 0x1.0p-53;
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + stddev * (r * cos(two_pi * u2)));
        if (i + 1 < n) out[i + 1] = (float)(mean + stddev * (r * sin(two_pi * u2)));
    }
}

void lux_cpu_rng_u32(uint32_t* out, size_t n, uint64_t seed) {
    xoshiro x;
    xo_seed(&x, seed);
    for (size_t i = 0; i < n; i++) out[i] = (uint32_t)(xo_next(&x) >> 32);
}

/* ------------------------------------------------------------------------ */
/* validation                                                               */
/* ------------------------------------------------------------------------ */

static int bits_ok(int bits) {
    return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8;
}
static int dtype_ok(int dt) { return dt == LUX_CPU_F32 || dt == LUX_CPU_F16 || dt == LUX_CPU_BF16; }

int lux_cpu_quant_check(int M, int K, int N, int group_size, int bits,
                        int x_dtype, int sb_dtype, int out_dtype) {
    if (M < 0 || K <= 0 || N < 0) return LUX_CPU_EINVAL;
    if (!bits_ok(bits)) return LUX_CPU_ENOTSUP;
    if (group_size != 32 && group_size != 64 && group_size != 128) return LUX_CPU_ENOTSUP;
    if (K % group_size != 0) return LUX_CPU_EINVAL;       /* also makes K*bits % 32 == 0 */
    if (!dtype_ok(x_dtype) || !dtype_ok(sb_dtype) || !dtype_ok(out_dtype)) return LUX_CPU_ENOTSUP;
    return LUX_CPU_OK;
}

/* ------------------------------------------------------------------------ */
/* bitstream                                                                */
/* ------------------------------------------------------------------------ */

/* code k of a row: bits [k*bits, k*bits+bits) of the row's LE bitstream */
static inline uint32_t get_code(const uint32_t* row, int k, int bits) {
    uint32_t bit = (uint32_t)k * (uint32_t)bits;
    uint32_t w = bit >> 5, sh = bit & 31u;
    uint64_t pair = row[w];
    if (sh + (uint32_t)bits > 32u) pair |= (uint64_t)row[w + 1] << 32;
    return (uint32_t)(pair >> sh) & ((1u << bits) - 1u);
}

int lux_cpu_pack_bits(uint32_t* w_q, const uint8_t* codes, int N, int K, int bits) {
    if (!w_q || !codes || N < 0 || K <= 0 || bits < 1 || bits > 8 || ((long)K * bits) % 32)
        return LUX_CPU_EINVAL;
    const int wpr = K * bits / 32;
    memset(w_q, 0, (size_t)N * wpr * 4);
    for (int n = 0; n < N; n++) {
        uint32_t* row = w_q + (size_t)n * wpr;
        for (int k = 0; k < K; k++) {
            uint32_t q = codes[(size_t)n * K + k] & ((1u << bits) - 1u);
            uint32_t bit = (uint32_t)k * (uint32_t)bits;
            uint32_t w = bit >> 5, sh = bit & 31u;
            row[w] |= q << sh;
            if (sh + (uint32_t)bits > 32u) row[w + 1] |= q >> (32u - sh);
        }
    }
    return LUX_CPU_OK;
}

int lux_cpu_unpack_bits(uint8_t* codes, const uint32_t* w_q, int N, int K, int bits) {
    if (!w_q || !codes || N < 0 || K <= 0 || bits < 1 || bits > 8 || ((long)K * bits) % 32)
        return LUX_CPU_EINVAL;
    const int wpr = K * bits / 32;
    for (int n = 0; n < N; n++)
        for (int k = 0; k < K; k++)
            codes[(size_t)n * K + k] = (uint8_t)get_code(w_q + (size_t)n * wpr, k, bits);
    return LUX_CPU_OK;
}

/* ------------------------------------------------------------------------ */
/* quantize / dequantize                                                    */
/* ------------------------------------------------------------------------ */

int lux_cpu_quantize(uint32_t* w_q, void* scales, void* biases, const float* w,
                     int N, int K, int group_size, int bits, int sb_dtype) {
    int rc = lux_cpu_quant_check(1, K, N, group_size, bits, LUX_CPU_F32, sb_dtype, LUX_CPU_F32);
    if (rc) return rc;
    if (!w_q || !scales || !biases || !w) return LUX_CPU_EINVAL;
    const int G = K / group_size, wpr = K * bits / 32;
    const float levels = (float)((1u << bits) - 1u);
    const float qmax = levels;
    memset(w_q, 0, (size_t)N * wpr * 4);
    for (int n = 0; n < N; n++) {
        uint32_t* row = w_q + (size_t)n * wpr;
        for (int g = 0; g < G; g++) {
            const float* wg = w + (size_t)n * K + (size_t)g * group_size;
            float mn = wg[0], mx = wg[0];
            for (int i = 1; i < group_size; i++) {
                if (wg[i] < mn) mn = wg[i];
                if (wg[i] > mx) mx = wg[i];
            }
            float scale = (mx - mn) / levels;
            store_el(scales, (size_t)n * G + g, sb_dtype, scale);
            store_el(biases, (size_t)n * G + g, sb_dtype, mn);
            float s = load_el(scales, (size_t)n * G + g, sb_dtype);
            float b = load_el(biases, (size_t)n * G + g, sb_dtype);
            for (int i = 0; i < group_size; i++) {
                uint32_t q = 0;
                if (s != 0.0f) {
                    float v = nearbyintf((wg[i] - b) / s);
                    if (!(v >= 0.0f)) v = 0.0f;           /* also maps NaN to 0 */
                    if (v > qmax) v = qmax;
                    q = (uint32_t)v;
                }
                int k = g * group_size + i;
                uint32_t bit = (uint32_t)k * (uint32_t)bits;
                uint32_t wi = bit >> 5, sh = bit & 31u;
                row[wi] |= q << sh;
                if (sh + (uint32_t)bits > 32u) row[wi + 1] |= q >> (32u - sh);
            }
        }
    }
    return LUX_CPU_OK;
}

int lux_cpu_dequantize(void* out, const uint32_t* w_q, const void* scales,
                       const void* biases, int N, int K, int group_size,
                       int bits, int sb_dtype, int out_dtype) {
    int rc = lux_cpu_quant_check(1, K, N, group_size, bits, LUX_CPU_F32, sb_dtype, out_dtype);
    if (rc) return rc;
    if (!out || !w_q || !scales || !biases) return LUX_CPU_EINVAL;
    const int G = K / group_size, wpr = K * bits / 32;
    for (int n = 0; n < N; n++) {
        const uint32_t* row = w_q + (size_t)n * wpr;
        for (int k = 0; k < K; k++) {
            int g = k / group_size;
            float s = load_el(scales, (size_t)n * G + g, sb_dtype);
            float b = load_el(biases, (size_t)n * G + g, sb_dtype);
            float v = fmaf(s, (float)get_code(row, k, bits), b);
            store_el(out, (size_t)n * K + k, out_dtype, v);
        }
    }
    return LUX_CPU_OK;
}

/* ------------------------------------------------------------------------ */
/* quantized matmul                                                         */
/* ------------------------------------------------------------------------ */

static void dequant_row_f32(float* dst, const uint32_t* row, const void* scales,
                            const void* biases, int n, int K, int group_size,
                            int bits, int sb_dtype) {
    const int G = K / group_size;
    for (int k = 0; k < K; k++) {
        int g = k / group_size;
        float s = load_el(scales, (size_t)n * G + g, sb_dtype);
        float b = load_el(biases, (size_t)n * G + g, sb_dtype);
        dst[k] = fmaf(s, (float)get_code(row, k, bits), b);
    }
}

int lux_cpu_quantized_matmul(void* y, const void* x, const uint32_t* w_q,
                             const void* scales, const void* biases,
                             int M, int K, int N, int group_size, int bits,
                             int x_dtype, int sb_dtype, int out_dtype) {
    return lux_cpu_quantized_matmul_wround(y, x, w_q, scales, biases, M, K, N, group_size, bits,
                                           x_dtype, sb_dtype, out_dtype, LUX_CPU_F32);
}

int lux_cpu_quantized_matmul_wround(void* y, const void* x, const uint32_t* w_q,
                                    const void* scales, const void* biases,
                                    int M, int K, int N, int group_size, int bits,
                                    int x_dtype, int sb_dtype, int out_dtype, int w_dtype) {
    int rc = lux_cpu_quant_check(M, K, N, group_size, bits, x_dtype, sb_dtype, out_dtype);
    if (!rc && !dtype_ok(w_dtype)) rc = LUX_CPU_ENOTSUP;
    if (rc) return rc;
    if ((M && N) && (!y || !x || !w_q || !scales || !biases)) return LUX_CPU_EINVAL;
    const int wpr = K * bits / 32;
    float* wrow = (float*)malloc((size_t)K * sizeof(float));
    float* xf = (float*)malloc((size_t)M * K * sizeof(float) + 4);
    if (!wrow || !xf) { free(wrow); free(xf); return LUX_CPU_EINVAL; }
    for (size_t i = 0; i < (size_t)M * K; i++) xf[i] = load_el(x, i, x_dtype);
    for (int n = 0; n < N; n++) {
        dequant_row_f32(wrow, w_q + (size_t)n * wpr, scales, biases, n, K, group_size, bits, sb_dtype);
        if (w_dtype != LUX_CPU_F32)
            for (int k = 0; k < K; k++) {
                uint16_t h = w_dtype == LUX_CPU_F16 ? lux_cpu_f32_to_f16(wrow[k]) : lux_cpu_f32_to_bf16(wrow[k]);
                wrow[k] = w_dtype == LUX_CPU_F16 ? lux_cpu_f16_to_f32(h) : lux_cpu_bf16_to_f32(h);
            }
        for (int m = 0; m < M; m++) {
            const float* xr = xf + (size_t)m * K;
            float sum = 0.0f;
            for (int k = 0; k < K; k++) sum += xr[k] * wrow[k];
            store_el(y, (size_t)m * N + n, out_dtype, sum);
        }
    }
    free(wrow);
    free(xf);
    return LUX_CPU_OK;
}

int lux_cpu_quantized_matmul_f64(double* y, const void* x, const uint32_t* w_q,
                                 const void* scales, const void* biases,
                                 int M, int K, int N, int group_size, int bits,
                                 int x_dtype, int sb_dtype) {
    int rc = lux_cpu_quant_check(M, K, N, group_size, bits, x_dtype, sb_dtype, LUX_CPU_F32);
    if (rc) return rc;
    if ((M && N) && (!y || !x || !w_q || !scales || !biases)) return LUX_CPU_EINVAL;
    const int wpr = K * bits / 32;
    float* wrow = (float*)malloc((size_t)K * sizeof(float));
    if (!wrow) return LUX_CPU_EINVAL;
    for (int n = 0; n < N; n++) {
        dequant_row_f32(wrow, w_q + (size_t)n * wpr, scales, biases, n, K, group_size, bits, sb_dtype);
        for (int m = 0; m < M; m++) {
            double sum = 0.0;
            for (int k = 0; k < K; k++)
                sum += (double)load_el(x, (size_t)m * K + k, x_dtype) * (double)wrow[k];
            y[(size_t)m * N + n] = sum;
        }
    }
    free(wrow);
    return LUX_CPU_OK;
}
