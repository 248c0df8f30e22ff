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

// one thread per (row, group): the group's codes fill whole words
// (group_size * bits is a multiple of 32), so no two threads share a word
__global__ __launch_bounds__(256) void quantize_kernel(const void* __restrict__ w,
                                                       uint32_t* __restrict__ wq,
                                                       void* __restrict__ sc, void* __restrict__ bi,
                                                       int N, int K, int gsize, int bits, int w_dt,
                                                       int sb_dt) {
    const int G = K / gsize, rw = (K * bits) >> 5;
    const size_t total = (size_t)N * G;
    const float levels = (float)((1u << bits) - 1u);
    for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (size_t)gridDim.x * blockDim.x) {
        const int n = (int)(t / G), g = (int)(t - (size_t)n * G);
        const size_t base = (size_t)n * K + (size_t)g * gsize;
        float mn = load_f(w, base, w_dt), mx = mn;
        for (int i = 1; i < gsize; i++) {
            const float v = load_f(w, base + i, w_dt);
            mn = v < mn ? v : mn;
            mx = v > mx ? v : mx;
        }
        // the codes are computed from the stored (rounded) scale and bias
        const float s = round_dt((mx - mn) / levels, sb_dt), b = round_dt(mn, sb_dt);
        store_f(sc, t, sb_dt, s);
        store_f(bi, t, sb_dt, b);
        uint32_t* row = wq + (size_t)n * rw;
        const int w0 = (g * gsize * bits) >> 5;
        uint64_t accb = 0;  // bit accumulator
        int nb = 0, wo = 0;
        for (int i = 0; i < gsize; i++) {
            uint32_t q = 0;
            if (s != 0.0f) {
                float v = rintf((load_f(w, base + i, w_dt) - b) / s);
                v = (v >= 0.0f) ? v : 0.0f;  // NaN -> 0
                v = v > levels ? levels : v;
                q = (uint32_t)v;
            }
            accb |= (uint64_t)q << nb;
            nb += bits;
            if (nb >= 32) {
                row[w0 + wo++] = (uint32_t)accb;
                accb >>= 32;
                nb -= 32;
            }
        }
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
                                                          int sb_dt, int out_dt) {
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
        store_f(y, i, out_dt, acc);
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

LuxStatus launch_quantize(const void* w, uint32_t* wq, void* scales, void* biases, int N, int K,
                          int group_size, int bits, int w_dtype, int sb_dtype, hipStream_t st) {
    const size_t groups = (size_t)N * (K / group_size);
    if (groups == 0) return LuxStatus::Ok;
    hipLaunchKernelGGL(quantize_kernel, dim3(grid_for(groups)), dim3(256), 0, st, w, wq, scales,
                       biases, N, K, group_size, bits, w_dtype, sb_dtype);
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

LuxStatus launch_qmm_generic(const QmmArgs& a, hipStream_t st) {
    const size_t total = (size_t)a.M * a.N;
    if (total == 0) return LuxStatus::Ok;
    hipLaunchKernelGGL(qmm_generic_kernel, dim3(grid_for(total)), dim3(256), 0, st, a.x, a.wq,
                       a.scales, a.biases, a.y, a.M, a.K, a.N, a.group_size, a.bits, a.x_dtype,
                       a.sb_dtype, a.out_dtype);
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

}  // namespace lxq
