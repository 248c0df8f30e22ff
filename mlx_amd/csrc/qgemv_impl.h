// qgemv_impl.h -- bandwidth-bound dequant-GEMV for small M (gfx950): kernel templates.
//
// y[m, n] = sum_k x[m, k] * (s[n,g] * q[n,k] + b[n,g]),  m < M <= 8.
//
// Work split: a wave owns a run of rows n; its 64 lanes split K.  Lane l of
// the wave takes "unit" u = l (+64, +128, ... for K > 4096) of every row: 64
// consecutive codes = 2*BITS words, read with 128-bit loads (plus one 64-bit
// load for BITS 3 and 5).  So lanes read consecutive memory and each lane's
// K range is the same for every row: the x values it needs are loaded from
// LDS once and reused across rows.
//
// Arithmetic (exact products): codes become 16-bit operands v(q) = 1 + q/2^BITS
// (one shift + one v_and_or_b32 per pair for BITS 2/4/8), multiplied with x by
// v_dot2_f32_{f16,bf16} in fp32.  Per group
//     s*sum x q + b*sum x  =  (s*2^BITS) * sum x v(q)  +  (b - s*2^BITS) * xs,
// xs = sum of x over the group, computed once per block.  fp32 activations
// use plain fp32 FMAs.  Lane partials are reduced with DPP row operations and
// readlane (no LDS).
#pragma once
#include "kernels.h"
#include "qcommon.h"

namespace lxq {
namespace gemv {

constexpr int kThreads = 256;  // 4 waves

template <int TX>
struct XLds {
    static constexpr int kElem = (TX == DT_F32) ? 4 : 2;
    // one 64-code unit = 64 elements + padding so that ds_read_b128 of
    // consecutive lanes spread over the LDS banks
    static constexpr int kUnitStride = (TX == DT_F32) ? 68 : 72;  // elements
};

template <int BITS>
__device__ __forceinline__ void load_unit(const uint32_t* __restrict__ p, uint32_t* w) {
    constexpr int W = 2 * BITS;
#pragma unroll
    for (int i = 0; i + 4 <= W; i += 4) {
        u32x4 v = *reinterpret_cast<const u32x4*>(p + i);
        w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
    }
    if constexpr (W % 4 == 2) {
        u32x2 v = *reinterpret_cast<const u32x2*>(p + (W - 2));
        w[W - 2] = v.x; w[W - 1] = v.y;
    }
}

template <int BITS, int TX, int MR, int RU>
__global__ __launch_bounds__(kThreads) void qgemv_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, int gsize,
    int sb_dt, int out_dt, int rows_per_wave) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    using XL = XLds<TX>;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int units = K >> 6;
    const int slabs = (units + 63) >> 6;
    const int G = K / gsize;
    const int row_words = (K * BITS) >> 5;
    const int x_row_elems = units * XL::kUnitStride;
    float* xs_lds = reinterpret_cast<float*>(smem + (size_t)MR * x_row_elems * XL::kElem);

    constexpr float kPow = MagicCfg<BITS, (TX == DT_F16 ? 10 : 7)>::kPow;
    // bf16 cannot hold 1 + q/256: 8-bit codes with bf16 x use v(q) = q
    constexpr bool kMagic = (TX != DT_F32) && !(TX == DT_BF16 && BITS == 8);
    // x order matches the operand pairing of the codes
    constexpr bool kApartX = kMagic && PairLayout<BITS>::kApart;

    // ---- stage x[M][K] into LDS (slot order + padding) and group sums ----
    for (int idx = threadIdx.x; idx < M * K; idx += kThreads) {
        const int m = idx / K, k = idx - m * K;
        const int u = k >> 6, c = k & 63;
        const int dst = m * x_row_elems + u * XL::kUnitStride + (kApartX ? x_slot<BITS>(c) : c);
        if constexpr (TX == DT_F32)
            reinterpret_cast<float*>(smem)[dst] = reinterpret_cast<const float*>(x)[idx];
        else
            reinterpret_cast<uint16_t*>(smem)[dst] = reinterpret_cast<const uint16_t*>(x)[idx];
    }
    // sums of x over every 32-code half unit: the bias term of a group is
    // b * (sum of x over the group) and a unit covers 2 halves
    const int H = K >> 5;
    for (int idx = threadIdx.x; idx < M * H; idx += kThreads) {
        const int m = idx / H, h = idx - m * H;
        float s = 0.f;
        for (int k = h * 32; k < h * 32 + 32; k++) s += load_f(x, (size_t)m * K + k, TX);
        xs_lds[idx] = s;
    }
    __syncthreads();

    const int n_begin = (blockIdx.x * (kThreads / 64) + wave) * rows_per_wave;
    const int n_end = min(N, n_begin + rows_per_wave);

    for (int n0 = n_begin; n0 < n_end; n0 += RU) {
        float acc[RU][MR];
#pragma unroll
        for (int r = 0; r < RU; r++)
#pragma unroll
            for (int m = 0; m < MR; m++) acc[r][m] = 0.f;

        for (int sl = 0; sl < slabs; sl++) {
            const int u = sl * 64 + lane;
            const bool active = u < units;
            const int g0 = (u * 64) / gsize;
            uint32_t wv[RU][2 * BITS];
            float sc[RU][2], bi[RU][2];
            // issue all loads of the batch first (memory-level parallelism)
#pragma unroll
            for (int r = 0; r < RU; r++) {
                const int n = n0 + r;
                if (active && n < n_end) {
                    load_unit<BITS>(wq + (size_t)n * row_words + (size_t)u * 2 * BITS, wv[r]);
                    sc[r][0] = load_f(scales, (size_t)n * G + g0, sb_dt);
                    bi[r][0] = load_f(biases, (size_t)n * G + g0, sb_dt);
                    if (gsize == 32) {
                        sc[r][1] = load_f(scales, (size_t)n * G + g0 + 1, sb_dt);
                        bi[r][1] = load_f(biases, (size_t)n * G + g0 + 1, sb_dt);
                    } else {
                        sc[r][1] = sc[r][0];
                        bi[r][1] = bi[r][0];
                    }
                }
            }
            if (!active) continue;
#pragma unroll
            for (int r = 0; r < RU; r++) {
                const int n = n0 + r;
                if (n >= n_end) continue;
                // per m: D0, D1 = sums over the two 32-code halves of the unit
                if constexpr (TX == DT_F32) {
                    float q[64];
#pragma unroll
                    for (int i = 0; i < 64; i++) q[i] = (float)unit_code<BITS>(wv[r], i);
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        if (m >= M) break;
                        const float* xl = reinterpret_cast<const float*>(smem) +
                                          m * x_row_elems + u * XL::kUnitStride;
                        float d0 = 0.f, d1 = 0.f;
#pragma unroll
                        for (int i = 0; i < 32; i++) d0 = fmaf(xl[i], q[i], d0);
#pragma unroll
                        for (int i = 32; i < 64; i++) d1 = fmaf(xl[i], q[i], d1);
                        const float h0 = xs_lds[m * H + 2 * u], h1 = xs_lds[m * H + 2 * u + 1];
                        acc[r][m] += (sc[r][0] * d0 + bi[r][0] * h0) + (sc[r][1] * d1 + bi[r][1] * h1);
                    }
                } else {
                    uint32_t pr[32];
                    if constexpr (kMagic)
                        unit_pairs_magic<BITS, (TX == DT_F16 ? 10 : 7)>(wv[r], pr);
                    else
                        unit_pairs_bf16_u8(wv[r], pr);
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        if (m >= M) break;
                        const u32x4* xl = reinterpret_cast<const u32x4*>(
                            reinterpret_cast<const uint16_t*>(smem) + m * x_row_elems +
                            u * XL::kUnitStride);
                        float d0 = 0.f, d1 = 0.f;
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            u32x4 xv = xl[i];
                            d0 = dot2(xv.x, pr[4 * i], d0, TX);
                            d0 = dot2(xv.y, pr[4 * i + 1], d0, TX);
                            d0 = dot2(xv.z, pr[4 * i + 2], d0, TX);
                            d0 = dot2(xv.w, pr[4 * i + 3], d0, TX);
                        }
#pragma unroll
                        for (int i = 4; i < 8; i++) {
                            u32x4 xv = xl[i];
                            d1 = dot2(xv.x, pr[4 * i], d1, TX);
                            d1 = dot2(xv.y, pr[4 * i + 1], d1, TX);
                            d1 = dot2(xv.z, pr[4 * i + 2], d1, TX);
                            d1 = dot2(xv.w, pr[4 * i + 3], d1, TX);
                        }
                        const float h0 = xs_lds[m * H + 2 * u], h1 = xs_lds[m * H + 2 * u + 1];
                        if constexpr (kMagic) {
                            // D = sum x v(q) = h + 2^-B sum x q  =>
                            // s sum x q + b h = (s 2^B) D + (b - s 2^B) h
                            acc[r][m] += ((sc[r][0] * kPow) * d0 + fmaf(-sc[r][0], kPow, bi[r][0]) * h0) +
                                         ((sc[r][1] * kPow) * d1 + fmaf(-sc[r][1], kPow, bi[r][1]) * h1);
                        } else {
                            acc[r][m] += (sc[r][0] * d0 + bi[r][0] * h0) + (sc[r][1] * d1 + bi[r][1] * h1);
                        }
                    }
                }
            }
        }
        // ---- reduce lane partials and store ----
#pragma unroll
        for (int r = 0; r < RU; r++) {
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const float v = wave_sum(acc[r][m]);
                if (lane == 0 && m < M && n0 + r < n_end) store_f(y, (size_t)m * N + n0 + r, out_dt, v);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Register-x variant for K <= 4096 (one 64-code unit per lane) and M <= 4:
// each wave owns R consecutive rows.  It issues its x loads first (L2
// hits), then the weight loads of all R rows, then computes row r as soon
// as row r has arrived, so the other rows' HBM traffic overlaps the math.
// No LDS and no barriers.
// ---------------------------------------------------------------------------

// x for one lane's unit: 64 values, permuted into the operand-pair order of
// the codes, plus the sums over the two 32-value halves
template <int BITS, int TX, bool APART>
__device__ __forceinline__ void lane_x_pairs(const void* __restrict__ x, size_t off, uint32_t* xp,
                                             float& h0, float& h1) {
    const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(x) + off);
    uint32_t nat[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        u32x4 v = p[i];
        nat[4 * i] = v.x; nat[4 * i + 1] = v.y; nat[4 * i + 2] = v.z; nat[4 * i + 3] = v.w;
    }
    // half sums: dot2 against (1, 1) is exact per product, fp32 accumulate
    const uint32_t one2 = TX == DT_F16 ? 0x3C003C00u : 0x3F803F80u;
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) a = dot2(nat[i], one2, a, TX);
#pragma unroll
    for (int i = 16; i < 32; i++) b = dot2(nat[i], one2, b, TX);
    h0 = a;
    h1 = b;
    if constexpr (APART) {
        // block of P codes = P/2 dwords; pair j = (x_j, x_{j+P/2})
        constexpr int P = PairLayout<BITS>::kCodesPerWord, D = P / 2;  // dwords per block
#pragma unroll
        for (int blk = 0; blk < 64 / P; blk++) {
#pragma unroll
            for (int j = 0; j < D; j++) {
                // element j lives in dword j/2 (half j%2); element j+P/2 in dword (j+D)/2 ... of the block
                const int e0 = j, e1 = j + D;  // element indices within the block (D = P/2)
                const uint32_t w0 = nat[blk * D + e0 / 2], w1 = nat[blk * D + e1 / 2];
                const uint32_t lo = (e0 & 1) ? (w0 >> 16) : (w0 & 0xffffu);
                const uint32_t hi = (e1 & 1) ? (w1 & 0xffff0000u) : (w1 << 16);
                xp[blk * D + j] = lo | hi;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) xp[i] = nat[i];
    }
}

// raw element i of a T_sb array (compile-time dtype: no branches, so the
// compiler keeps every load of the wave in flight)
template <int DT>
__device__ __forceinline__ float load_c(const void* __restrict__ p, size_t i) {
    if constexpr (DT == DT_F32) return reinterpret_cast<const float*>(p)[i];
    else if constexpr (DT == DT_F16) return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    else return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

template <int BITS, int TX, int SB, int MR, int R>
__global__ __launch_bounds__(kThreads) void qgemv_reg_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, int gsize,
    int out_dt) {
    constexpr bool kMagic = (TX != DT_F32) && !(TX == DT_BF16 && BITS == 8);
    constexpr bool kApartX = kMagic && PairLayout<BITS>::kApart;
    constexpr float kPow = MagicCfg<BITS, (TX == DT_F16 ? 10 : 7)>::kPow;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * (kThreads / 64) + wave) * R;
    if (n0 >= N) return;  // wave-uniform
    const int units = K >> 6;
    const bool active = lane < units;
    // loads are unconditional: idle lanes and rows past N read clamped (valid)
    // addresses and their results are never stored
    const int u = active ? lane : units - 1;
    const int G = K / gsize;
    const int row_words = (K * BITS) >> 5;
    const int g0 = (u * 64) / gsize;
    const int g1 = g0 + (gsize == 32 ? 1 : 0);

    // ---- x first (L2-resident, shared by every wave) ----
    uint32_t xp[MR][32];
    float xf[TX == DT_F32 ? MR : 1][TX == DT_F32 ? 64 : 1];
    float h0[MR], h1[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) {
        const int mc = m < M ? m : M - 1;
        if constexpr (TX == DT_F32) {
            const u32x4* p = reinterpret_cast<const u32x4*>(
                reinterpret_cast<const float*>(x) + (size_t)mc * K + u * 64);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                u32x4 v = p[i];
                xf[m][4 * i] = __uint_as_float(v.x); xf[m][4 * i + 1] = __uint_as_float(v.y);
                xf[m][4 * i + 2] = __uint_as_float(v.z); xf[m][4 * i + 3] = __uint_as_float(v.w);
            }
        } else {
            lane_x_pairs<BITS, TX, kApartX>(x, (size_t)mc * K + u * 64, xp[m], h0[m], h1[m]);
        }
    }

    // ---- weight loads of all R rows ----
    uint32_t wv[R][2 * BITS];
    float sc[R][2], bi[R][2];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int n = (n0 + r < N) ? n0 + r : N - 1;
        load_unit<BITS>(wq + (size_t)n * row_words + (size_t)u * 2 * BITS, wv[r]);
        sc[r][0] = load_c<SB>(scales, (size_t)n * G + g0);
        bi[r][0] = load_c<SB>(biases, (size_t)n * G + g0);
    }
    // group 32: the unit's second half has its own scale and bias
    if (gsize == 32) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int n = (n0 + r < N) ? n0 + r : N - 1;
            sc[r][1] = load_c<SB>(scales, (size_t)n * G + g1);
            bi[r][1] = load_c<SB>(biases, (size_t)n * G + g1);
        }
    } else {
#pragma unroll
        for (int r = 0; r < R; r++) {
            sc[r][1] = sc[r][0];
            bi[r][1] = bi[r][0];
        }
    }

    if constexpr (TX == DT_F32) {
#pragma unroll
        for (int m = 0; m < MR; m++) {
            float a = 0.f, b = 0.f;
#pragma unroll
            for (int i = 0; i < 32; i++) a += xf[m][i];
#pragma unroll
            for (int i = 32; i < 64; i++) b += xf[m][i];
            h0[m] = a;
            h1[m] = b;
        }
    }

    float acc[R][MR];
#pragma unroll
    for (int r = 0; r < R; r++) {
        if constexpr (TX == DT_F32) {
            float q[64];
#pragma unroll
            for (int i = 0; i < 64; i++) q[i] = (float)unit_code<BITS>(wv[r], i);
#pragma unroll
            for (int m = 0; m < MR; m++) {
                float d0 = 0.f, d1 = 0.f;
#pragma unroll
                for (int i = 0; i < 32; i++) d0 = fmaf(xf[m][i], q[i], d0);
#pragma unroll
                for (int i = 32; i < 64; i++) d1 = fmaf(xf[m][i], q[i], d1);
                acc[r][m] = (sc[r][0] * d0 + bi[r][0] * h0[m]) + (sc[r][1] * d1 + bi[r][1] * h1[m]);
            }
        } else {
            uint32_t pr[32];
            if constexpr (kMagic)
                unit_pairs_magic<BITS, (TX == DT_F16 ? 10 : 7)>(wv[r], pr);
            else
                unit_pairs_bf16_u8(wv[r], pr);
            const float s0 = kMagic ? sc[r][0] * kPow : sc[r][0];
            const float s1 = kMagic ? sc[r][1] * kPow : sc[r][1];
            const float c0 = kMagic ? fmaf(-sc[r][0], kPow, bi[r][0]) : bi[r][0];
            const float c1 = kMagic ? fmaf(-sc[r][1], kPow, bi[r][1]) : bi[r][1];
#pragma unroll
            for (int m = 0; m < MR; m++) {
                float d0 = 0.f, d1 = 0.f;
#pragma unroll
                for (int i = 0; i < 16; i++) d0 = dot2(xp[m][i], pr[i], d0, TX);
#pragma unroll
                for (int i = 16; i < 32; i++) d1 = dot2(xp[m][i], pr[i], d1, TX);
                acc[r][m] = (s0 * d0 + c0 * h0[m]) + (s1 * d1 + c1 * h1[m]);
            }
        }
        if (!active) {
#pragma unroll
            for (int m = 0; m < MR; m++) acc[r][m] = 0.f;
        }
    }

    // ---- reduce across the wave; lane r*MR+m stores (row r, x row m) ----
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int m = 0; m < MR; m++) {
            const float v = wave_sum(acc[r][m]);
            if (lane == r * MR + m && m < M && n0 + r < N) store_f(y, (size_t)m * N + n0 + r, out_dt, v);
        }
    }
}

template <int BITS, int TX, int SB, int MR, int R>
LuxStatus launch_reg(const QmmArgs& a, hipStream_t st) {
    const int waves = (a.N + R - 1) / R;
    const int blocks = (waves + 3) / 4;
    hipLaunchKernelGGL((qgemv_reg_kernel<BITS, TX, SB, MR, R>), dim3(blocks), dim3(kThreads), 0, st,
                       a.x, a.wq, a.scales, a.biases, a.y, a.M, a.K, a.N, a.group_size, a.out_dtype);
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

// rows per wave: keep the in-flight weight words per lane near 64
template <int BITS, int TX, int MR>
LuxStatus launch_reg_r(const QmmArgs& a, hipStream_t st) {
    constexpr int R = (MR >= 4) ? 4 : (BITS <= 4 ? 8 : 4);
    switch (a.sb_dtype) {
    case DT_F32: return launch_reg<BITS, TX, DT_F32, MR, R>(a, st);
    case DT_F16: return launch_reg<BITS, TX, DT_F16, MR, R>(a, st);
    default: return launch_reg<BITS, TX, DT_BF16, MR, R>(a, st);
    }
}

template <int BITS, int TX, int MR>
LuxStatus launch_t(const QmmArgs& a, hipStream_t st) {
    constexpr int RU = 4;
    using XL = XLds<TX>;
    const int units = a.K / 64;
    const size_t lds = (size_t)MR * units * XL::kUnitStride * XL::kElem + (size_t)MR * (a.K / 32) * 4;
    if (lds > 64 * 1024) return LuxStatus::NotSupported;
    (void)units;
    // rows per wave: enough waves to cover the chip several times over
    const int waves_wanted = 256 * 8;
    int rpw = (a.N + waves_wanted - 1) / waves_wanted;
    rpw = ((rpw + RU - 1) / RU) * RU;
    if (rpw < RU) rpw = RU;
    const int waves = (a.N + rpw - 1) / rpw;
    const int blocks = (waves + 3) / 4;
    auto kern = qgemv_kernel<BITS, TX, MR, RU>;
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024) != hipSuccess)
            return LuxStatus::Internal;
        attr_set = true;
    }
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(kThreads), lds, st, a.x, a.wq, a.scales, a.biases,
                       a.y, a.M, a.K, a.N, a.group_size, a.sb_dtype, a.out_dtype, rpw);
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

template <int BITS, int TX>
LuxStatus launch_m(const QmmArgs& a, hipStream_t st) {
    if (a.K <= 4096 && (a.M <= 4 && (TX != DT_F32 || a.M == 1))) {
        if (a.M <= 1) return launch_reg_r<BITS, TX, 1>(a, st);
        if (a.M <= 2) return launch_reg_r<BITS, TX, 2>(a, st);
        return launch_reg_r<BITS, TX, 4>(a, st);
    }
    if (a.M <= 1) return launch_t<BITS, TX, 1>(a, st);
    if (a.M <= 2) return launch_t<BITS, TX, 2>(a, st);
    if (a.M <= 4) return launch_t<BITS, TX, 4>(a, st);
    return launch_t<BITS, TX, 8>(a, st);
}

template <int BITS>
LuxStatus launch_b(const QmmArgs& a, hipStream_t st) {
    switch (a.x_dtype) {
    case DT_F32: return launch_m<BITS, DT_F32>(a, st);
    case DT_F16: return launch_m<BITS, DT_F16>(a, st);
    default: return launch_m<BITS, DT_BF16>(a, st);
    }
}

// one explicit instantiation per bit width lives in qgemv_b<BITS>.hip
extern template LuxStatus launch_b<2>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_b<3>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_b<4>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_b<5>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_b<6>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_b<8>(const QmmArgs&, hipStream_t);

}  // namespace gemv
}  // namespace lxq
