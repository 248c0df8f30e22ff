// qmm_skinny.h -- MFMA kernel for small M (2..16 rows of x), 4- and 8-bit
// codes, f16/bf16 activations (gfx950).
//
// y[m, n] = sum_g s[n,g] * sum_{k in g} q[n,k] x[m,k] + b[n,g] * sum_{k in g} x[m,k]
//
// Work split: a 16-row tile of W is the A operand of v_mfma_f32_16x16x32
// (row i = lane % 16), x is the B operand (column m = lane % 16; columns
// past M repeat row M-1 and are never stored).  A block of 4 waves owns one
// tile for KS = 4, two for KS = 2, four for KS = 1; the KS waves of a tile
// split its K range, GW groups each, and their partial sums meet in LDS.
//
// Every MFMA covers 32 codes of one group: lane group c = lane / 16 holds 8
// of them, so the group's partial D = sum v(q) x is complete after GS/32
// MFMAs and is scaled by s[n,g] in fp32 right away (v(q) = A0 + q U, see
// Form).  One more MFMA per group with an all-ones A operand yields
// sx = sum_{k in g} x; the offset and bias terms sum_g (b/kPow - A0 s) sx
// are a [16 x G] x [G x 16] product that v_mfma_f32_16x16x4_f32 adds at the
// end.
//
// x sits in LDS (M rows, row stride 2K + 16 bytes: the 16 B pad puts the 16
// rows a B-operand read touches in 16 different bank groups).  The wave's
// weight loads are all issued up front (GW groups, <= 32 loads).
#pragma once
#include "kernels.h"
#include "qcommon.h"
#include "qgemv_impl.h"

namespace lxq {
namespace skinny {

using gemv::buf_rsrc;
using gemv::lds_ptr;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;

template <int TX>
__device__ __forceinline__ f32x4 mfma32(const u4& a, const u4& b, const f32x4& c) {
    if constexpr (TX == DT_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                     0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                      __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Code operand v = A0 + q * U (exact in T); per group sum v x = A0 sx + U sum q x,
// so s sum q x + b sx = kPow * (s D + (b / kPow - s A0) sx) with kPow = 1/U.
//   f16, 4-bit: q at mantissa bits 4..7 of 1.0: v = 1 + q/64 (A0 = 1, kPow = 64)
//   f16, 8-bit: q at bits 0..7 of 1024:        v = 1024 + q  (A0 = 1024)
//   bf16, 4-bit: q at bits 0..3 of 128:        v = 128 + q   (A0 = 128)
//   bf16, 8-bit: v = q through fp32            (A0 = 0)
// The offset A0 cancels against its own sx term; keeping A0/kPow small keeps
// that cancellation within fp32's headroom (8x for 4-bit f16, ~10x otherwise).
template <int BITS, int TX>
struct Form {
    static constexpr bool kCvt = (BITS == 8 && TX == DT_BF16);  // 8-bit codes exceed bf16's mantissa
    static constexpr bool kHigh = (BITS == 4 && TX == DT_F16);   // codes at bits 4..7
    static constexpr float kA0 = kCvt ? 0.f : kHigh ? 1.f : (TX == DT_F16 ? 1024.f : 128.f);
    static constexpr float kPow = kHigh ? 64.f : 1.f;
    static constexpr uint32_t kMagic = kHigh ? 0x3C003C00u : TX == DT_F16 ? 0x64006400u : 0x43004300u;
    static constexpr uint32_t kMask = BITS == 8 ? 0x00FF00FFu : kHigh ? 0x00F000F0u : 0x000F000Fu;
    static constexpr uint32_t kOne2 = TX == DT_F16 ? 0x3C003C00u : 0x3F803F80u;
    static constexpr int kWordsPerMfma = BITS / 4;  // 8 codes
};

// A operand (8 codes) of one MFMA from BITS/4 words.  The masks and the
// magic live in VGPRs (vm, vmagic) so that the compiler emits its own
// v_and_or_b32 (whose results the MFMA may read: the compiler inserts the
// VALU -> MFMA wait states for its own instructions, not for inline asm).
template <int BITS, int TX>
__device__ __forceinline__ u4 code_operand(const uint32_t* w, uint32_t vm, uint32_t vmagic) {
    using F = Form<BITS, TX>;
    u4 r;
    if constexpr (BITS == 4 && F::kHigh) {
        // pairs (c_j, c_{j+4}) moved to bits 4..7: x order x0 x4 x1 x5 x2 x6 x3 x7
        r.x = ((w[0] << 4) & vm) | vmagic;
        r.y = (w[0] & vm) | vmagic;
        r.z = ((w[0] >> 4) & vm) | vmagic;
        r.w = ((w[0] >> 8) & vm) | vmagic;
    } else if constexpr (BITS == 4) {
        // pairs (c_j, c_{j+4}) at bits 0..3: x order x0 x4 x1 x5 x2 x6 x3 x7
        r.x = (w[0] & vm) | vmagic;
        r.y = ((w[0] >> 4) & vm) | vmagic;
        r.z = ((w[0] >> 8) & vm) | vmagic;
        r.w = ((w[0] >> 12) & vm) | vmagic;
    } else if constexpr (!F::kCvt) {
        // pairs (c0,c2) (c1,c3) of each word: x order x0 x2 x1 x3 x4 x6 x5 x7
        r.x = (w[0] & vm) | vmagic;
        r.y = ((w[0] >> 8) & vm) | vmagic;
        r.z = (w[1] & vm) | vmagic;
        r.w = ((w[1] >> 8) & vm) | vmagic;
    } else {
        // natural pairs: the fp32 value of a byte is an exact bf16 in its upper half
        uint32_t f[8];
#pragma unroll
        for (int i = 0; i < 8; i++) f[i] = __float_as_uint((float)((w[i >> 2] >> (8 * (i & 3))) & 0xFFu));
        r.x = __builtin_amdgcn_perm(f[1], f[0], 0x07060302u);
        r.y = __builtin_amdgcn_perm(f[3], f[2], 0x07060302u);
        r.z = __builtin_amdgcn_perm(f[5], f[4], 0x07060302u);
        r.w = __builtin_amdgcn_perm(f[7], f[6], 0x07060302u);
    }
    return r;
}

// B operand: 8 consecutive x values (natural order n0..n3) permuted into the
// code operand's order
template <int BITS, int TX>
__device__ __forceinline__ u4 x_operand(const u4& n) {
    using F = Form<BITS, TX>;
    if constexpr (BITS == 4) {
        return u4{__builtin_amdgcn_perm(n.z, n.x, 0x05040100u), __builtin_amdgcn_perm(n.z, n.x, 0x07060302u),
                  __builtin_amdgcn_perm(n.w, n.y, 0x05040100u), __builtin_amdgcn_perm(n.w, n.y, 0x07060302u)};
    } else if constexpr (!F::kCvt) {
        return u4{__builtin_amdgcn_perm(n.y, n.x, 0x05040100u), __builtin_amdgcn_perm(n.y, n.x, 0x07060302u),
                  __builtin_amdgcn_perm(n.w, n.z, 0x05040100u), __builtin_amdgcn_perm(n.w, n.z, 0x07060302u)};
    } else {
        return n;
    }
}

template <int SB>
__device__ __forceinline__ float sb_at(const uint8_t* p, int i) {
    if constexpr (SB == DT_F32) return reinterpret_cast<const float*>(p)[i];
    else if constexpr (SB == DT_F16) return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    else return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

template <int BITS, int GS>
struct Geo {
    static constexpr int kMfma = GS / 32;                   // MFMAs per group
    static constexpr int kWords = GS * BITS / 128;          // words per lane per group
    static constexpr int kLaneBytes = 4 * kWords;           // contiguous bytes per lane per group
    static constexpr int kGroupBytes = GS * BITS / 8;       // bytes of a group in a row
};

// LDS: x rows | scale rows | bias rows | partial sums of the K-split
__host__ __device__ constexpr size_t skinny_lds_bytes(int M, int K, int G, int sb_size, int tiles) {
    return (size_t)M * (2 * K + 16) + 2 * (size_t)16 * tiles * G * sb_size + (size_t)(kWaves - tiles) * 64 * 16;
}

template <int BITS, int TX, int SB, int GS, int GW, bool EPI>
__global__ __launch_bounds__(64 * kWaves) void qmm_skinny_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, int KS, Epilogue ep) {
    using F = Form<BITS, TX>;
    using Q = Geo<BITS, GS>;
    constexpr int kSb = SB == DT_F32 ? 4 : 2;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tiles = kWaves / KS;                 // tiles per block
    const int tile = wave / KS, part = wave % KS;  // this wave's tile and K part
    const int G = K / GS;
    const int XS = 2 * K + 16;                     // x row stride in LDS
    const int n_blk = blockIdx.x * 16 * tiles;     // first row of the block
    const int n_tile = n_blk + 16 * tile;
    const int i = lane & 15, c = lane >> 4;        // A: row i of the tile, lane group c
    uint8_t* const lx = lds;
    uint8_t* const ls = lds + (size_t)M * XS;
    uint8_t* const lb = ls + (size_t)16 * tiles * G * kSb;
    float* const lred = reinterpret_cast<float*>(lb + (size_t)16 * tiles * G * kSb);

    // ---- 1. DMA: x rows, the block's scale and bias rows ----
    {
        const auto xr = buf_rsrc(x, (uint32_t)M * K * 2);
        const int kc = K / 8;  // 16-byte chunks per x row
        for (int m = 0; m < M; m++)
            for (int c0 = wave * 64; c0 < kc; c0 += 64 * kWaves)
                if (c0 + lane < kc)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr)(lx + m * XS + c0 * 16), 16,
                                                             (uint32_t)(m * K * 2 + (c0 + lane) * 16), 0, 0, 0);
        const uint32_t row = (uint32_t)G * kSb;
        const uint32_t sbytes = ((uint32_t)N * row + 15u) & ~15u;  // tail chunk: buffer slack
        const auto sr = buf_rsrc(scales, sbytes), br = buf_rsrc(biases, sbytes);
        const int sc = (int)(16 * tiles * row / 16);  // the block's rows, 16 B chunks (rows are 16-row aligned)
        for (int c0 = wave * 64; c0 < sc; c0 += 64 * kWaves)
            if (c0 + lane < sc) {
                const uint32_t off = (uint32_t)n_blk * row + (uint32_t)(c0 + lane) * 16;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_ptr)(ls + c0 * 16), 16, off, 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(br, (lds_ptr)(lb + c0 * 16), 16, off, 0, 0, 0);
            }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. this wave's codes: GW groups of row n_tile + i, lane group c's slice ----
    constexpr int W = Q::kWords;
    uint32_t wv[GW][W];
    {
        const uint32_t row_bytes = (uint32_t)K * BITS / 8;
        const auto wr = buf_rsrc(wq, (uint32_t)N * row_bytes);
        const int n = n_tile + i < N ? n_tile + i : N - 1;  // rows past N: valid data, never stored
        const uint32_t base = (uint32_t)n * row_bytes + (uint32_t)(part * GW) * Q::kGroupBytes + c * Q::kLaneBytes;
#pragma unroll
        for (int g = 0; g < GW; g++) {
            const uint32_t off = base + g * Q::kGroupBytes;
            if constexpr (W == 1) {
                wv[g][0] = __builtin_amdgcn_raw_buffer_load_b32(wr, off, 0, 0);
            } else if constexpr (W == 2) {
                const u2 v = __builtin_amdgcn_raw_buffer_load_b64(wr, off, 0, 0);
                wv[g][0] = v.x; wv[g][1] = v.y;
            } else {
#pragma unroll
                for (int q = 0; q < W; q += 4) {
                    const u4 v = __builtin_amdgcn_raw_buffer_load_b128(wr, off + 4 * q, 0, 0);
                    wv[g][q] = v.x; wv[g][q + 1] = v.y; wv[g][q + 2] = v.z; wv[g][q + 3] = v.w;
                }
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    {
        constexpr int NW = GW * (W >= 4 ? W / 4 : 1);
        static_assert(NW < 64, "vmcnt holds 6 bits");
        __builtin_amdgcn_s_waitcnt((NW & 0xF) | ((NW >> 4) << 14) | (0x7 << 4) | (0xF << 8));
    }
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // ---- 3. groups: per group, MFMAs of codes and of ones, then scale ----
    const int j = lane & 15;                       // B: column m = j
    const int jm = j < M ? j : M - 1;
    const uint8_t* xrow = lx + jm * XS + (size_t)(part * GW) * GS * 2 + c * (GS / 4) * 2;
    const uint8_t* srow = ls + (size_t)(16 * tile + 4 * c) * G * kSb;  // D rows 4c..4c+3 of the tile
    const u4 ones = {F::kOne2, F::kOne2, F::kOne2, F::kOne2};
    const uint32_t vm = vconst(F::kMask), vmagic = vconst(F::kMagic);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float sx[GW];  // sum of x over group g of this wave, column m = lane % 16
#pragma unroll
    for (int g = 0; g < GW; g++) {
        f32x4 d = {0.f, 0.f, 0.f, 0.f}, dx = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < Q::kMfma; t++) {
            const u4 xn = *reinterpret_cast<const u4*>(xrow + (size_t)g * GS * 2 + t * 16);
            d = mfma32<TX>(code_operand<BITS, TX>(&wv[g][t * F::kWordsPerMfma], vm, vmagic), x_operand<BITS, TX>(xn), d);
            dx = mfma32<TX>(ones, xn, dx);
        }
        sx[g] = dx[0];
        const int gg = part * GW + g;
#pragma unroll
        for (int r = 0; r < 4; r++) acc[r] = fmaf(sb_at<SB>(srow + (size_t)r * G * kSb, gg), d[r], acc[r]);
    }

    // ---- 4. offset and bias: acc[n][m] += sum_g (b / kPow - A0 s)[n][g] * sx[m][g] ----
    {
        const int k = lane >> 4;  // A[i][k] lane i + 16k; B[k][m] lane m + 16k
        const uint8_t* s_i = ls + (size_t)(16 * tile + i) * G * kSb;
        const uint8_t* b_i = lb + (size_t)(16 * tile + i) * G * kSb;
#pragma unroll
        for (int t = 0; t < GW / 4; t++) {
            const int gg = part * GW + 4 * t + k;
            const float a = fmaf(-F::kA0, sb_at<SB>(s_i, gg), sb_at<SB>(b_i, gg) * (1.f / F::kPow));
            const float bx = k == 0 ? sx[4 * t] : k == 1 ? sx[4 * t + 1] : k == 2 ? sx[4 * t + 2] : sx[4 * t + 3];
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, bx, acc, 0, 0, 0);
        }
    }

    // ---- 5. K-split partials meet in LDS; part 0 stores ----
    if (KS > 1) {
        if (part > 0) {
            float* p = lred + ((size_t)(tile * (KS - 1) + part - 1) * 64 + lane) * 4;
            *reinterpret_cast<f32x4*>(p) = acc;
        }
        __syncthreads();
        if (part == 0) {
            for (int q = 1; q < KS; q++) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(lred + ((size_t)(tile * (KS - 1) + q - 1) * 64 + lane) * 4);
                acc += v;
            }
        }
    }
    if (part == 0 && j < M) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int n = n_tile + 4 * c + r;
            if (n < N) store_out<EPI>(y, (size_t)j * N + n, n, ep, acc[r] * F::kPow);
        }
    }
}

}  // namespace skinny

// launcher (qmm_skinny.hip): NotSupported unless 2 <= M <= 16, bits 4 or 8,
// 16-bit x, and K splits into 4, 2 or 1 parts of 8, 16 or 32 groups
LuxStatus launch_qmm_skinny(const QmmArgs& a, hipStream_t st);

}  // namespace lxq
