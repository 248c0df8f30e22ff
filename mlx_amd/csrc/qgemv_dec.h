// qgemv_dec.h -- MFMA decode kernel for 2 <= M <= 8 rows of x, 4-bit codes,
// f16/bf16 activations, K % 1024 == 0 (gfx950).
//
// y[m, n] = sum_g s[n,g] * sum_{k in g} q[n,k] x[m,k] + b[n,g] * sum_{k in g} x[m,k]
//
// Work split: a block owns TILES 16-row tiles of W over the whole K; its
// K/KW waves (at most 8) split K, KW codes each, and their partial sums meet
// in LDS.  More tiles per block share each x operand (and the block's copy
// of x) among more MFMAs and give each wave independent MFMA chains.  Every wave issues all its loads first -- the scales and biases of its
// own row's groups, then per tile 8 weight loads of 128 bits per lane (W row
// n0 + lane % 16, lane group c = lane / 16 reading bytes 16c .. 16c+15 of
// each 64-byte quarter of a 256-code segment) -- and computes each segment
// as it lands.
//
// MFMA: v_mfma_f32_16x16x32 with A = x (row m = lane % 16; rows past M
// re-read row M-1 and are never stored) and B = the codes as exact operands
// v = 1 + q/kPow (DForm: the code in the top mantissa bits of 1.0), so lane (n, c) of the
// accumulator holds rows m = 4c .. 4c+3 of output column n: the lane's own W
// row, whose scales it holds in registers.  An MFMA must stay within one
// group; a 128-bit load gives lane group c codes 32c .. 32c+31 of a 128-code
// run, so the registers are regrouped across lane groups first:
//   group 128: none (the run is one group; register e is codes 32c + 8e);
//   group 64: v_permlane32_swap of registers (0,2) and (1,3): registers 0, 1
//     hold the first group, 2, 3 the second;
//   group 32: then v_permlane16_swap of (0,1) and (2,3): register e is group e.
// Per group: D = sum v x over the group's MFMAs (fresh accumulator), and
// acc += s D + (b/kPow - s) sx with sx = sum_{k in g} x from one MFMA of x
// against all-ones per 32 codes; y = kPow acc.  The x operands (LDS reads
// and their permutation into the code order) and sx are computed once per
// group and shared by the two tiles.
//
// x is copied into LDS by buffer->LDS DMA before the weight loads (rows of
// 2K + 16 bytes: the 16 rows an A-operand read touches fall in different bank
// groups), so the one vmcnt wait for it leaves every weight load in flight.
// With xw = 0 the block's waves copy x together and a barrier publishes it;
// with xw = 1 each wave copies only its own K part, and its vmcnt wait alone
// makes that part visible to it (no barrier: a wave need not wait for the
// others' copies).
#pragma once
#include "kernels.h"
#include "qcommon.h"
#include "qmm_skinny.h"

namespace lxq {
namespace dec {

using gemv::buf_rsrc;
using gemv::lds_ptr;
using skinny::f32x4;
using skinny::mfma32;
using skinny::u4;
using skinny::x_operand;

constexpr int kMaxM = 8;

// Code operand v = 1 + q/kPow, exact in T: the 4-bit code sits in the top
// mantissa bits of 1.0 (f16: bits 4..7, kPow = 64; bf16: bits 3..6,
// kPow = 16).  Per group sum v x = sx + sum q x / kPow, so
// s sum q x + b sx = kPow (s D + (b/kPow - s) sx).  Keeping the offset at 1
// keeps the cancellation of the sx terms within ~kPow/8 of the result.
template <int TX>
struct DForm {
    static constexpr float kPow = TX == DT_F16 ? 64.f : 16.f;
    static constexpr uint32_t kMagic = TX == DT_F16 ? 0x3C003C00u : 0x3F803F80u;  // 1.0 in both halves
    static constexpr uint32_t kMask = TX == DT_F16 ? 0x00F000F0u : 0x00780078u;
};

// B operand of one MFMA from one word of 8 codes c0..c7: f16 pairs
// (c0,c4) (c1,c5) (c2,c6) (c3,c7), i.e. x order x0 x4 x1 x5 x2 x6 x3 x7 (the
// order skinny::x_operand produces).  The mask and the magic sit in VGPRs so
// that the compiler emits v_and_or_b32 (and its own VALU -> MFMA waits).
template <int TX>
__device__ __forceinline__ u4 dec_code_operand(uint32_t w, uint32_t vm, uint32_t vmagic) {
    if constexpr (TX == DT_F16)
        return u4{((w << 4) & vm) | vmagic, (w & vm) | vmagic, ((w >> 4) & vm) | vmagic, ((w >> 8) & vm) | vmagic};
    else
        return u4{((w << 3) & vm) | vmagic, ((w >> 1) & vm) | vmagic, ((w >> 5) & vm) | vmagic,
                  ((w >> 9) & vm) | vmagic};
}

// code offset (within a 256-code segment) of the 8 codes lane group c holds
// in register e of load i (bytes 64 i .. 64 i + 63 of the segment) after the
// regrouping for group size GS
template <int GS>
__device__ __host__ constexpr int code_off(int i, int e, int c) {
    return GS == 128 ? 128 * i + 32 * c + 8 * e
         : GS == 64  ? 128 * i + 64 * (e >> 1) + (c < 2 ? 32 * c : 32 * (c - 2) + 16) + 8 * (e & 1)
                     : 128 * i + 32 * e + 8 * c;
}
// group (within the segment) of register e of load i
template <int GS>
__device__ __host__ constexpr int reg_group(int i, int e) {
    return GS == 128 ? i : GS == 64 ? 2 * i + (e >> 1) : 4 * i + e;
}

template <int GS>
__device__ __forceinline__ void regroup(u4& d) {
    if constexpr (GS <= 64) {
        const auto p = __builtin_amdgcn_permlane32_swap(d.x, d.z, false, false);
        const auto q = __builtin_amdgcn_permlane32_swap(d.y, d.w, false, false);
        d.x = p[0]; d.z = p[1];
        d.y = q[0]; d.w = q[1];
    }
    if constexpr (GS == 32) {
        const auto p = __builtin_amdgcn_permlane16_swap(d.x, d.y, false, false);
        const auto q = __builtin_amdgcn_permlane16_swap(d.z, d.w, false, false);
        d.x = p[0]; d.y = p[1];
        d.z = q[0]; d.w = q[1];
    }
}

__device__ __forceinline__ uint32_t u4_at(const u4& v, int e) { return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; }

// scale/bias of group g from a lane's register copy of its row's groups
template <int SB>
__device__ __forceinline__ float sb_reg(const uint32_t* r, int g) {
    if constexpr (SB == DT_F32) return __uint_as_float(r[g]);
    else if constexpr (SB == DT_F16) return f16_to_f32(g & 1 ? r[g >> 1] >> 16 : r[g >> 1] & 0xffffu);
    else return __uint_as_float(g & 1 ? r[g >> 1] & 0xffff0000u : r[g >> 1] << 16);
}

template <int GS, int SB, int KW>
struct DGeo {
    static constexpr int kSb = SB == DT_F32 ? 4 : 2;
    static constexpr int kGW = KW / GS;                  // groups per wave
    static constexpr int kSbWords = kGW * kSb / 4;       // scale dwords per row per wave
    static constexpr int kSbLoads = kSbWords / 4;        // 128-bit loads of them
    static constexpr bool kFits = kSbWords % 4 == 0;   // scale rows of a wave are whole 16-byte chunks
};

// a block shape the kernel takes: whole 16-byte scale chunks per wave, and
// every load of a wave (weights, scales, biases) countable by vmcnt
template <int GS, int SB, int TILES, int KW>
constexpr bool dec_ok() {
    using Q = DGeo<GS, SB, KW>;
    return Q::kFits && (KW / 256) * 2 * TILES + 2 * TILES * Q::kSbLoads < 64;
}

// LDS: the M rows of x, then the partial sums of waves 1.. for the K reduction
__host__ __device__ constexpr size_t dec_lds_bytes(int M, int K, int tiles, int kw) {
    return (size_t)M * (2 * K + 16) + (size_t)(K / kw - 1) * tiles * 4 * 64 * 4;
}

template <int TX, int SB, int GS, bool EPI, int TILES, int KW>
__global__ __launch_bounds__(512) void qgemv_dec_kernel(const void* __restrict__ x, const uint32_t* __restrict__ wq,
                                                        const void* __restrict__ scales,
                                                        const void* __restrict__ biases, void* __restrict__ y,
                                                        int M, int K, int N, int xw, Epilogue ep) {
    using F = DForm<TX>;
    using Q = DGeo<GS, SB, KW>;
    static_assert(dec_ok<GS, SB, TILES, KW>(), "block shape");
    constexpr int kTiles = TILES, kKW = KW, kSegs = KW / 256;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = blockDim.x >> 6;
    const int j = lane & 15, c = lane >> 4;
    const int n0 = blockIdx.x * 16 * kTiles;
    const int G = K / GS;
    const int XS = 2 * K + 16;  // x row stride in LDS
    float* const red = reinterpret_cast<float*>(lds + (size_t)M * XS);

    // ---- 1. x rows into LDS (DMA) ----
    {
        const auto xr = buf_rsrc(x, (uint32_t)M * K * 2);
        // 16-byte chunks of an x row: all K (a multiple of 64 chunks) shared by
        // the block's waves, or the wave's own KW codes (a multiple of 64 chunks)
        const int c_first = xw ? wave * (kKW / 8) : wave * 64;
        const int c_end = xw ? (wave + 1) * (kKW / 8) : K / 8;
        const int c_step = xw ? 64 : 64 * nwaves;
        for (int m = 0; m < M; m++)
            for (int c0 = c_first; c0 < c_end; c0 += c_step)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr)(lds + m * XS + c0 * 16), 16,
                                                         (uint32_t)(m * K * 2 + (c0 + lane) * 16), 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. this wave's scales and biases, then its weights (segment-major,
    // the order they are used); rows past N re-read row N-1 (never stored) ----
    u4 wv[kSegs][2][kTiles];
    uint32_t sr[kTiles][Q::kSbWords], br[kTiles][Q::kSbWords];
    {
        int nt[kTiles];
#pragma unroll
        for (int t = 0; t < kTiles; t++) nt[t] = n0 + 16 * t + j < N ? n0 + 16 * t + j : N - 1;
        const uint32_t sb_row = (uint32_t)G * Q::kSb;
        const auto srs = buf_rsrc(scales, (uint32_t)N * sb_row), brs = buf_rsrc(biases, (uint32_t)N * sb_row);
#pragma unroll
        for (int t = 0; t < kTiles; t++) {
            const uint32_t off = (uint32_t)nt[t] * sb_row + (uint32_t)wave * Q::kGW * Q::kSb;
#pragma unroll
            for (int q = 0; q < Q::kSbLoads; q++) {
                const u4 a = __builtin_amdgcn_raw_buffer_load_b128(srs, off + 16u * q, 0, 0);
                const u4 b = __builtin_amdgcn_raw_buffer_load_b128(brs, off + 16u * q, 0, 0);
                sr[t][4 * q] = a.x; sr[t][4 * q + 1] = a.y; sr[t][4 * q + 2] = a.z; sr[t][4 * q + 3] = a.w;
                br[t][4 * q] = b.x; br[t][4 * q + 1] = b.y; br[t][4 * q + 2] = b.z; br[t][4 * q + 3] = b.w;
            }
        }
        const uint32_t row_bytes = (uint32_t)K / 2;
        const auto wr = buf_rsrc(wq, (uint32_t)N * row_bytes);
#pragma unroll
        for (int s = 0; s < kSegs; s++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int t = 0; t < kTiles; t++)
                    wv[s][i][t] = __builtin_amdgcn_raw_buffer_load_b128(
                        wr, (uint32_t)nt[t] * row_bytes + (uint32_t)wave * (kKW / 2) + 16u * c + 128u * s + 64u * i,
                        0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // ---- 3. the x DMA was issued before the scale and weight loads: wait
    // for it alone, then (xw = 0) the barrier publishes every wave's part ----
    {
        constexpr int NW = kSegs * 2 * kTiles + 2 * kTiles * Q::kSbLoads;
        static_assert(NW < 64, "vmcnt holds 6 bits");
        __builtin_amdgcn_s_waitcnt((NW & 0xF) | ((NW >> 4) << 14) | (0x7 << 4) | (0xF << 8));
    }
    if (!xw) __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // ---- 4. segments in arrival order ----
    const int mr = j < M ? j : M - 1;  // A row m = lane % 16
    const uint8_t* xrow = lds + mr * XS + (size_t)wave * kKW * 2;
    const u4 ones = {F::kMagic, F::kMagic, F::kMagic, F::kMagic};  // 1.0 in every element
    const uint32_t vm = vconst(F::kMask), vmagic = vconst(F::kMagic);
    f32x4 acc[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    constexpr int kRegsPerGroup = GS == 128 ? 4 : GS == 64 ? 2 : 1;
#pragma unroll
    for (int s = 0; s < kSegs; s++) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            u4 d[kTiles];
#pragma unroll
            for (int t = 0; t < kTiles; t++) {
                d[t] = wv[s][i][t];
                regroup<GS>(d[t]);
            }
#pragma unroll
            for (int e0 = 0; e0 < 4; e0 += kRegsPerGroup) {
                f32x4 dg[kTiles], dx = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < kTiles; t++) dg[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int e = e0; e < e0 + kRegsPerGroup; e++) {
                    const u4 xn = *reinterpret_cast<const u4*>(xrow + 2 * (256 * s + code_off<GS>(i, e, c)));
                    const u4 xa = x_operand<4, TX>(xn);
#pragma unroll
                    for (int t = 0; t < kTiles; t++)
                        dg[t] = mfma32<TX>(xa, dec_code_operand<TX>(u4_at(d[t], e), vm, vmagic), dg[t]);
                    dx = mfma32<TX>(xn, ones, dx);
                }
                const int g = s * (256 / GS) + reg_group<GS>(i, e0);  // group within the wave
#pragma unroll
                for (int t = 0; t < kTiles; t++) {
                    const float sc = sb_reg<SB>(sr[t], g), bi = sb_reg<SB>(br[t], g);
                    const float cc = fmaf(-1.f, sc, bi * (1.f / F::kPow));
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[t][r] = fmaf(sc, dg[t][r], fmaf(cc, dx[r], acc[t][r]));
                }
            }
        }
    }

    // ---- 5. K parts meet in LDS; wave 0 stores ----
    if (nwaves > 1) {
        if (wave > 0) {
#pragma unroll
            for (int t = 0; t < kTiles; t++)
                *reinterpret_cast<f32x4*>(red + ((size_t)((wave - 1) * kTiles + t) * 64 + lane) * 4) = acc[t];
        }
        __syncthreads();
        if (wave == 0) {
            for (int w2 = 1; w2 < nwaves; w2++)
#pragma unroll
                for (int t = 0; t < kTiles; t++)
                    acc[t] += *reinterpret_cast<const f32x4*>(red + ((size_t)((w2 - 1) * kTiles + t) * 64 + lane) * 4);
        }
    }
    if (wave == 0) {
        // accumulator: lane (n = lane % 16, c) holds rows m = 4c .. 4c+3
#pragma unroll
        for (int t = 0; t < kTiles; t++) {
            const int n = n0 + 16 * t + j;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = 4 * c + r;
                if (m < M && n < N) store_out<EPI>(y, (size_t)m * N + n, n, ep, acc[t][r] * F::kPow);
            }
        }
    }
}

}  // namespace dec

// launcher (qgemv_dec.hip): NotSupported unless 2 <= M <= 8, 4-bit codes,
// f16/bf16 x, K % 1024 == 0 with K / 1024 <= 8 waves, the scale rows of a
// wave fit in registers (not f32 scales with group size 32), 32-bit offsets
LuxStatus launch_qgemv_dec(const QmmArgs& a, hipStream_t st);

}  // namespace lxq
