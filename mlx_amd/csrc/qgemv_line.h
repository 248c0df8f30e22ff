// qgemv_line.h -- one row of x (M == 1), K <= 4096: the dequant-GEMV that
// streams whole cache lines (gfx950).
//
// Included after qgemv_impl.h (it uses its buffer, operand and reduction
// helpers) by the per-bit-width translation units.
//
// A block is 4 waves, wave w owns R consecutive rows (R = 4, 6 or 7: see
// line_rows7 and line_rows_narrow below).  Every load is issued
// at the start, straight into registers:
//   0. with R = 7 and the wave's own x: the first row's codes (below), so
//      that the HBM stream is under way while steps 1-2 pass through the
//      CU's queue;
//   1. x: the lane's code chunks' x values (L2-resident after first touch),
//      or, for the widths and types where it measured faster, the block's
//      x once (16 bytes per thread), shared through LDS after the codes are
//      issued;
//   2. the wave's R scale rows and R bias rows, as whole 16-byte chunks;
//   3. a block barrier, so that the x and scale requests of all four waves
//      enter the CU's vector-memory queue ahead of every other code request;
//   4. the codes: for each row, NI wave loads of SPAN contiguous bytes (lane
//      l takes the l-th 16- or 12-byte chunk, 4*WPI bytes = NC codes), with
//      the non-temporal cache policy.  Each wave instruction covers whole
//      128-byte lines, so a line is requested once and not kept in L2.
// The scale rows go through a per-wave LDS area (written by the wave itself,
// no barrier) so that each lane reads the scale of its own chunk.  Rows are
// then computed in arrival order (the compiler's in-order vmcnt waits), so
// the arithmetic of early rows overlaps the stream of later ones, and the R
// row sums are reduced together with permlane swaps and DPP.
//
// Measured against the variants this replaced (same box, c1 M = 1):
// x staged per block in LDS behind a barrier left the block waiting for its
// slowest wave's x (an L2 hit queued behind every CU's code misses; +0.3 to
// +1.2 us); scales as 2-byte loads per (row, chunk) cost +0.3 us of load
// issue; LDS-DMA of the scale rows followed by a partial vmcnt wait read
// stale LDS now and then (an LDS-DMA write is not ordered with the register
// loads issued after it), so every load here returns into registers.
//
// Chunk widths: 2/4/8-bit codes 16 bytes (64/32/16 codes), 3/6-bit codes 12
// bytes (32/16 codes: one 3-word period), so a chunk never splits a code and,
// for group sizes >= 32, lies in one group (2-bit codes with group size 32:
// two groups, TWO).  5-bit codes stay on the stream kernel.
#pragma once
#include "qgemv_impl.h"

namespace lxq {
namespace gemv {

template <int BITS>
struct LineCfg {
    static constexpr bool kOk = BITS == 2 || BITS == 3 || BITS == 4 || BITS == 6 || BITS == 8;
    static constexpr int WPI = (BITS == 3 || BITS == 6) ? 3 : 4;  // words per lane per wave load
    static constexpr int NC = 32 * WPI / BITS;                     // codes per chunk
    static constexpr int SPAN = 64 * 4 * WPI;                      // bytes per wave load
    // wave loads per row at K = 4096
    static constexpr int kMaxNI = (4096 * BITS / 8 + SPAN - 1) / SPAN;
};

typedef uint32_t v3u32 __attribute__((ext_vector_type(3)));

// Operand form of the whole-line kernel: op_kind's, except 3- and 6-bit
// codes with f16 x, which take the subnormal form too (OP_SUB3 / OP_SUB6,
// line_partial): about 1.4 / 2 VALU per code against 2.7 for the
// magic-number pairs.
template <int BITS, int TX>
constexpr int line_op() {
    return (BITS == 3 && TX == DT_F16) ? OP_SUB3 : (BITS == 6 && TX == DT_F16) ? OP_SUB6 : op_kind<BITS, TX>();
}
constexpr int kCachePolicyNT = 2;  // buffer-load cache policy bit: non-temporal

// x operands of one chunk of NC_ codes (default: the whole-line chunk)
template <int BITS, int TX, int OP, int NC_ = LineCfg<BITS>::NC>
struct LineX {
    static constexpr int NC = NC_;
    static constexpr int kRegs = OP == OP_F32 ? NC : NC / 2;
    uint32_t v[kRegs];
    float h0, h1;  // sums of x over the chunk's two halves (times 2^-24 for the subnormal forms)
};

// nat: the chunk's x values in natural order (NC elements)
template <int BITS, int TX, int OP, int NC_ = LineCfg<BITS>::NC>
__device__ __forceinline__ void prep_line_x(const uint32_t* nat, LineX<BITS, TX, OP, NC_>& o) {
    constexpr int NC = NC_;
    if constexpr (OP == OP_F32) {
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int i = 0; i < NC; i++) {
            o.v[i] = nat[i];
            if (i < NC / 2) a += __uint_as_float(nat[i]);
            else b += __uint_as_float(nat[i]);
        }
        o.h0 = a;
        o.h1 = b;
    } else {
        constexpr int NW = NC / 2;  // 32-bit words of x
        const uint32_t one2 = TX == DT_F16 ? 0x3C003C00u : 0x3F803F80u;
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int i = 0; i < NW; i++) {
            if (i < NW / 2) a = dot2(nat[i], one2, a, TX);
            else b = dot2(nat[i], one2, b, TX);
        }
        if constexpr (OP == OP_SUB4 || OP == OP_SUB3) {
            // code word (4-bit) or 24-bit group (3-bit) j covers x[8j..8j+7] =
            // nat[4j..4j+3]; operand pairs (x0,x4) (x1,x5) (x2,x6) (x3,x7)
            // [4-bit: mask 0xF, mask 0xF0, >>8 then the same]
#pragma unroll
            for (int j = 0; j < NC / 8; j++) {
                o.v[4 * j]     = __builtin_amdgcn_perm(nat[4 * j + 2], nat[4 * j], 0x05040100u);
                o.v[4 * j + 1] = __builtin_amdgcn_perm(nat[4 * j + 2], nat[4 * j], 0x07060302u);
                o.v[4 * j + 2] = __builtin_amdgcn_perm(nat[4 * j + 3], nat[4 * j + 1], 0x05040100u);
                o.v[4 * j + 3] = __builtin_amdgcn_perm(nat[4 * j + 3], nat[4 * j + 1], 0x07060302u);
            }
            a *= 0x1p-24f;
            b *= 0x1p-24f;
        } else if constexpr (OP == OP_SUB8 || OP == OP_SUB6) {
            // code word (8-bit) or 24-bit group (6-bit) j covers x[4j..4j+3] =
            // nat[2j], nat[2j+1]: (x0,x2) (x1,x3)
#pragma unroll
            for (int j = 0; j < NC / 4; j++) {
                o.v[2 * j]     = __builtin_amdgcn_perm(nat[2 * j + 1], nat[2 * j], 0x05040100u);
                o.v[2 * j + 1] = __builtin_amdgcn_perm(nat[2 * j + 1], nat[2 * j], 0x07060302u);
            }
            a *= 0x1p-24f;
            b *= 0x1p-24f;
        } else if constexpr (OP == OP_MAGIC && PairLayout<BITS>::kApart) {
            // a code word holds P codes; pair j = (x_j, x_{j+P/2})
            constexpr int P = PairLayout<BITS>::kCodesPerWord, D = P / 2;
#pragma unroll
            for (int blk = 0; blk < NC / P; blk++) {
#pragma unroll
                for (int j = 0; j < D; j++) {
                    const int e0 = j, e1 = j + D;
                    const uint32_t w0 = nat[blk * D + e0 / 2], w1 = nat[blk * D + e1 / 2];
                    const uint32_t lo = (e0 & 1) ? (w0 >> 16) : (w0 & 0xffffu);
                    const uint32_t hi = (e1 & 1) ? (w1 & 0xffff0000u) : (w1 << 16);
                    o.v[blk * D + j] = lo | hi;
                }
            }
        } else {
            // natural pairs (x_{2p}, x_{2p+1})
#pragma unroll
            for (int i = 0; i < NW; i++) o.v[i] = nat[i];
        }
        o.h0 = a;
        o.h1 = b;
    }
}

// partial of one chunk for one row.  TWO: s0/b0 cover the chunk's first half
// and s1/b1 its second (2-bit codes, group size 32); otherwise s1/b1 unused.
// w: the chunk's NC_ * BITS / 32 code words.
template <int BITS, int TX, int OP, bool TWO, int NC_ = LineCfg<BITS>::NC>
__device__ __forceinline__ float line_partial(const uint32_t* w, const LineX<BITS, TX, OP, NC_>& xo, float s0, float b0,
                                              float s1, float b1) {
    constexpr int NC = NC_, WPI = NC_ * BITS / 32;
    if constexpr (OP == OP_SUB4) {
        float a = 0.f, c = 0.f;
#pragma unroll
        for (int j = 0; j < WPI; j++) {
            const uint32_t wj = w[j], w8 = wj >> 8;
            a = dot2(xo.v[4 * j], wj & 0x000F000Fu, a, DT_F16);
            c = dot2(xo.v[4 * j + 1], wj & 0x00F000F0u, c, DT_F16);
            a = dot2(xo.v[4 * j + 2], w8 & 0x000F000Fu, a, DT_F16);
            c = dot2(xo.v[4 * j + 3], w8 & 0x00F000F0u, c, DT_F16);
        }
        return fmaf(s0, fmaf(c, 0.0625f, a), b0 * (xo.h0 + xo.h1));
    } else if constexpr (OP == OP_SUB3) {
        // The chunk's 96 bits as four 24-bit groups of 8 codes.  Per group,
        // t keeps codes 0..3 in its low half at bits 0, 3, 6, 9 and moves
        // codes 4..7 to the same places of its high half; a mask then leaves
        // one pair (code j, code 4 + j) as two f16 subnormals q 2^(p-24) at
        // bit p = 0, 3, 6 (pair 3, at bit 9, is shifted down to 0 first: a
        // code above bit 7 would reach the exponent field).  One accumulator
        // per position, combined as a0 + a3 / 8 + a6 / 64.
        static_assert(WPI == 3 && NC == 32, "3-bit chunks");
        const uint32_t g[4] = {w[0], __builtin_amdgcn_alignbit(w[1], w[0], 24),
                               __builtin_amdgcn_alignbit(w[2], w[1], 16), w[2] >> 8};
        float a0 = 0.f, a3 = 0.f, a6 = 0.f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t t = (g[q] & 0x0000FFFFu) | ((g[q] << 4) & 0xFFFF0000u);
            a0 = dot2(xo.v[4 * q], t & 0x00070007u, a0, DT_F16);
            a3 = dot2(xo.v[4 * q + 1], t & 0x00380038u, a3, DT_F16);
            a6 = dot2(xo.v[4 * q + 2], t & 0x01C001C0u, a6, DT_F16);
            a0 = dot2(xo.v[4 * q + 3], (t >> 9) & 0x00070007u, a0, DT_F16);
        }
        return fmaf(s0, fmaf(a6, 0.015625f, fmaf(a3, 0.125f, a0)), b0 * (xo.h0 + xo.h1));
    } else if constexpr (OP == OP_SUB6) {
        // Four 24-bit groups of 4 codes; t as for 3-bit codes (codes 0, 1 in
        // the low half at bits 0, 6; codes 2, 3 at the same places of the
        // high half).  Pair (0, 2) by a mask, pair (1, 3) shifted down to
        // bit 0 first: both f16 subnormals q 2^-24, one accumulator.
        static_assert(WPI == 3 && NC == 16, "6-bit chunks");
        const uint32_t g[4] = {w[0], __builtin_amdgcn_alignbit(w[1], w[0], 24),
                               __builtin_amdgcn_alignbit(w[2], w[1], 16), w[2] >> 8};
        float d = 0.f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t t = (g[q] & 0x0000FFFFu) | ((g[q] << 4) & 0xFFFF0000u);
            d = dot2(xo.v[2 * q], t & 0x003F003Fu, d, DT_F16);
            d = dot2(xo.v[2 * q + 1], (t >> 6) & 0x003F003Fu, d, DT_F16);
        }
        return fmaf(s0, d, b0 * (xo.h0 + xo.h1));
    } else if constexpr (OP == OP_SUB8) {
        float d = 0.f;
#pragma unroll
        for (int j = 0; j < WPI; j++) {
            const uint32_t wj = w[j], w8 = wj >> 8;
            d = dot2(xo.v[2 * j], wj & 0x00FF00FFu, d, DT_F16);
            d = dot2(xo.v[2 * j + 1], w8 & 0x00FF00FFu, d, DT_F16);
        }
        return fmaf(s0, d, b0 * (xo.h0 + xo.h1));
    } else if constexpr (OP == OP_F32) {
        float d0 = 0.f, d1 = 0.f;
        if constexpr (BITS == 4) {
            // nibble planes: code 2e of a word is byte e of lo, code 2e + 1
            // byte e of hi, each one v_cvt_f32_ubyte{e} (the asm keeps the
            // compiler from folding the masks back into an extract per
            // code); same codes, same FMA order as the generic form
#pragma unroll
            for (int j = 0; j < WPI; j++) {
                uint32_t lo = w[j] & 0x0F0F0F0Fu, hi = (w[j] >> 4) & 0x0F0F0F0Fu;
                asm("" : "+v"(lo), "+v"(hi));
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int i = 8 * j + 2 * e;
                    float& d = i < NC / 2 ? d0 : d1;
                    d = fmaf(__uint_as_float(xo.v[i]), (float)((lo >> (8 * e)) & 0xffu), d);
                    d = fmaf(__uint_as_float(xo.v[i + 1]), (float)((hi >> (8 * e)) & 0xffu), d);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < NC / 2; i++) d0 = fmaf(__uint_as_float(xo.v[i]), (float)unit_code<BITS>(w, i), d0);
#pragma unroll
            for (int i = NC / 2; i < NC; i++) d1 = fmaf(__uint_as_float(xo.v[i]), (float)unit_code<BITS>(w, i), d1);
        }
        if constexpr (TWO) return (s0 * d0 + b0 * xo.h0) + (s1 * d1 + b1 * xo.h1);
        else return s0 * (d0 + d1) + b0 * (xo.h0 + xo.h1);
    } else {
        constexpr int NP = NC / 2;
        uint32_t pr[NP];
        if constexpr (OP == OP_MAGIC)
            unit_pairs_magic<BITS, (TX == DT_F16 ? 10 : 7), WPI>(w, pr);
        else
            unit_pairs_bf16_u8<WPI>(w, pr);
        // pairs of the first NP/2 lie in the chunk's first half (pairs stay
        // inside one code word in the apart layout)
        float d0 = 0.f, d1 = 0.f;
#pragma unroll
        for (int i = 0; i < NP / 2; i++) d0 = dot2(xo.v[i], pr[i], d0, TX);
#pragma unroll
        for (int i = NP / 2; i < NP; i++) d1 = dot2(xo.v[i], pr[i], d1, TX);
        if constexpr (OP == OP_MAGIC) {
            // D = sum x v(q) = h + sum x q / kPow  =>  s sum x q + b h = (s kPow) D + (b - s kPow) h
            constexpr float kPow = MagicCfg<BITS, (TX == DT_F16 ? 10 : 7)>::kPow;
            if constexpr (TWO)
                return ((s0 * kPow) * d0 + fmaf(-s0, kPow, b0) * xo.h0) +
                       ((s1 * kPow) * d1 + fmaf(-s1, kPow, b1) * xo.h1);
            else
                return (s0 * kPow) * (d0 + d1) + fmaf(-s0, kPow, b0) * (xo.h0 + xo.h1);
        } else {
            if constexpr (TWO) return (s0 * d0 + b0 * xo.h0) + (s1 * d1 + b1 * xo.h1);
            else return s0 * (d0 + d1) + b0 * (xo.h0 + xo.h1);
        }
    }
}

// Four 64-lane sums at once; afterwards lanes with (lane & 15) == 0 hold the
// sum of v[sum4_index(lane)].
__device__ __forceinline__ float sum4(const float* v) {
    const float w0 = swap32_sum(v[0], v[1]), w1 = swap32_sum(v[2], v[3]);
    float z = swap16_sum(w0, w1);  // 16-lane rows: v0 v2 v1 v3
    z += dpp_f<0x128>(z);          // row_ror:8
    z += dpp_f<0xB1>(z);           // quad_perm [1,0,3,2]
    z += dpp_f<0x4E>(z);           // quad_perm [2,3,0,1]
    z += dpp_f<0x141>(z);          // row_half_mirror
    return z;
}
__device__ __host__ __forceinline__ int sum4_index(int lane) {
    const int row = lane >> 4;
    return ((row & 1) << 1) | (row >> 1);
}

template <int SB>
__device__ __forceinline__ float sb_value(uint32_t raw) {
    if constexpr (SB == DT_F32) return __uint_as_float(raw);
    else if constexpr (SB == DT_F16) return f16_to_f32(raw & 0xffffu);
    else return bf16_to_f32(raw & 0xffffu);
}

// SBQ: 128-bit loads per lane (1, 2 or 4) that cover a wave's R scale rows
// plus the lead of the first row within its 16-byte chunk (line_sb_loads)
template <int BITS, int TX, int SB, int R, int NI, bool TWO, bool EPI, int SBQ>
__global__ __launch_bounds__(256) void qgemv_line_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int K, int N, int gshift, Epilogue ep) {
    using C = LineCfg<BITS>;
    constexpr int OP = line_op<BITS, TX>();
    constexpr int XE = TX == DT_F32 ? 4 : 2;
    constexpr int kSb = SB == DT_F32 ? 4 : 2;
    constexpr int NC = C::NC, WPI = C::WPI;
    constexpr int XW = NC * XE / 4;  // 32-bit words of x per chunk
    constexpr int NT = TWO ? 2 : 1;  // groups per chunk
    static_assert(R == 4 || R == 6 || R == 7, "rows per wave");
    static_assert(NI * 64 * NC <= 4096, "the lanes' chunks lie in the block's copy of x");
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    const uint32_t sb_row = (uint32_t)(K >> gshift) * kSb;
    const int nb0 = blockIdx.x * (4 * R);
    const int n0 = nb0 + wave * R;

    // lane chunk c = i * 64 + lane covers codes [c NC, c NC + NC); chunks past
    // K read zeros (codes, x and scales), so their partials are 0
    bool ok[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) ok[i] = (uint32_t)(i * 64 + lane) * NC < (uint32_t)K;

    // row r's codes: whole lines, non-temporal (rows past N re-read row
    // N - 1, never stored)
    constexpr bool XSH = !(BITS == 4 && TX != DT_F32);
    uint32_t w[R][NI][WPI];
    auto row_loads = [&](int r) {
        // the block's rows (the compiler computes this once, where the
        // first row's loads are issued)
        const size_t wleft = (size_t)(N - nb0) * row_bytes;
        const auto wr = buf_rsrc(reinterpret_cast<const uint8_t*>(wq) + (size_t)nb0 * row_bytes,
                                 (uint32_t)(wleft < 0x7fffffffu ? wleft : 0x7fffffffu));
        const int n = n0 + r < N ? n0 + r : N - 1;
        const uint32_t soff = (uint32_t)(n - nb0) * row_bytes;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const uint32_t voff = ok[i] ? (uint32_t)(i * C::SPAN + lane * 4 * WPI) : kZeroOff;
            if constexpr (WPI == 4) {
                const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(wr, voff, soff, kCachePolicyNT);
                w[r][i][0] = v.x; w[r][i][1] = v.y; w[r][i][2] = v.z; w[r][i][3] = v.w;
            } else {
                const v3u32 v = __builtin_amdgcn_raw_buffer_load_b96(wr, voff, soff, kCachePolicyNT);
                w[r][i][0] = v.x; w[r][i][1] = v.y; w[r][i][2] = v.z;
            }
        }
        // issue the rows in order: loads return in issue order and the
        // rows are computed in this order (left free, the scheduler
        // interleaved the rows' loads, and the first rows' arithmetic then
        // waited for most of the stream: 7.9 against 7.5 us at c1)
        __builtin_amdgcn_sched_barrier(0);
    };
    // ---- 0. 7-row waves that load their own x: the first row's codes go
    // out ahead of x and the scale rows, so the HBM stream has begun while
    // those pass through the CU's queue.  Measured (same box, back-to-back
    // launches, µs): c1 7.29 -> 7.14 (f16 x), 7.62 -> 7.39 (bf16 x); the
    // first two rows 7.16; only the row's first 1 KB 7.34; the scale rows
    // also ahead of x 7.42; no block barrier 7.70.  With 4-row waves (N =
    // 4096, 11008) or x shared through LDS (c0, c4 3/6-bit) it was 0.16-0.63
    // slower, so they keep x first. ----
    constexpr bool kEarlyRow = !XSH && R == 7;
    if constexpr (kEarlyRow) row_loads(0);
    __builtin_amdgcn_sched_barrier(0);

    // ---- 1. x.  XSH: once per block, thread t loading 16-byte chunks t,
    // t + 256, ... of the 4096 codes' x (past K: zeros), shared through LDS
    // (step 6); else each wave loads its lanes' chunks.  Measured (same box,
    // stream launches, µs): shared x 4.80 against 5.21 at configs[0] (f32
    // x), 6.95 against 7.12 at 2-bit, 8.90 against 9.09 at 6-bit, level at
    // 3- and 8-bit, but 7.67 against 7.37-7.54 at configs[1] (4-bit, f16 x),
    // where the block barrier before the x reads costs more than the queue
    // time of the per-wave copies. ----
    constexpr int kXQ = XSH ? 4096 * XE / 4096 : 1;  // 16-byte chunks per thread
    const int tid = threadIdx.x;
    uint32_t xq[kXQ][4];
    uint32_t xw[XSH ? 1 : NI][XW];
    {
        const auto xr = buf_rsrc(x, (uint32_t)K * XE);
        if constexpr (XSH) {
#pragma unroll
            for (int q = 0; q < kXQ; q++) {
                const uint32_t c = (uint32_t)(q * 256 + tid);
                const uint32_t off = c * 16u < (uint32_t)K * XE ? c * 16u : kZeroOff;
                const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
                xq[q][0] = v.x; xq[q][1] = v.y; xq[q][2] = v.z; xq[q][3] = v.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const uint32_t off = ok[i] ? (uint32_t)(i * 64 + lane) * NC * XE : kZeroOff;
#pragma unroll
                for (int j = 0; j < XW / 4; j++) {
                    const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16 * j, 0, 0);
                    xw[i][4 * j] = v.x; xw[i][4 * j + 1] = v.y; xw[i][4 * j + 2] = v.z; xw[i][4 * j + 3] = v.w;
                }
            }
        }
    }
    // ---- 2. the wave's R scale rows and R bias rows (R * sb_row bytes
    // each, from the 16-byte chunk holding the first), 16 bytes per lane ----
    constexpr int kSbQ = SBQ;  // 128-bit loads per array
    uint32_t sraw[kSbQ][4], braw[kSbQ][4];
    uint32_t s_lead;
    {
        const size_t sb_first = (size_t)n0 * sb_row;
        s_lead = (uint32_t)(sb_first & 15u);
        const size_t sb_base = sb_first - s_lead;
        const size_t stotal = (size_t)N * sb_row;
        // rows past N read zeros (never stored); the last chunk may run into
        // the buffer's tail slack (kTailPad)
        const size_t sleft = sb_base < stotal ? ((stotal - sb_base + 15u) & ~(size_t)15u) : 0;
        const uint32_t sbytes = (uint32_t)(sleft < 0x7fffffffu ? sleft : 0x7fffffffu);
        const auto sr = buf_rsrc(static_cast<const uint8_t*>(scales) + sb_base, sbytes);
        const auto br = buf_rsrc(static_cast<const uint8_t*>(biases) + sb_base, sbytes);
        const uint32_t nch = (s_lead + (uint32_t)R * sb_row + 15u) >> 4;  // chunks of the wave's rows
#pragma unroll
        for (int q = 0; q < kSbQ; q++) {
            const uint32_t c = (uint32_t)(q * 64 + lane);
            const uint32_t off = c < nch ? c * 16u : kZeroOff;
            const v4u32 a = __builtin_amdgcn_raw_buffer_load_b128(sr, off, 0, 0);
            const v4u32 b = __builtin_amdgcn_raw_buffer_load_b128(br, off, 0, 0);
            sraw[q][0] = a.x; sraw[q][1] = a.y; sraw[q][2] = a.z; sraw[q][3] = a.w;
            braw[q][0] = b.x; braw[q][1] = b.y; braw[q][2] = b.z; braw[q][3] = b.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // ---- 3. every wave's x and scale requests ahead of its (other) code
    // requests ----
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // ---- 4. the (other) rows' codes ----
#pragma unroll
    for (int r = kEarlyRow ? 1 : 0; r < R; r++) row_loads(r);
    __builtin_amdgcn_sched_barrier(0);

    // ---- 5. the scale rows into the wave's LDS area (every lane writes,
    // so no lane-dependent use can pull the loads past the codes), then
    // each lane's scale and bias of every (row, chunk) ----
    __shared__ __attribute__((aligned(16))) uint8_t lsb[4][2][kSbQ * 1024];
    {
        uint8_t* ls = lsb[wave][0];
        uint8_t* lb = lsb[wave][1];
#pragma unroll
        for (int q = 0; q < kSbQ; q++) {
            *reinterpret_cast<v4u32*>(ls + (q * 64 + lane) * 16) = v4u32{sraw[q][0], sraw[q][1], sraw[q][2], sraw[q][3]};
            *reinterpret_cast<v4u32*>(lb + (q * 64 + lane) * 16) = v4u32{braw[q][0], braw[q][1], braw[q][2], braw[q][3]};
        }
    }
    float sc[R][NI][NT], bi[R][NI][NT];
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
#pragma unroll
            for (int t = 0; t < NT; t++) {
                // chunks past K: group 0 of the row, times zero codes and x
                const uint32_t g = ok[i] ? ((uint32_t)(i * 64 + lane) * NC + t * (NC / 2)) >> gshift : 0u;
                const uint32_t off = s_lead + (uint32_t)r * sb_row + g * kSb;
                if constexpr (SB == DT_F32) {
                    sc[r][i][t] = *reinterpret_cast<const float*>(lsb[wave][0] + off);
                    bi[r][i][t] = *reinterpret_cast<const float*>(lsb[wave][1] + off);
                } else {
                    sc[r][i][t] = sb_value<SB>(*reinterpret_cast<const uint16_t*>(lsb[wave][0] + off));
                    bi[r][i][t] = sb_value<SB>(*reinterpret_cast<const uint16_t*>(lsb[wave][1] + off));
                }
            }
        }
    }

    // ---- 6. x operands.  XSH: x into the block's LDS copy (the first
    // loads to land: the wait leaves the codes in flight), a barrier, then
    // each lane's chunks (chunks past K hold zeros: their partials are
    // exactly 0); else the wave's own loads ----
    LineX<BITS, TX, OP> xo[NI];
    if constexpr (XSH) {
        __shared__ __attribute__((aligned(16))) uint8_t lx[4096 * XE];
#pragma unroll
        for (int q = 0; q < kXQ; q++)
            *reinterpret_cast<v4u32*>(lx + (q * 256 + tid) * 16) = v4u32{xq[q][0], xq[q][1], xq[q][2], xq[q][3]};
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NI; i++) {
            uint32_t xn[XW];
            const uint8_t* src = lx + (i * 64 + lane) * NC * XE;
#pragma unroll
            for (int j = 0; j < XW / 4; j++) {
                const v4u32 v = *reinterpret_cast<const v4u32*>(src + 16 * j);
                xn[4 * j] = v.x; xn[4 * j + 1] = v.y; xn[4 * j + 2] = v.z; xn[4 * j + 3] = v.w;
            }
            prep_line_x<BITS, TX, OP>(xn, xo[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NI; i++) prep_line_x<BITS, TX, OP>(xw[i], xo[i]);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 7. rows in arrival order ----
    constexpr int RP = R <= 4 ? 4 : 8;
    float acc[RP];
#pragma unroll
    for (int r = 0; r < RP; r++) acc[r] = 0.f;
#pragma unroll
    for (int r = 0; r < R; r++) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            // chunks past K hold zero codes and x: their partial is exactly 0
            const float s0 = ok[i] ? sc[r][i][0] : 0.f, b0 = ok[i] ? bi[r][i][0] : 0.f;
            const float s1 = ok[i] ? sc[r][i][NT - 1] : 0.f, b1 = ok[i] ? bi[r][i][NT - 1] : 0.f;
            a += line_partial<BITS, TX, OP, TWO>(w[r][i], xo[i], s0, b0, s1, b1);
        }
        acc[r] = a;
        // rows in arrival order, one at a time
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- 8. reduce the R row sums together; one lane per row stores ----
    if constexpr (RP == 8) {
        const float z = sum8(acc, lane) * out_scale<OP>();
        const int r = sum8_index(lane);
        if ((lane & 7) == 0 && r < R && n0 + r < N) store_out<EPI>(y, (size_t)n0 + r, n0 + r, ep, z);
    } else {
        const float z = sum4(acc) * out_scale<OP>();
        const int r = sum4_index(lane);
        if ((lane & 15) == 0 && n0 + r < N) store_out<EPI>(y, (size_t)n0 + r, n0 + r, ep, z);
    }
}

// 128-bit loads per lane that cover R scale rows of G groups plus the lead
// of the first row within its 16-byte chunk
inline int line_sb_loads(int R, int G, int sb_dtype) {
    const int q = (R * G * (sb_dtype == DT_F32 ? 4 : 2) + 15 + 1023) / 1024;
    return q <= 1 ? 1 : q <= 2 ? 2 : 4;
}

template <int BITS, int TX, int SB, int R, int NI, bool TWO, int SBQ>
LuxStatus launch_line_k(const QmmArgs& a, hipStream_t st) {
    if (planned(a, "qgemv_line_kernel")) return LuxStatus::Ok;
    const int gshift = a.group_size == 32 ? 5 : a.group_size == 64 ? 6 : 7;
    const int blocks = (a.N + 4 * R - 1) / (4 * R);
    if (a.has_epilogue())
        hipLaunchKernelGGL((qgemv_line_kernel<BITS, TX, SB, R, NI, TWO, true, SBQ>), dim3(blocks), dim3(256), 0, st,
                           a.x, a.wq, a.scales, a.biases, a.y, a.K, a.N, gshift, a.epi());
    else
        hipLaunchKernelGGL((qgemv_line_kernel<BITS, TX, SB, R, NI, TWO, false, SBQ>), dim3(blocks), dim3(256), 0, st,
                           a.x, a.wq, a.scales, a.biases, a.y, a.K, a.N, gshift, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

// Rows per wave: 7 where that spreads the blocks over the 256 CUs more
// evenly than 4 (c1, N = 14336: 512 blocks, 2 per CU, against 896 = 3.5 per
// CU; measured 7.03 against 7.27 us), else 4.
inline bool line_rows7(int N) {
    auto balance = [](int blocks) {
        const int rounds = (blocks + 255) / 256;
        return (double)blocks / (256.0 * rounds);
    };
    return balance((N + 27) / 28) > balance((N + 15) / 16) + 0.05;
}

template <int BITS, int TX, int SB, int NI, bool TWO, int R>
LuxStatus launch_line_q(const QmmArgs& a, hipStream_t st) {
    switch (line_sb_loads(R, a.K / a.group_size, SB)) {
    case 1: return launch_line_k<BITS, TX, SB, R, NI, TWO, 1>(a, st);
    case 2: return launch_line_k<BITS, TX, SB, R, NI, TWO, 2>(a, st);
    default: return launch_line_k<BITS, TX, SB, R, NI, TWO, 4>(a, st);
    }
}

// Rows per wave for 2- to 4-bit codes with 16-bit x: of R = 7, 6, 4 the one
// whose busiest CU holds the fewest rows (ceil(blocks / 256) blocks of 4R
// rows), the larger R on a tie.  Measured against the rule above (same box,
// bit-identical outputs, µs per launch, K = 4096 unless noted): N = 11008
// 3-bit 6.29 -> 6.18 (R 6 against 4), 4-bit 6.31 -> 6.24, 2-bit 5.82 ->
// 5.63, K = 2048 4.36 -> 4.23; N = 12288 4-bit 6.70 -> 6.54; N = 5120
// 4-bit 4.35 -> 4.02, 3-bit 4.59 -> 4.10 (R 6 against 7).  Over the whole
// R = 2..8 range at N = 11008 the time followed the busiest CU's rows (48
// rows 6.2-6.8 us, 60 rows 7.2, 64 rows 7.6), fewer blocks winning a tie.
// 6- and 8-bit codes were slower with R = 6 (8.45 -> 9.25, 9.43 -> 9.64)
// and keep the rule above, as does f32 x (not measured).
inline int line_rows_narrow(int N) {
    int best = 4, best_rows = 1 << 30;
    for (int R : {7, 6, 4}) {
        const int blocks = (N + 4 * R - 1) / (4 * R);
        const int rows = (blocks + 255) / 256 * 4 * R;
        if (rows < best_rows) best = R, best_rows = rows;
    }
    return best;
}

template <int BITS, int TX, int SB, int NI, bool TWO>
LuxStatus launch_line_r(const QmmArgs& a, hipStream_t st) {
    if constexpr (BITS <= 4 && TX != DT_F32) {
        switch (line_rows_narrow(a.N)) {
        case 7: return launch_line_q<BITS, TX, SB, NI, TWO, 7>(a, st);
        case 6: return launch_line_q<BITS, TX, SB, NI, TWO, 6>(a, st);
        default: return launch_line_q<BITS, TX, SB, NI, TWO, 4>(a, st);
        }
    }
    if (line_rows7(a.N)) return launch_line_q<BITS, TX, SB, NI, TWO, 7>(a, st);
    return launch_line_q<BITS, TX, SB, NI, TWO, 4>(a, st);
}

template <int BITS, int TX, int SB, int NI>
LuxStatus launch_line_ni(const QmmArgs& a, hipStream_t st) {
    if constexpr (BITS == 2) {
        // a 64-code chunk covers two groups of 32
        if (a.group_size == 32) return launch_line_r<BITS, TX, SB, NI, true>(a, st);
    }
    return launch_line_r<BITS, TX, SB, NI, false>(a, st);
}

template <int BITS, int TX, int SB>
LuxStatus launch_line_sb(const QmmArgs& a, hipStream_t st) {
    using C = LineCfg<BITS>;
    const int ni = (int)(((size_t)a.K * BITS / 8 + C::SPAN - 1) / C::SPAN);
    if (ni <= 1) return launch_line_ni<BITS, TX, SB, 1>(a, st);
    if constexpr (C::kMaxNI >= 2) {
        if (ni == 2) return launch_line_ni<BITS, TX, SB, 2>(a, st);
    }
    if constexpr (C::kMaxNI >= 4) {
        if (ni <= 4) return launch_line_ni<BITS, TX, SB, 4>(a, st);
    }
    return LuxStatus::NotSupported;
}

// M == 1, K <= 4096 (K % 64 == 0), 2/3/4/6/8-bit codes; NotSupported otherwise
template <int BITS, int TX>
LuxStatus launch_line(const QmmArgs& a, hipStream_t st) {
    if constexpr (!LineCfg<BITS>::kOk) {
        return LuxStatus::NotSupported;
    } else {
        if (a.M != 1 || a.K > 4096 || a.K % 64 != 0) return LuxStatus::NotSupported;
        switch (a.sb_dtype) {
        case DT_F32: return launch_line_sb<BITS, TX, DT_F32>(a, st);
        case DT_F16: return launch_line_sb<BITS, TX, DT_F16>(a, st);
        default: return launch_line_sb<BITS, TX, DT_BF16>(a, st);
        }
    }
}

}  // namespace gemv
}  // namespace lxq
