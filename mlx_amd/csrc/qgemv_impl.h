// qgemv_impl.h -- bandwidth-bound dequant-GEMV for small M (gfx950): the
// stream and split-K kernels, the helpers the other GEMV kernels share, and
// the per-bit-width launcher (launch_m).
//
// y[m, n] = sum_k x[m, k] * (s[n,g] * q[n,k] + b[n,g]).
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
// xs = sum of x over the group.  fp32 activations use plain fp32 FMAs.
#pragma once
#include "kernels.h"
#include "qcommon.h"

namespace lxq {
namespace gemv {

// ---------------------------------------------------------------------------
// Streaming kernel for K <= 4096 (one 64-code unit per lane): M <= 4 with
// 16-bit x, M == 1 with f32 x.
//
// A block is 4 waves (one per SIMD); wave w owns R consecutive rows.  Per
// block, x and the scale/bias rows of the block's 4R rows are copied into
// LDS by buffer->LDS DMA, once.  Each wave then loads its rows' packed
// words straight into registers (buffer loads: wave-uniform row offsets in
// SGPRs, no per-lane address arithmetic) and computes row r as soon as row
// r's loads have landed, so the HBM stream overlaps the arithmetic.  Lane
// partials of all rows are reduced together with permlane swaps and DPP.
//
// Operands (exact products, fp32 accumulation):
//   f16 x, 4-bit: a code kept in place inside a 16-bit half is an f16
//     subnormal, value q * 2^(p-24) for bit position p: the codes at p = 0
//     and p = 4 of each half need only a mask (the other two after one
//     shift by 8), and sum x*v = 2^-24 (sum_{p=0} x q + 16 sum_{p=4} x q).
//   f16 x, 8-bit: bytes 0 and 2 (and, after a shift by 8, bytes 1 and 3)
//     are subnormals q * 2^-24.
//   otherwise the "1 + q/2^P" operands of unit_pairs_magic (bf16 cannot use
//     subnormals: x * q * 2^-133 underflows fp32), or fp32 FMAs for f32 x.
// ---------------------------------------------------------------------------

typedef __attribute__((address_space(3))) void* lds_ptr;
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
typedef uint32_t v2u32 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}
// a per-lane buffer offset that reads zeros: every buffer here is < 2^31 bytes
constexpr uint32_t kZeroOff = 0x80000000u;

constexpr int kStreamWaves = 4;

// Staged x of the stream kernel: unit u (64 elements, 8 or 16 chunks of 16 B)
// keeps logical chunk j in slot j ^ x_swz(u).  Lane u reads its own unit, so
// the lanes of one LDS pass read units 128 or 256 B apart; the swizzle puts
// them in different bank groups (16 consecutive lanes hit 16 distinct 16-byte
// slots of a 256-byte window).
template <int XE>
__device__ __host__ __forceinline__ int x_swz(int u) {
    return XE == 4 ? (u & 15) : ((u & 7) ^ ((u >> 3) & 1));
}

enum : int { OP_SUB4 = 0, OP_SUB8 = 1, OP_MAGIC = 2, OP_BF16U8 = 3, OP_F32 = 4, OP_SUB3 = 5, OP_SUB6 = 6 };
template <int BITS, int TX>
constexpr int op_kind() {
    return TX == DT_F32 ? OP_F32
         : (TX == DT_F16 && BITS == 4) ? OP_SUB4
         : (TX == DT_F16 && BITS == 8) ? OP_SUB8
         : (TX == DT_BF16 && BITS == 8) ? OP_BF16U8
         : OP_MAGIC;
}

// load instructions per 64-code unit (2*BITS words: 128-bit loads + one 64-bit)
template <int BITS>
constexpr int unit_loads() { return (2 * BITS) / 4 + ((2 * BITS) % 4 ? 1 : 0); }

template <int BITS>
__device__ __forceinline__ void load_unit_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                              uint32_t* w) {
    constexpr int W = 2 * BITS;
#pragma unroll
    for (int i = 0; i + 4 <= W; i += 4) {
        const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 4 * i, soff, 0);
        w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
    }
    if constexpr (W % 4 == 2) {
        const v2u32 v = __builtin_amdgcn_raw_buffer_load_b64(r, voff + 4 * (W - 2), soff, 0);
        w[W - 2] = v.x; w[W - 1] = v.y;
    }
}

template <int TX, int SB, int MR, int R>
struct StreamLds {
    static constexpr int kSb = SB == DT_F32 ? 4 : 2;
    static constexpr int kXRow = (TX == DT_F32 ? 4 : 2) * 4096;  // one x row, K <= 4096
    static constexpr int kRows = kStreamWaves * R;
    // the block's scale rows (at most 128 groups) plus 16 B of alignment slack
    static constexpr int kSbBytes = kRows * 128 * kSb + 16;
    static constexpr int X = 0;
    static constexpr int S = MR * kXRow;
    static constexpr int B = S + kSbBytes;
    static constexpr int BYTES = B + kSbBytes;
};

// x operands of one lane's unit for one row of x
template <int BITS, int TX, int OP>
struct XOps {
    static constexpr int kRegs = OP == OP_F32 ? 64 : 32;
    uint32_t v[kRegs];
    float h0, h1;  // sums of x over the unit's two 32-code halves (scaled for OP_SUB*)
    float hs;      // h0 + h1
};

template <int BITS, int TX, int OP>
__device__ __forceinline__ void prep_x(const uint8_t* lx, int sw, XOps<BITS, TX, OP>& o) {
    // lx: the lane's staged unit, logical chunk i in slot i ^ sw (x_swz)
    if constexpr (OP == OP_F32) {
        const v4u32* p = reinterpret_cast<const v4u32*>(lx);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const v4u32 t = p[i ^ sw];
            o.v[4 * i] = t.x; o.v[4 * i + 1] = t.y; o.v[4 * i + 2] = t.z; o.v[4 * i + 3] = t.w;
        }
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) a += __uint_as_float(o.v[i]);
#pragma unroll
        for (int i = 32; i < 64; i++) b += __uint_as_float(o.v[i]);
        o.h0 = a;
        o.h1 = b;
        o.hs = a + b;
    } else {
        uint32_t nat[32];
        const v4u32* p = reinterpret_cast<const v4u32*>(lx);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const v4u32 t = p[i ^ sw];
            nat[4 * i] = t.x; nat[4 * i + 1] = t.y; nat[4 * i + 2] = t.z; nat[4 * i + 3] = t.w;
        }
        // half sums: dot2 against (1, 1) is exact per product, fp32 accumulate
        const uint32_t one2 = TX == DT_F16 ? 0x3C003C00u : 0x3F803F80u;
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) a = dot2(nat[i], one2, a, TX);
#pragma unroll
        for (int i = 16; i < 32; i++) b = dot2(nat[i], one2, b, TX);
        if constexpr (OP == OP_SUB4) {
            // word j covers x[8j..8j+7] = nat[4j..4j+3]; operand order per word:
            // (x0,x4) (x1,x5) (x2,x6) (x3,x7)  [mask 0xF, mask 0xF0, >>8 then the same]
#pragma unroll
            for (int j = 0; j < 8; j++) {
                o.v[4 * j]     = __builtin_amdgcn_perm(nat[4 * j + 2], nat[4 * j], 0x05040100u);
                o.v[4 * j + 1] = __builtin_amdgcn_perm(nat[4 * j + 2], nat[4 * j], 0x07060302u);
                o.v[4 * j + 2] = __builtin_amdgcn_perm(nat[4 * j + 3], nat[4 * j + 1], 0x05040100u);
                o.v[4 * j + 3] = __builtin_amdgcn_perm(nat[4 * j + 3], nat[4 * j + 1], 0x07060302u);
            }
            o.h0 = a * 0x1p-24f;
            o.h1 = b * 0x1p-24f;
            o.hs = (a + b) * 0x1p-24f;
        } else if constexpr (OP == OP_SUB8) {
            // word j covers x[4j..4j+3] = nat[2j], nat[2j+1]: (x0,x2) (x1,x3)
#pragma unroll
            for (int j = 0; j < 16; j++) {
                o.v[2 * j]     = __builtin_amdgcn_perm(nat[2 * j + 1], nat[2 * j], 0x05040100u);
                o.v[2 * j + 1] = __builtin_amdgcn_perm(nat[2 * j + 1], nat[2 * j], 0x07060302u);
            }
            o.h0 = a * 0x1p-24f;
            o.h1 = b * 0x1p-24f;
            o.hs = (a + b) * 0x1p-24f;
        } else {
            constexpr bool kApart = (OP == OP_MAGIC) && PairLayout<BITS>::kApart;
            if constexpr (kApart) {
                // block of P codes = P/2 dwords; pair j = (x_j, x_{j+P/2})
                constexpr int P = PairLayout<BITS>::kCodesPerWord, D = P / 2;
#pragma unroll
                for (int blk = 0; blk < 64 / P; blk++) {
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
#pragma unroll
                for (int i = 0; i < 32; i++) o.v[i] = nat[i];
            }
            o.h0 = a;
            o.h1 = b;
            o.hs = a + b;
        }
    }
}

// factor that turns the reduced lane partials into y
template <int OP>
constexpr float out_scale() { return (OP == OP_SUB4 || OP == OP_SUB8 || OP == OP_SUB3 || OP == OP_SUB6) ? 0x1p24f : 1.f; }

// partial of one row for one row of x.  TWO (group size 32): s0/b0 cover
// codes 0..31 and s1/b1 codes 32..63; otherwise one group covers the unit
// and s1/b1 are unused.
template <int BITS, int TX, int OP, bool TWO>
__device__ __forceinline__ float row_partial(const uint32_t* w, const XOps<BITS, TX, OP>& xo, float s0,
                                             float b0, float s1, float b1) {
    if constexpr (OP == OP_SUB4) {
        // a: codes at bit 0 (q * 2^-24); c: codes at bit 4 (16 q * 2^-24)
        float a0 = 0.f, c0 = 0.f, a1 = 0.f, c1 = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t wj = w[j], w8 = wj >> 8;
            float& a = (TWO && j >= 4) ? a1 : a0;
            float& c = (TWO && j >= 4) ? c1 : c0;
            a = dot2(xo.v[4 * j], wj & 0x000F000Fu, a, DT_F16);
            c = dot2(xo.v[4 * j + 1], wj & 0x00F000F0u, c, DT_F16);
            a = dot2(xo.v[4 * j + 2], w8 & 0x000F000Fu, a, DT_F16);
            c = dot2(xo.v[4 * j + 3], w8 & 0x00F000F0u, c, DT_F16);
        }
        if constexpr (TWO)
            return fmaf(s0, fmaf(c0, 0.0625f, a0), fmaf(s1, fmaf(c1, 0.0625f, a1), fmaf(b0, xo.h0, b1 * xo.h1)));
        else
            return fmaf(s0, fmaf(c0, 0.0625f, a0), b0 * xo.hs);
    } else if constexpr (OP == OP_SUB8) {
        float d0 = 0.f, d1 = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t wj = w[j], w8 = wj >> 8;
            float& d = j < 8 ? d0 : d1;
            d = dot2(xo.v[2 * j], wj & 0x00FF00FFu, d, DT_F16);
            d = dot2(xo.v[2 * j + 1], w8 & 0x00FF00FFu, d, DT_F16);
        }
        if constexpr (TWO) return fmaf(s0, d0, fmaf(s1, d1, fmaf(b0, xo.h0, b1 * xo.h1)));
        else return fmaf(s0, d0 + d1, b0 * xo.hs);
    } else if constexpr (OP == OP_F32) {
        float d0 = 0.f, d1 = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) d0 = fmaf(__uint_as_float(xo.v[i]), (float)unit_code<BITS>(w, i), d0);
#pragma unroll
        for (int i = 32; i < 64; i++) d1 = fmaf(__uint_as_float(xo.v[i]), (float)unit_code<BITS>(w, i), d1);
        if constexpr (TWO) return (s0 * d0 + b0 * xo.h0) + (s1 * d1 + b1 * xo.h1);
        else return s0 * (d0 + d1) + b0 * xo.hs;
    } else {
        uint32_t pr[32];
        if constexpr (OP == OP_MAGIC)
            unit_pairs_magic<BITS, (TX == DT_F16 ? 10 : 7)>(w, pr);
        else
            unit_pairs_bf16_u8(w, pr);
        float d0 = 0.f, d1 = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) d0 = dot2(xo.v[i], pr[i], d0, TX);
#pragma unroll
        for (int i = 16; i < 32; i++) d1 = dot2(xo.v[i], pr[i], d1, TX);
        if constexpr (OP == OP_MAGIC) {
            // D = sum x v(q) = h + sum x q / kPow  =>  s sum x q + b h = (s kPow) D + (b - s kPow) h
            constexpr float kPow = MagicCfg<BITS, (TX == DT_F16 ? 10 : 7)>::kPow;
            if constexpr (TWO)
                return ((s0 * kPow) * d0 + fmaf(-s0, kPow, b0) * xo.h0) +
                       ((s1 * kPow) * d1 + fmaf(-s1, kPow, b1) * xo.h1);
            else
                return (s0 * kPow) * (d0 + d1) + fmaf(-s0, kPow, b0) * xo.hs;
        } else {
            if constexpr (TWO) return (s0 * d0 + b0 * xo.h0) + (s1 * d1 + b1 * xo.h1);
            else return s0 * (d0 + d1) + b0 * xo.hs;
        }
    }
}

__device__ __forceinline__ float swap32_sum(float a, float b) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float swap16_sum(float a, float b) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Eight 64-lane sums at once.  permlane32 swaps fold value pairs into lane
// halves, permlane16 swaps into 16-lane rows, then an 8-lane rotate merges
// two values per row and DPP finishes each 8-lane group.  Afterwards lanes
// with (lane & 7) == 0 hold the sum of v[sum8_index(lane)].
__device__ __forceinline__ float sum8(const float* v, int lane) {
    const float w0 = swap32_sum(v[0], v[1]), w1 = swap32_sum(v[2], v[3]);
    const float w2 = swap32_sum(v[4], v[5]), w3 = swap32_sum(v[6], v[7]);
    const float u0 = swap16_sum(w0, w1), u1 = swap16_sum(w2, w3);  // rows: v0 v2 v1 v3 / v4 v6 v5 v7
    const bool hi = lane & 8;
    const float a = hi ? u1 : u0, b = hi ? u0 : u1;
    float z = a + dpp_f<0x128>(b);  // row_ror:8
    z += dpp_f<0xB1>(z);            // quad_perm [1,0,3,2]
    z += dpp_f<0x4E>(z);            // quad_perm [2,3,0,1]
    z += dpp_f<0x141>(z);           // row_half_mirror
    return z;
}
__device__ __host__ __forceinline__ int sum8_index(int lane) {
    const int row = lane >> 4, half = (lane >> 3) & 1;
    return 4 * half + (((row & 1) << 1) | (row >> 1));
}

template <int BITS, int TX, int SB, int MR, int R, bool TWO, bool EPI>
__global__ __launch_bounds__(64 * kStreamWaves) void qgemv_stream_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, int gshift,
    Epilogue ep) {
    using L = StreamLds<TX, SB, MR, R>;
    constexpr int OP = op_kind<BITS, TX>();
    constexpr int XE = TX == DT_F32 ? 4 : 2;
    constexpr int W = 2 * BITS;
    __shared__ __attribute__((aligned(16))) uint8_t lds[L::BYTES];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int units = K >> 6;
    const bool active = lane < units;
    const int u = active ? lane : units - 1;
    const int G = K >> gshift;  // groups per row; group size 1 << gshift
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    const uint32_t sb_row = (uint32_t)G * L::kSb;
    const int nb0 = blockIdx.x * L::kRows;
    const int n0 = nb0 + wave * R;

    // Weight and scale buffer resources start at the block's first row (its
    // scales at the 16-byte chunk holding them), so every offset below stays
    // far under 2^31 whatever N is; the zero-reading offset kZeroOff lies
    // past every resource's size.
    const size_t sb_first = (size_t)nb0 * sb_row;
    const uint32_t sb_lead = (uint32_t)(sb_first & 15u);  // row nb0's scales within their chunk
    const size_t sb_base = sb_first - sb_lead;

    // ---- 1. x rows (zeros past K and past M) and the block's scale/bias rows into LDS ----
    {
        const auto xr = buf_rsrc(x, (uint32_t)M * K * XE);
        constexpr int XC = MR * L::kXRow / 16;  // 16-byte chunks
        const int kc = K * XE / 16;            // chunks of one x row
#pragma unroll
        for (int c0 = 0; c0 < XC; c0 += 64 * kStreamWaves) {
            const int cw = c0 + wave * 64, c = cw + lane;
            const int m = c / (L::kXRow / 16), cc = c % (L::kXRow / 16);
            // LDS slot cc holds the unit's chunk (cc % CPU) ^ swz, read back by prep_x
            constexpr int CPU = 4 * XE;  // 16-byte chunks per 64-element unit
            const int xu = cc / CPU, src = xu * CPU + ((cc % CPU) ^ x_swz<XE>(xu));
            const uint32_t voff = (cc < kc && m < M) ? (uint32_t)(m * K * XE + src * 16) : kZeroOff;
            if (cw < XC)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr)(lds + L::X + cw * 16), 16, voff, 0, 0, 0);
        }
        // whole 16-byte chunks: the last one may run into the buffer's tail slack
        const size_t sleft = (((size_t)N * sb_row - sb_base) + 15u) & ~(size_t)15u;
        const uint32_t sbytes = (uint32_t)(sleft < 0x7fffffffu ? sleft : 0x7fffffffu);
        const auto sr = buf_rsrc(static_cast<const uint8_t*>(scales) + sb_base, sbytes);
        const auto br = buf_rsrc(static_cast<const uint8_t*>(biases) + sb_base, sbytes);
        const int sc = (int)((sb_lead + L::kRows * sb_row + 15) / 16);
        for (int cw = wave * 64; cw < sc; cw += 64 * kStreamWaves) {
            if (cw + lane < sc) {
                const uint32_t voff = (uint32_t)(cw + lane) * 16;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_ptr)(lds + L::S + cw * 16), 16, voff, 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(br, (lds_ptr)(lds + L::B + cw * 16), 16, voff, 0, 0, 0);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. this wave's rows into registers; rows past N re-read row N-1
    // (never stored), idle lanes read zeros ----
    uint32_t w[R][W];
    {
        const size_t wleft = (size_t)(N - nb0) * row_bytes;
        const auto wr = buf_rsrc(reinterpret_cast<const uint8_t*>(wq) + (size_t)nb0 * row_bytes,
                                 (uint32_t)(wleft < 0x7fffffffu ? wleft : 0x7fffffffu));
        const uint32_t voff = active ? (uint32_t)lane * (8 * BITS) : kZeroOff;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int n = n0 + r < N ? n0 + r : N - 1;
            load_unit_buf<BITS>(wr, voff, (uint32_t)(n - nb0) * row_bytes, w[r]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // ---- 3. this wave's DMA was issued before its NW weight loads: wait for
    // it, then the barrier publishes every wave's part ----
    {
        constexpr int NW = R * unit_loads<BITS>();
        static_assert(NW < 64, "vmcnt holds 6 bits");
        __builtin_amdgcn_s_waitcnt((NW & 0xF) | ((NW >> 4) << 14) | (0x7 << 4) | (0xF << 8));
    }
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // ---- 4. x operands ----
    XOps<BITS, TX, OP> xo[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) prep_x<BITS, TX, OP>(lds + L::X + m * L::kXRow + u * 64 * XE, x_swz<XE>(u), xo[m]);

    // ---- 5. rows in arrival order ----
    // the unit's first group (codes 64u..): group size 32 -> 2u (and 2u+1)
    const int g0 = (u << 6) >> gshift;
    const uint8_t* ls = lds + L::S + sb_lead + (size_t)(wave * R) * sb_row + g0 * L::kSb;
    const uint8_t* lb = lds + L::B + sb_lead + (size_t)(wave * R) * sb_row + g0 * L::kSb;
    constexpr int V = R * MR, VP = (V + 7) / 8 * 8;
    float acc[VP];
#pragma unroll
    for (int i = 0; i < VP; i++) acc[i] = 0.f;
#pragma unroll
    for (int r = 0; r < R; r++) {
        float s0, b0, s1 = 0.f, b1 = 0.f;
        if constexpr (SB == DT_F32) {
            const float* ps = reinterpret_cast<const float*>(ls + r * sb_row);
            const float* pb = reinterpret_cast<const float*>(lb + r * sb_row);
            s0 = ps[0];
            b0 = pb[0];
            if constexpr (TWO) { s1 = ps[1]; b1 = pb[1]; }
        } else {
            const uint16_t* ps = reinterpret_cast<const uint16_t*>(ls + r * sb_row);
            const uint16_t* pb = reinterpret_cast<const uint16_t*>(lb + r * sb_row);
            s0 = SB == DT_F16 ? f16_to_f32(ps[0]) : bf16_to_f32(ps[0]);
            b0 = SB == DT_F16 ? f16_to_f32(pb[0]) : bf16_to_f32(pb[0]);
            if constexpr (TWO) {
                s1 = SB == DT_F16 ? f16_to_f32(ps[1]) : bf16_to_f32(ps[1]);
                b1 = SB == DT_F16 ? f16_to_f32(pb[1]) : bf16_to_f32(pb[1]);
            }
        }
#pragma unroll
        for (int m = 0; m < MR; m++) acc[r * MR + m] = row_partial<BITS, TX, OP, TWO>(w[r], xo[m], s0, b0, s1, b1);
    }
    // idle lanes (K < 4096) hold zero codes and x; zero them outright so a
    // non-finite scale they read cannot leak into the sums
    if (units < 64) {
#pragma unroll
        for (int i = 0; i < V; i++) acc[i] = active ? acc[i] : 0.f;
    }

    // ---- 6. reduce 8 values at a time; lanes with (lane & 7) == 0 store ----
#pragma unroll
    for (int c = 0; c < VP / 8; c++) {
        const float z = sum8(acc + 8 * c, lane) * out_scale<OP>();
        const int v = 8 * c + sum8_index(lane);
        const int r = v / MR, m = v % MR;
        if ((lane & 7) == 0 && v < V && m < M && n0 + r < N) store_out<EPI>(y, (size_t)m * N + n0 + r, n0 + r, ep, z);
    }
}

template <int BITS, int TX, int SB, int MR, int R, bool EPI>
LuxStatus launch_stream_e(const QmmArgs& a, hipStream_t st) {
    if (planned(a, "qgemv_stream_kernel")) return LuxStatus::Ok;
    const int rows = kStreamWaves * R;
    const int blocks = (a.N + rows - 1) / rows;
    const int gshift = a.group_size == 32 ? 5 : a.group_size == 64 ? 6 : 7;
    if (a.group_size == 32)
        hipLaunchKernelGGL((qgemv_stream_kernel<BITS, TX, SB, MR, R, true, EPI>), dim3(blocks),
                           dim3(64 * kStreamWaves), 0, st, a.x, a.wq, a.scales, a.biases, a.y, a.M, a.K,
                           a.N, gshift, a.epi());
    else
        hipLaunchKernelGGL((qgemv_stream_kernel<BITS, TX, SB, MR, R, false, EPI>), dim3(blocks),
                           dim3(64 * kStreamWaves), 0, st, a.x, a.wq, a.scales, a.biases, a.y, a.M, a.K,
                           a.N, gshift, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

template <int BITS, int TX, int SB, int MR, int R>
LuxStatus launch_stream(const QmmArgs& a, hipStream_t st) {
    return a.has_epilogue() ? launch_stream_e<BITS, TX, SB, MR, R, true>(a, st)
                            : launch_stream_e<BITS, TX, SB, MR, R, false>(a, st);
}

// rows per wave: 4 (measured over R = 2..7 at K = 4096: equal to R = 7 at
// N = 14336 and 6-9 % faster at N = 11008 and 4096, where 28-row blocks
// leave the CUs unevenly loaded)
template <int BITS, int TX, int MR>
LuxStatus launch_stream_r(const QmmArgs& a, hipStream_t st) {
    constexpr int R = 4;
    switch (a.sb_dtype) {
    case DT_F32: return launch_stream<BITS, TX, DT_F32, MR, R>(a, st);
    case DT_F16: return launch_stream<BITS, TX, DT_F16, MR, R>(a, st);
    default: return launch_stream<BITS, TX, DT_BF16, MR, R>(a, st);
    }
}

// ---------------------------------------------------------------------------
// Split-K streaming kernel: M == MR (1, or 2 with 16-bit x), 4096 < K <= 32768.
//
// The stream kernel's arithmetic with K split over the waves of a block: a
// block owns R rows; its KS = ceil(K / 4096) waves split K into parts of
// PU <= 64 units (one 64-code unit per lane), each wave loads its part of the
// R rows straight into registers and computes the R x MR partials as the
// stream kernel does, and the parts meet in LDS.  x (MR rows, all of K, units swizzled as in
// the stream kernel) and the block's R scale and bias rows are copied into
// (dynamic) LDS by buffer->LDS DMA once per block; one vmcnt wait plus a
// barrier publishes them while the weight loads stay in flight.
// ---------------------------------------------------------------------------
constexpr int kSplitMaxWaves = 8;
// rows per block: 8 for one row of x with codes of <= 4 bits (the block's
// copy of x, K * sizeof(x) bytes, then serves twice the weight bytes), else 4
// (R * MR <= 8 partials per wave, and the weight words stay in registers).
// Measured against 4 rows, same box: K = 14336, N = 4096 9.6-9.7 us against
// 10.0-10.2; K = 8192, N = 28672 29.4-29.9 against 32.7; f32 x, K = N = 8192
// 17.9-18.8 against 20.7.
constexpr bool kSplitRows8 = true;
__host__ __device__ constexpr int split_rows(int mr, int bits) { return kSplitRows8 && mr == 1 && bits <= 4 ? 8 : 4; }

// LDS bytes of the split kernel with R rows per block: x, a zero unit (read
// by idle lanes), then the R scale and R bias rows (16-byte aligned, with
// room for the lead of the first row within its chunk), then the waves'
// partials
__host__ __device__ constexpr size_t split_sb_bytes(int R, int K, int gs, int sb_bytes) {
    return ((size_t)R * (K / gs) * sb_bytes + 16 + 15) & ~(size_t)15;
}
__host__ __device__ constexpr size_t split_lds_bytes(int mr, int R, int K, int xe, int gs, int sb_bytes) {
    return ((size_t)mr * K + 64) * xe + 2 * split_sb_bytes(R, K, gs, sb_bytes) + (size_t)kSplitMaxWaves * 8 * 4;
}

// R: rows per block, split_rows(MR, BITS), or 4 where 8 rows of scales do
// not fit the LDS (f32 x and scales at the largest K)
template <int BITS, int TX, int SB, int MR, int R, bool TWO, bool EPI>
__global__ __launch_bounds__(64 * kSplitMaxWaves) void qgemv_split_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int K, int N, int gshift, int pu, Epilogue ep) {
    // f16 x with 4-bit codes: the magic-number form, not the subnormal one.
    // Against the oracle's fp64 accumulation the subnormal form's error
    // grows with K (median 2.5e-6 of max|y| at K = 4096, 1e-5 at K = 14336,
    // above the fp32 gate); the other forms stay within 2.4e-6 there.
    constexpr int OP = op_kind<BITS, TX>() == OP_SUB4 ? OP_MAGIC : op_kind<BITS, TX>();
    constexpr int XE = TX == DT_F32 ? 4 : 2;
    constexpr int W = 2 * BITS;
    constexpr int kSb = SB == DT_F32 ? 4 : 2;
    static_assert(R * MR <= 8, "one sum8 pass");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = blockDim.x >> 6;
    const int units = K >> 6;
    const int u = wave * pu + lane;                 // this lane's unit
    const bool active = lane < pu && u < units;
    const int G = K >> gshift;
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    const uint32_t sb_row = (uint32_t)G * kSb;
    const int n0 = blockIdx.x * R;
    const size_t sbb = split_sb_bytes(R, K, 1 << gshift, kSb);
    uint8_t* const lx = lds;
    uint8_t* const lzero = lds + (size_t)MR * K * XE;  // one unit of zeros
    uint8_t* const lsd = lzero + 64 * XE;
    uint8_t* const lbd = lsd + sbb;
    float* const red = reinterpret_cast<float*>(lbd + sbb);

    // scale rows of the block from the 16-byte chunk holding row n0's first
    const size_t sb_first = (size_t)n0 * sb_row;
    const uint32_t sb_lead = (uint32_t)(sb_first & 15u);
    const size_t sb_base = sb_first - sb_lead;

    // ---- 1. x and the block's scale/bias rows into LDS, and the zero unit ----
    {
        if (wave == 0 && lane < 4 * XE) *reinterpret_cast<v4u32*>(lzero + lane * 16) = v4u32{0u, 0u, 0u, 0u};
        const auto xr = buf_rsrc(x, (uint32_t)MR * K * XE);
        constexpr int CPU = 4 * XE;  // 16-byte chunks per 64-element unit
        const int kc = K * XE / 16;  // chunks of one x row
        for (int cw = wave * 64; cw < MR * kc; cw += 64 * nwaves) {
            const int cc = cw + lane;
            if (cc < MR * kc) {
                // LDS slot c of row m holds the unit's chunk (c % CPU) ^ swz, read back by prep_x
                const int m = cc / kc, c = cc % kc;
                const int xu = c / CPU, src = m * kc + xu * CPU + ((c % CPU) ^ x_swz<XE>(xu));
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr)(lx + cw * 16), 16, (uint32_t)src * 16, 0, 0, 0);
            }
        }
        const size_t sleft = (((size_t)N * sb_row - sb_base) + 15u) & ~(size_t)15u;
        const uint32_t sbytes = (uint32_t)(sleft < 0x7fffffffu ? sleft : 0x7fffffffu);
        const auto sr = buf_rsrc(static_cast<const uint8_t*>(scales) + sb_base, sbytes);
        const auto br = buf_rsrc(static_cast<const uint8_t*>(biases) + sb_base, sbytes);
        // all R rows: chunks past the array read zeros (rows past N)
        const int sc = (int)((sb_lead + (uint32_t)R * sb_row + 15) / 16);
        for (int cw = wave * 64; cw < sc; cw += 64 * nwaves) {
            if (cw + lane < sc) {
                const uint32_t voff = (uint32_t)(cw + lane) * 16;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_ptr)(lsd + cw * 16), 16, voff, 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(br, (lds_ptr)(lbd + cw * 16), 16, voff, 0, 0, 0);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. this wave's part of the block's rows into registers; rows past
    // N re-read row N-1 (never stored), idle lanes read zeros ----
    uint32_t w[R][W];
    {
        const size_t wleft = (size_t)(N - n0) * row_bytes;
        const auto wr = buf_rsrc(reinterpret_cast<const uint8_t*>(wq) + (size_t)n0 * row_bytes,
                                 (uint32_t)(wleft < 0x7fffffffu ? wleft : 0x7fffffffu));
        const uint32_t voff = active ? (uint32_t)u * (8 * BITS) : kZeroOff;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int n = n0 + r < N ? n0 + r : N - 1;
            load_unit_buf<BITS>(wr, voff, (uint32_t)(n - n0) * row_bytes, w[r]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // ---- 3. this wave's DMAs were issued before its NW weight loads: wait
    // for them (and for the zero unit's LDS writes), then the barrier
    // publishes every wave's part.  The count holds only while every weight
    // load is issued above: every lane uses every row's words below, with no
    // lane-dependent branch the compiler could sink a row's loads into. ----
    {
        constexpr int NW = R * unit_loads<BITS>();
        static_assert(NW < 64, "vmcnt holds 6 bits");
        __builtin_amdgcn_s_waitcnt((NW & 0xF) | ((NW >> 4) << 14) | (0x7 << 4));
    }
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // ---- 4. x operands of the lane's unit (idle lanes: the zero unit, zero
    // codes and zero scales, so their partials are exactly 0), then the rows
    // in arrival order ----
    XOps<BITS, TX, OP> xo[MR];
#pragma unroll
    for (int m = 0; m < MR; m++)
        prep_x<BITS, TX, OP>(active ? lx + ((size_t)m * K + (size_t)u * 64) * XE : lzero, active ? x_swz<XE>(u) : 0,
                             xo[m]);
    const int uc = active ? u : 0;
    const int g0 = (uc << 6) >> gshift;
    const uint8_t* ls = lsd + sb_lead + g0 * kSb;
    const uint8_t* lb = lbd + sb_lead + g0 * kSb;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = 0.f;
#pragma unroll
    for (int r = 0; r < R; r++) {
        float s0, b0, s1 = 0.f, b1 = 0.f;
        if constexpr (SB == DT_F32) {
            const float* ps = reinterpret_cast<const float*>(ls + r * sb_row);
            const float* pb = reinterpret_cast<const float*>(lb + r * sb_row);
            s0 = ps[0];
            b0 = pb[0];
            if constexpr (TWO) { s1 = ps[1]; b1 = pb[1]; }
        } else {
            const uint16_t* ps = reinterpret_cast<const uint16_t*>(ls + r * sb_row);
            const uint16_t* pb = reinterpret_cast<const uint16_t*>(lb + r * sb_row);
            s0 = SB == DT_F16 ? f16_to_f32(ps[0]) : bf16_to_f32(ps[0]);
            b0 = SB == DT_F16 ? f16_to_f32(pb[0]) : bf16_to_f32(pb[0]);
            if constexpr (TWO) {
                s1 = SB == DT_F16 ? f16_to_f32(ps[1]) : bf16_to_f32(ps[1]);
                b1 = SB == DT_F16 ? f16_to_f32(pb[1]) : bf16_to_f32(pb[1]);
            }
        }
        {
            // idle lanes: scales zeroed by a mask, not a branch (with a
            // branch per row at group size 32 the compiler kept every row's
            // decoded codes live at once and spilled them to scratch)
            const uint32_t am = active ? ~0u : 0u;
            s0 = __uint_as_float(__float_as_uint(s0) & am);
            b0 = __uint_as_float(__float_as_uint(b0) & am);
            s1 = __uint_as_float(__float_as_uint(s1) & am);
            b1 = __uint_as_float(__float_as_uint(b1) & am);
        }
#pragma unroll
        for (int m = 0; m < MR; m++) acc[r * MR + m] = row_partial<BITS, TX, OP, TWO>(w[r], xo[m], s0, b0, s1, b1);
    }

    // ---- 5. lane sums (lanes with (lane & 7) == 0 hold value sum8_index),
    // then the K parts meet in LDS and wave 0 stores ----
    const float z = sum8(acc, lane) * out_scale<OP>();
    if ((lane & 7) == 0) red[wave * 8 + sum8_index(lane)] = z;
    __syncthreads();
    if (wave == 0 && lane < R * MR) {
        float t = 0.f;
        for (int p = 0; p < nwaves; p++) t += red[p * 8 + lane];
        const int n = n0 + lane / MR, m = lane % MR;
        if (n < N) store_out<EPI>(y, (size_t)m * N + n, n, ep, t);
    }
}

template <int BITS, int TX, int SB, int MR, int R, bool TWO, bool EPI>
LuxStatus launch_split_k(const QmmArgs& a, hipStream_t st, int ks, int pu, size_t lds) {
    if (planned(a, "qgemv_split_kernel")) return LuxStatus::Ok;
    auto kern = qgemv_split_kernel<BITS, TX, SB, MR, R, TWO, EPI>;
    // once per instantiation; a function-local static initializes exactly once
    // even when several threads make the first call together
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return LuxStatus::Internal;
    const int gshift = a.group_size == 32 ? 5 : a.group_size == 64 ? 6 : 7;
    const int blocks = (a.N + R - 1) / R;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * ks), lds, st, a.x, a.wq, a.scales, a.biases, a.y, a.K, a.N,
                       gshift, pu, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

// one block's scale rows and its weight rows (relative to the block's first
// row) stay far below 2^31; x is below 128 KB
template <int BITS, int TX, int SB, int MR, int R>
LuxStatus launch_split_r(const QmmArgs& a, hipStream_t st, int ks, int pu, size_t lds) {
    const bool epi = a.has_epilogue();
    if (a.group_size == 32)
        return epi ? launch_split_k<BITS, TX, SB, MR, R, true, true>(a, st, ks, pu, lds)
                   : launch_split_k<BITS, TX, SB, MR, R, true, false>(a, st, ks, pu, lds);
    return epi ? launch_split_k<BITS, TX, SB, MR, R, false, true>(a, st, ks, pu, lds)
               : launch_split_k<BITS, TX, SB, MR, R, false, false>(a, st, ks, pu, lds);
}

// M == MR rows of x, 4096 < K <= 32768 (K % 64 == 0), x, scales and rows
// of 32-bit offsets, LDS within 160 KB; NotSupported otherwise
template <int BITS, int TX, int SB, int MR>
LuxStatus launch_split_sb(const QmmArgs& a, hipStream_t st) {
    if (a.M != MR || a.K <= 4096 || a.K % 64 != 0) return LuxStatus::NotSupported;
    const int units = a.K / 64;
    const int ks = (units + 63) / 64;
    if (ks > kSplitMaxWaves) return LuxStatus::NotSupported;
    const int pu = (units + ks - 1) / ks;
    constexpr int XE = TX == DT_F32 ? 4 : 2, kSb = SB == DT_F32 ? 4 : 2;
    constexpr int R = split_rows(MR, BITS);
    const size_t lds = split_lds_bytes(MR, R, a.K, XE, a.group_size, kSb);
    if (lds <= 160 * 1024) return launch_split_r<BITS, TX, SB, MR, R>(a, st, ks, pu, lds);
    // 8 rows of scales do not fit (f32 x and scales at the largest K): 4 rows
    if constexpr (R == 8) {
        const size_t lds4 = split_lds_bytes(MR, 4, a.K, XE, a.group_size, kSb);
        if (lds4 <= 160 * 1024) return launch_split_r<BITS, TX, SB, MR, 4>(a, st, ks, pu, lds4);
    }
    return LuxStatus::NotSupported;
}

template <int BITS, int TX, int MR>
LuxStatus launch_split(const QmmArgs& a, hipStream_t st) {
    switch (a.sb_dtype) {
    case DT_F32: return launch_split_sb<BITS, TX, DT_F32, MR>(a, st);
    case DT_F16: return launch_split_sb<BITS, TX, DT_F16, MR>(a, st);
    default: return launch_split_sb<BITS, TX, DT_BF16, MR>(a, st);
    }
}

// M == 1, K <= 4096: the whole-line kernel of qgemv_line.h (defined there,
// instantiated by the per-bit-width translation units); NotSupported for
// shapes it does not take
template <int BITS, int TX>
LuxStatus launch_line(const QmmArgs& a, hipStream_t st);

// 2 <= M <= 4, K <= 4096: the K-split whole-line kernel of qgemv_mx.h
// (defined there, instantiated by the per-bit-width translation units);
// NotSupported for shapes it does not take
template <int BITS>
LuxStatus launch_mx_b(const QmmArgs& a, hipStream_t st);

template <int BITS, int TX>
LuxStatus launch_m(const QmmArgs& a, hipStream_t st) {
    if (a.M == 1 && a.K <= 4096) {
        const LuxStatus s = launch_line<BITS, TX>(a, st);
        if (s != LuxStatus::NotSupported) return s;
    }
    if (a.M == 1 && a.K > 4096) {
        const LuxStatus s = launch_split<BITS, TX, 1>(a, st);
        if (s != LuxStatus::NotSupported) return s;
    }
    if constexpr (TX != DT_F32) {
        if (a.M == 2 && a.K > 4096) {
            const LuxStatus s = launch_split<BITS, TX, 2>(a, st);
            if (s != LuxStatus::NotSupported) return s;
        }
    }
    if (a.K <= 4096 && (a.M <= 4 && (TX != DT_F32 || a.M == 1))) {
        if (a.M <= 1) return launch_stream_r<BITS, TX, 1>(a, st);
        if constexpr (TX != DT_F32) {
            if (a.M <= 2) return launch_stream_r<BITS, TX, 2>(a, st);
            return launch_stream_r<BITS, TX, 4>(a, st);
        }
    }
    return LuxStatus::NotSupported;
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
