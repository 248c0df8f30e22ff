// qgemm_rw.h -- compute-bound dequant GEMM for large M (gfx950, MFMA) with
// each wave's W operand dequantized in its own registers: 4- and 8-bit
// codes, f16/bf16 activations.
//
// y[M, N] = x[M, K] . T(w_hat)[N, K]^T, T = the activation type: the
// "dequantize to the activation type, then matmul" semantics of the large
// GEMM (w_hat = RNE_T(fmaf(scale, q, bias)) in fp32, fp32 accumulation on
// v_mfma_f32_32x32x16_{bf16,f16}).
//
// Block tile 128 (M) x 256 (N), K step 64.  NW waves (8: two per SIMD, or
// 4: one); wave w owns the WN = 256 / NW columns n0 + w WN .. +WN and all
// 128 rows, i.e. 4 x NT MFMA tiles of 32 x 32.  No two waves share a
// column, so every code is dequantized exactly once per block, by the wave
// that multiplies it, straight into the MFMA's B operand registers: the W
// tile never passes through LDS as values.  With two waves per SIMD the
// hardware runs one wave's dequantization while the other's MFMAs execute.
//
// Lane (c = lane % 32, h = lane / 32) of a 32 x 32 x 16 MFMA holds 8
// consecutive k of row/column c.  Within a K step of 64 the lane half h owns
// k in [32 h, 32 h + 32), and k sub-step j takes [32 h + 8 j, +8) from both
// operands.  A lane's codes of a step are then one contiguous 4 BITS-byte
// run of its column's row (one 16-byte chunk at 4 bits), and its x operand
// of sub-step j is 16-byte chunk 4 h + j of the row's 128-byte step.
//
// LDS (all filled by global->LDS transfers, global_load_lds_dwordx4, issued
// D steps ahead, so no vector-memory load lands in registers in the loop
// and the explicit per-step waits count every transfer in flight):
//   x ring      D + BAR stages of 128 rows x 128 B (16-byte chunk c of row r
//               at position c ^ swz(r): conflict-free fragment reads)
//   code ring   D + 1 stages; wave-private: each wave copies and reads only
//               its own columns' codes (a lane reads back exactly the 16
//               bytes it copied)
//   scale ring  3 windows; wave-private; a window holds one 16-byte chunk
//               of each of the wave's columns' scale and bias rows, i.e.
//               GS / (4 sizeof(T_sb)) K steps
// One barrier every BAR K steps guards the shared x ring: at it every wave
// has read the steps before and its transfers of the next BAR steps have
// landed.
//
// The B operand: masks leave pairs of codes in place in the two halves of a
// word, as the f16 subnormals q 2^(p-24) (p = the code's bit position in its
// half), and v_fma_mix_f32 computes fma(s 2^(24-p), q 2^(p-24), b), whose
// product is exactly s q: each value is fmaf(s, q, b) bit for bit, one
// instruction per code (2^(24-p) s is exact for |s| < 2^103).
//
// Work units: tiles (K halves for a split last round, K parts for a shape
// with few tiles; qsplit.h).  Grid: one block per unit, or, where there are
// more units than CUs and the output is 16-bit, one block per CU running
// units b, b + 256, ... (whole tiles first, halves last): at each hand-over
// the next unit's first transfers go out before the finished tile is
// staged and stored, so its prologue latency runs under the output stage,
// and no block waits for a slot.  The output tile is staged in LDS and
// stored as whole 16-byte chunks of rows.  Tiles are dealt to the 8 XCDs
// (block b runs on XCD b % 8) in 4 x 8 groups of M x N tiles, so the 32
// blocks an XCD runs at once share 4 x slabs and 8 W slabs in its L2.
#pragma once
#include <cstdlib>

#include "kernels.h"
#include "qcommon.h"
#include "qsplit.h"

namespace lxq {
namespace rw {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr int BN = 256, BK = 64;
constexpr int kCUs = 256;

template <int TX_, int BITS_, int SB_, int GS_, int NW_, int D_, int BAR_, int MT_>
struct Cfg {
    static constexpr int TX = TX_, BITS = BITS_, SB = SB_, GS = GS_, NW = NW_;
    static constexpr int MT = MT_;                 // 32-row M tiles per block
    static constexpr int BM = 32 * MT;
    static constexpr int kXStage = BM * BK * 2;    // one K step of the block's x rows
    static constexpr int D = D_;                   // K steps of transfers in flight
    static constexpr int BAR = BAR_;               // K steps per barrier
    static constexpr int kSb = SB == DT_F32 ? 4 : 2;
    static constexpr int kThreads = 64 * NW;
    static constexpr int WN = BN / NW;             // columns per wave
    static constexpr int NT = WN / 32;             // 32-column tiles per wave
    // x transfers per wave per step (whole 1 KiB ones, or one with the
    // first kXL lanes where the stage is smaller than a transfer per wave)
    static constexpr int kXI = MT * 4 >= NW ? MT * 4 / NW : 1;
    static constexpr int kXL = MT * 4 >= NW ? 64 : 64 * MT * 4 / NW;
    static constexpr int kCI = NT * BITS / 4;      // code transfers per wave per step
    static constexpr int kWS = GS / (4 * kSb);     // K steps per scale window
    static constexpr int kSS = 1 + (D + kWS - 1) / kWS < 3 ? 3 : 1 + (D + kWS - 1) / kWS;  // scale windows
    static constexpr int kSI = NW == 4 ? 2 : 1;    // scale transfers per wave per window
    static constexpr int kXS = D + BAR;            // x stages
    static constexpr int kCS = D + 1;              // code stages
    static constexpr int kCodeStage = BN * 8 * BITS;
    static constexpr int kWinSlot = BN * 32;       // scale and bias chunk of every column
    static constexpr int kC0 = kXS * kXStage;
    static constexpr int kS0 = kC0 + kCS * kCodeStage;
    static constexpr int kLds = kS0 + kSS * kWinSlot;
    static constexpr int kUnroll = kWS > BAR ? kWS : BAR;  // loop unroll: whole windows and barrier groups
    static_assert(kWS >= 2 && kWS <= 16 && 16 % kWS == 0, "scale window of 2..16 steps");
    static_assert(BAR == 1 || BAR == 2 || BAR == 4, "steps per barrier");
    static_assert(D > BAR, "a barrier step waits for the next BAR batches with younger ones in flight");
    static_assert((kSS - 1) * kWS >= D, "a scale window slot is refilled only after its last read");
    static_assert(kLds <= 160 * 1024, "LDS budget");
    static_assert(kLds >= BM * (BN * 2 + 16) && kLds >= BM / 2 * (BN * 4 + 16), "the output tile's LDS passes fit");
    static_assert(MT == 1 || MT == 2 || MT == 4, "32, 64 or 128 rows per block");
    // transfers of the batch of step k (k % kUnroll == p)
    static constexpr int batch(int p) { return kXI + kCI + (p % kWS == 0 ? kSI : 0); }
    // transfers a step (k % kUnroll == P) may leave in flight when it waits:
    // at a barrier step (k + 1 a multiple of BAR) the batches of k + BAR + 1
    // .. k + D (those of k + 1 .. k + BAR must have landed for the barrier),
    // at the others those of k + 2 .. k + D (k + 1's codes and scales)
    static constexpr int young(int P) {
        int n = 0;
        for (int d = ((P + 1) % BAR == 0 ? BAR + 1 : 2); d <= D; d++) n += batch(P + d);
        return n;
    }
};

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// block barrier that is also a compiler memory fence and a scheduling
// boundary (the builtin alone lets LDS accesses and MFMAs move across it)
__device__ __forceinline__ void barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// global -> LDS: lane l copies 16 bytes from sbase + voff to LDS m0 + 16 l
__device__ __forceinline__ void dma16(uint32_t m0v, const void* sbase, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" : : "s"(m0v), "v"(voff), "s"(sbase) : "memory", "m0");
}
// the same with a per-lane 64-bit address
__device__ __forceinline__ void dma16a(uint32_t m0v, const void* addr) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(m0v), "v"(addr) : "memory", "m0");
}

__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

template <int TX>
__device__ __forceinline__ f32x16 mfma(const u4& a, const u4& b, const f32x16& c) {
    if constexpr (TX == DT_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                      0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                     0, 0, 0);
}

// two fp32 values -> a packed pair of T, RNE, one packed conversion (a
// scalar f16 cast of an fmaf result would fuse into v_fma_mixlo_f16, which
// rounds once where the format rounds twice)
template <int TX>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    if constexpr (TX == DT_BF16) {
        typedef __bf16 t2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, t2));
    } else {
        typedef _Float16 t2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, t2));
    }
}
__device__ __forceinline__ float lo(uint32_t m) { return (float)__builtin_bit_cast(h2, m)[0]; }
__device__ __forceinline__ float hi(uint32_t m) { return (float)__builtin_bit_cast(h2, m)[1]; }

// scale and bias of a lane's column for one K step, as the fma_mix factors
struct SB2 {
    float s24, s20, b;
};

template <int SB>
__device__ __forceinline__ float sb_val(uint32_t raw) {
    if constexpr (SB == DT_F32) return __uint_as_float(raw);
    else if constexpr (SB == DT_F16) return f16_to_f32(raw & 0xffffu);
    else return bf16_to_f32(raw & 0xffffu);
}

// B operand of sub-step j: codes 8 j .. 8 j + 7 of the lane's 32 (in BITS
// words cw[]), dequantized to T
template <int BITS, int TX>
__device__ __forceinline__ u4 b_operand(const uint32_t* cw, int j, const SB2& f) {
    float q[8];
    if constexpr (BITS == 4) {
        const uint32_t w = cw[j], w8 = w >> 8;
        const uint32_t m0 = w & 0x000F000Fu, m1 = w & 0x00F000F0u;   // codes 0, 4 at p = 0; 1, 5 at p = 4
        const uint32_t m2 = w8 & 0x000F000Fu, m3 = w8 & 0x00F000F0u; // codes 2, 6; 3, 7
        q[0] = fmaf(f.s24, lo(m0), f.b); q[4] = fmaf(f.s24, hi(m0), f.b);
        q[1] = fmaf(f.s20, lo(m1), f.b); q[5] = fmaf(f.s20, hi(m1), f.b);
        q[2] = fmaf(f.s24, lo(m2), f.b); q[6] = fmaf(f.s24, hi(m2), f.b);
        q[3] = fmaf(f.s20, lo(m3), f.b); q[7] = fmaf(f.s20, hi(m3), f.b);
    } else {
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const uint32_t w = cw[2 * j + e];
            const uint32_t ma = w & 0x00FF00FFu, mb = (w >> 8) & 0x00FF00FFu;  // codes 0, 2; 1, 3
            q[4 * e] = fmaf(f.s24, lo(ma), f.b);     q[4 * e + 2] = fmaf(f.s24, hi(ma), f.b);
            q[4 * e + 1] = fmaf(f.s24, lo(mb), f.b); q[4 * e + 3] = fmaf(f.s24, hi(mb), f.b);
        }
    }
    u4 r;
    r.x = pack2<TX>(q[0], q[1]);
    r.y = pack2<TX>(q[2], q[3]);
    r.z = pack2<TX>(q[4], q[5]);
    r.w = pack2<TX>(q[6], q[7]);
    return r;
}

// per-wave constants of the K loop
template <class C>
struct Ctx {
    uint8_t* lds;
    uint32_t lds_addr;           // LDS address of lds
    const uint8_t* x;            // x + the block's first K step (bytes)
    const uint8_t* wq;           // w_q + the block's first K step (bytes)
    uint32_t xoff[C::kXI];       // per x transfer: the lane's row (clamped) and swizzled chunk
    uint32_t coff[C::kCI];       // per code transfer: the lane's column (clamped) and chunk
    const uint8_t* sp[C::kSI];   // per scale transfer: the lane's column's scale or bias row, first window
    int wave, lane, KT;
    int frag;                    // byte of the lane's fragment row in an x stage (row r, chunk 4 h at j = 0)
    int sw;                      // swz(r)
    int sb_lds[2];               // per tile: the lane's scale byte in a window slot (group 0 of the window)
};

// the batch of step kt (< KT: clamped to the last step, whose data a
// transfer past the end re-reads into a stage nobody reads): x, codes and,
// where a window starts (WIN), the window's scales and biases
template <class C, bool WIN>
__device__ __forceinline__ void issue(const Ctx<C>& t, int kt) {
    const int k = kt < t.KT ? kt : t.KT - 1;
    const int xs = kt % C::kXS, cs = kt % C::kCS;
    {
        const uint32_t base = t.lds_addr + (uint32_t)(xs * C::kXStage) + (uint32_t)(t.wave * C::kXI * C::kXL * 16);
        const uint8_t* src = t.x + (size_t)k * (BK * 2);
        if (C::kXL == 64 || t.lane < C::kXL) {
#pragma unroll
            for (int i = 0; i < C::kXI; i++) dma16(base + (uint32_t)(C::kXL * 16 * i), src, t.xoff[i]);
        }
    }
    {
        const uint32_t base = t.lds_addr + (uint32_t)(C::kC0 + cs * C::kCodeStage) + (uint32_t)(t.wave * C::kCI * 1024);
        const uint8_t* src = t.wq + (size_t)k * (8 * C::BITS);
#pragma unroll
        for (int i = 0; i < C::kCI; i++) dma16(base + 1024u * i, src, t.coff[i]);
    }
    if constexpr (WIN) {
        const int win = k / C::kWS;
        const uint32_t base = t.lds_addr + (uint32_t)(C::kS0 + (kt / C::kWS) % C::kSS * C::kWinSlot) +
                              (uint32_t)(t.wave * C::WN * 32);
#pragma unroll
        for (int i = 0; i < C::kSI; i++) dma16a(base + 1024u * i, t.sp[i] + (size_t)win * 16);
    }
}

// registers carried from one K step to the next
template <class C>
struct Regs {
    u4 a[C::MT];                  // A fragments of sub-step 0 of the current step (reads in flight)
    u4 a3[C::MT];                 // A fragments of sub-step 3 of the previous step
    u4 b3[C::NT];                 // B operands of sub-step 3 of the previous step
    uint32_t cw[C::NT][C::BITS];  // codes of the current step (the lane's 4 BITS bytes per tile)
    SB2 f[C::NT];                 // scale factors of the current step
};

// codes and raw scale/bias words of step kt (its batch has landed for this wave)
template <class C>
__device__ __forceinline__ void read_step(const Ctx<C>& t, int kt, uint32_t (&cw)[C::NT][C::BITS],
                                          uint32_t (&rs)[C::NT], uint32_t (&rb)[C::NT]) {
    const uint8_t* cst = t.lds + C::kC0 + (kt % C::kCS) * C::kCodeStage + t.wave * C::kCI * 1024 + t.lane * 16;
#pragma unroll
    for (int tt = 0; tt < C::NT; tt++)
#pragma unroll
        for (int e = 0; e < C::BITS / 4; e++) {
            const u4 v = *reinterpret_cast<const u4*>(cst + (tt * (C::BITS / 4) + e) * 1024);
            cw[tt][4 * e] = v.x; cw[tt][4 * e + 1] = v.y; cw[tt][4 * e + 2] = v.z; cw[tt][4 * e + 3] = v.w;
        }
    // group of the lane's codes within the window: ((kt % kWS) 64 + 32 h) / GS
    const int gi = ((kt % C::kWS) * 64 + 32 * (t.lane >> 5)) / C::GS;
    const uint8_t* win = t.lds + C::kS0 + (kt / C::kWS) % C::kSS * C::kWinSlot + gi * C::kSb;
#pragma unroll
    for (int tt = 0; tt < C::NT; tt++) {
        const uint8_t* p = win + t.sb_lds[tt];
        if constexpr (C::SB == DT_F32) {
            rs[tt] = *reinterpret_cast<const uint32_t*>(p);
            rb[tt] = *reinterpret_cast<const uint32_t*>(p + C::WN * 16);
        } else {
            // the aligned dword holding the value, shifted into the low half
            const uint8_t* q = p - (gi & 1) * 2;
            const int sh = (gi & 1) * 16;
            rs[tt] = *reinterpret_cast<const uint32_t*>(q) >> sh;
            rb[tt] = *reinterpret_cast<const uint32_t*>(q + C::WN * 16) >> sh;
        }
    }
}

template <int SB, int NT>
__device__ __forceinline__ void factors(const uint32_t (&rs)[NT], const uint32_t (&rb)[NT], SB2 (&f)[NT]) {
#pragma unroll
    for (int tt = 0; tt < NT; tt++) {
        const float s = sb_val<SB>(rs[tt]);
        f[tt].s24 = s * 0x1p24f;
        f[tt].s20 = s * 0x1p20f;
        f[tt].b = sb_val<SB>(rb[tt]);
    }
}

// A fragments of sub-step j of the x stage of step kt
template <class C>
__device__ __forceinline__ void read_a(const Ctx<C>& t, int kt, int j, u4 (&a)[C::MT]) {
    const uint8_t* X = t.lds + (kt % C::kXS) * C::kXStage + t.frag;
    const int off = (((4 * (t.lane >> 5) + j) ^ t.sw) << 4);
#pragma unroll
    for (int i = 0; i < C::MT; i++) a[i] = *reinterpret_cast<const u4*>(X + i * 32 * 128 + off);
}

// the MT x NT MFMAs of one sub-step
template <int TX, int MT, int NT>
__device__ __forceinline__ void mfmas(f32x16 (&acc)[MT][NT], const u4 (&a)[MT], const u4 (&b)[NT]) {
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int tt = 0; tt < NT; tt++) acc[i][tt] = mfma<TX>(a[i], b[tt], acc[i][tt]);
}

// one MFMA, then up to V VALU instructions, repeated N times: the order the
// scheduler keeps for one sub-step (the VALU of the next sub-step's B
// operands runs while the matrix unit works)
template <int N, int V>
__device__ __forceinline__ void interleave() {
#pragma unroll
    for (int m = 0; m < N; m++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, V, 0);  // VALU
    }
}
// DS LDS reads first, then N MFMAs each followed by up to V VALU
template <int DS, int N, int V>
__device__ __forceinline__ void phase() {
    __builtin_amdgcn_sched_group_barrier(0x100, DS, 0);  // DS read
    interleave<N, V>();
}

// K step kt (kt % kUnroll == P).  On entry: the A fragments of sub-step 0
// of kt are being read, the operands of sub-step 3 of kt - 1 are in
// registers with their MFMAs not yet issued, the codes and scales of kt are
// in registers.  The step issues the batch of kt + D, runs those 4 NT
// MFMAs (which cover the reads), then sub-steps 0..2 of kt, each with the
// next sub-step's fragment reads issued before its MFMAs and the next B
// operands built between them; sub-step 3's operands are left for the next
// step.  Under sub-step 2: the wait for the transfers kt + 1 needs (at a
// barrier step, those of kt + 1 .. kt + BAR), kt + 1's codes and scales.
// At the end: the barrier (every BAR steps) and kt + 1's first fragments.
template <class C, int P>
__device__ __forceinline__ void step(const Ctx<C>& t, Regs<C>& r, f32x16 (&acc)[C::MT][C::NT], int kt) {
    constexpr int NT = C::NT, TX = C::TX, BITS = C::BITS, MT = C::MT;
    constexpr int V = (BITS == 4 ? 17 : 18) / MT + 1;  // VALU per MFMA of a B-operand build
    constexpr bool kBarrier = (P + 1) % C::BAR == 0;
    issue<C, (P + C::D) % C::kWS == 0>(t, kt + C::D);
    u4 b[NT];
#pragma unroll
    for (int tt = 0; tt < NT; tt++) b[tt] = b_operand<BITS, TX>(r.cw[tt], 0, r.f[tt]);
    mfmas<TX, MT, NT>(acc, r.a3, r.b3);
    uint32_t cwn[NT][BITS], rs[NT], rb[NT];
#pragma unroll
    for (int j = 0; j < 3; j++) {
        u4 an[MT], bn[NT];
        read_a(t, kt, j + 1, an);
        if (j == 2) {
            wait_vm<C::young(P)>();
            read_step(t, kt + 1, cwn, rs, rb);
        }
#pragma unroll
        for (int tt = 0; tt < NT; tt++) bn[tt] = b_operand<BITS, TX>(r.cw[tt], j + 1, r.f[tt]);
        mfmas<TX, MT, NT>(acc, j == 0 ? r.a : r.a3, b);
#pragma unroll
        for (int i = 0; i < MT; i++) r.a3[i] = an[i];
#pragma unroll
        for (int tt = 0; tt < NT; tt++) b[tt] = bn[tt];
    }
#pragma unroll
    for (int tt = 0; tt < NT; tt++) {
        r.b3[tt] = b[tt];
#pragma unroll
        for (int e = 0; e < BITS; e++) r.cw[tt][e] = cwn[tt][e];
    }
    factors<C::SB, NT>(rs, rb, r.f);
    // the order the scheduler keeps within the step: per sub-step phase the
    // fragment reads of the next sub-step first, then each MFMA followed by
    // a share of the VALU that builds the next B operands
    constexpr int kDsExtra = NT * (BITS / 4) + 2 * NT;  // codes and scale reads of kt + 1
    phase<MT, MT * NT, V>();
    phase<MT, MT * NT, V>();
    phase<MT, MT * NT, V>();
    phase<MT + kDsExtra, MT * NT, V>();
    wait_lgkm0();
    if constexpr (kBarrier) barrier();
    else __builtin_amdgcn_sched_barrier(0);
    read_a(t, kt + 1, 0, r.a);
}

template <class C, int P>
__device__ __forceinline__ void steps(const Ctx<C>& t, Regs<C>& r, f32x16 (&acc)[C::MT][C::NT], int kt) {
    if constexpr (P < C::kUnroll) {
        step<C, P>(t, r, acc, kt + P);
        steps<C, P + 1>(t, r, acc, kt);
    }
}

template <class C, int D0>
__device__ __forceinline__ void prologue_issue(const Ctx<C>& t) {
    if constexpr (D0 < C::D) {
        issue<C, D0 % C::kWS == 0>(t, D0);
        prologue_issue<C, D0 + 1>(t);
    }
}

// what one work unit is: a whole tile, one K half of a tile of the split
// last round, or one of nsplit K parts; its M / N tile and K steps
struct Unit {
    int tile, part, KT, k0, m0, n0;
};

template <class C>
__device__ __forceinline__ Unit unit_of(int u, int tiles, int split_from, int nsplit, int mtiles, int ntiles,
                                        int KT) {
    Unit w;
    w.tile = u;
    w.part = -1;
    w.KT = KT;
    w.k0 = 0;
    if (nsplit > 1) {
        // K parts: unit u = part * tiles + tile (the blocks running together
        // share a K range, i.e. the same x columns)
        w.tile = u % tiles;
        w.part = u / tiles;
        w.KT = KT / nsplit;
        w.k0 = w.part * w.KT;
    } else if (u >= split_from) {
        // units below split_from are whole tiles; the rest are the two K
        // halves (all first halves, then all second halves) of tiles split_from ..
        const int r = tiles - split_from, i = u - split_from;
        w.part = i >= r;
        w.tile = split_from + i - w.part * r;
        w.KT = KT >> 1;
        w.k0 = w.part * w.KT;
    }
    // tile -> (M tile, N tile): groups of 256 tiles, 32 per XCD as 4 x 8
    // M x N tiles, where the shape has whole groups; the rest in order
    const int tile = w.tile;
    const int groups = (mtiles == 4 || mtiles == 8 || mtiles == 16 || mtiles == 32) && ntiles % 8 == 0
                           ? mtiles * ntiles / 256 : 0;
    int mt, nt;
    if (tile < groups * 256) {
        const int g = tile >> 8, xcd = tile & 7, l = (tile >> 3) & 31;
        const int s = 8 * g + xcd, sm = mtiles / 4;  // super-tile s: 4 M x 8 N tiles
        mt = 4 * (s % sm) + (l & 3);
        nt = 8 * (s / sm) + (l >> 2);
    } else {
        const int r = tile - groups * 256, n_done = groups * 256 / mtiles;
        mt = r % mtiles;
        nt = n_done + r / mtiles;
    }
    w.m0 = mt * C::BM;
    w.n0 = nt * BN;
    return w;
}

// the K-loop constants of unit w for this wave and lane
template <class C>
__device__ __forceinline__ void setup_ctx(Ctx<C>& t, const Unit& w, uint8_t* lds, const uint16_t* x,
                                          const uint32_t* wq, const void* scales, const void* biases, int M, int K,
                                          int N, int wave, int lane) {
    constexpr int NT = C::NT, BITS = C::BITS, NW = C::NW, GS = C::GS, BM = C::BM;
    const int c = lane & 31, h = lane >> 5;
    const int m0 = w.m0, n0 = w.n0, k0 = w.k0;
    t.lds = lds;
    t.lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    t.x = reinterpret_cast<const uint8_t*>(x) + (size_t)k0 * BK * 2;
    t.wq = reinterpret_cast<const uint8_t*>(wq) + (size_t)k0 * 8 * BITS;
    t.wave = wave;
    t.lane = lane;
    t.KT = w.KT;
    // x transfers: wave w, transfer i fills the kXL * 16 bytes from block q
    // = w kXI + i on, 8 lanes per 128-byte row: lane -> row q kXL / 8 +
    // lane / 8, LDS chunk lane % 8, which holds global chunk (lane % 8) ^
    // swz(row)
#pragma unroll
    for (int i = 0; i < C::kXI; i++) {
        const int row = (wave * C::kXI + i) * (C::kXL / 8) + (lane >> 3);
        const int rg = min(m0 + min(row, BM - 1), M - 1);  // rows past M: valid data, never stored
        t.xoff[i] = ((uint32_t)rg * (uint32_t)K + (uint32_t)(((lane & 7) ^ swz(row)) << 3)) * 2u;
    }
    // code transfers: tile tt, part e: column n0 + w WN + 32 tt + c, the 16
    // bytes at 16 (2 h + e) [8-bit] / 16 h [4-bit] of the column's step
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
#pragma unroll
    for (int tt = 0; tt < NT; tt++)
#pragma unroll
        for (int e = 0; e < BITS / 4; e++) {
            const int n = min(n0 + wave * C::WN + 32 * tt + c, N - 1);  // columns past N: never stored
            t.coff[tt * (BITS / 4) + e] = (uint32_t)n * row_bytes + (uint32_t)(16 * ((BITS / 4) * h + e));
        }
    // scale transfers: 4 waves: transfer 0 = the scales of the wave's 64
    // columns (lane = column), transfer 1 = the biases; 8 waves: one
    // transfer, lanes 0..31 scales and 32..63 biases of the 32 columns
    const size_t sb_row = (size_t)(K / GS) * C::kSb;
    const size_t sb_first = (size_t)k0 * 64 / GS * C::kSb;  // the unit's first group
#pragma unroll
    for (int i = 0; i < C::kSI; i++) {
        const bool bias = NW == 4 ? i == 1 : h == 1;
        const int col = NW == 4 ? lane : c;
        const int n = min(n0 + wave * C::WN + col, N - 1);
        t.sp[i] = static_cast<const uint8_t*>(bias ? biases : scales) + (size_t)n * sb_row + sb_first;
    }
    t.frag = c * 128;
    t.sw = swz(c);
#pragma unroll
    for (int tt = 0; tt < 2; tt++) t.sb_lds[tt] = wave * C::WN * 32 + (32 * tt + c) * 16;
}

// rows [32 I0, 32 I1) of the block's tile, through the output stage, in
// 16-bit type TO into LDS at dst (row stride rs bytes, row 32 I0 first):
// lane (c, h) holds column c and rows 8 (v / 4) + 4 h + v % 4 of each 32 x
// 32 tile, so VGPRs v and v + 1 are two rows of one column, converted
// together
template <class C, bool EPI, int TO, int I0 = 0, int I1 = C::MT>
__device__ __forceinline__ void stage16(uint8_t* dst, int rs, const f32x16 (&acc)[C::MT][C::NT], const Epilogue& ep,
                                        int n0, int N, int wave, int c, int h) {
#pragma unroll
    for (int i = I0; i < I1; i++)
#pragma unroll
        for (int tt = 0; tt < C::NT; tt++) {
            const int nl = wave * C::WN + 32 * tt + c;  // column within the tile
#pragma unroll
            for (int v = 0; v < 16; v += 2) {
                const int ml = 32 * (i - I0) + 8 * (v >> 2) + 4 * h + (v & 3);
                float o0 = acc[i][tt][v], o1 = acc[i][tt][v + 1];
                if constexpr (EPI) {
                    if (n0 + nl < N) {
                        o0 = apply_epilogue(ep, (size_t)(n0 + nl), o0);
                        o1 = apply_epilogue(ep, (size_t)(n0 + nl), o1);
                    }
                }
                const uint32_t pk = pack2<TO>(o0, o1);
                uint8_t* d = dst + ml * rs + nl * 2;
                *reinterpret_cast<uint16_t*>(d) = (uint16_t)pk;
                *reinterpret_cast<uint16_t*>(d + rs) = (uint16_t)(pk >> 16);
            }
        }
}

// a 16-bit output tile handed over in a persistent grid: 16-byte chunks per
// thread (chunk j of thread tid: row tid / 32 + j kThreads / 32, columns
// 8 (tid % 32) ..+8), and the LDS above the rings where it is staged half
// its rows at a time while the next unit's first transfers land -- where
// that fits; else it is staged in the rings before those transfers are
// issued
template <class C>
constexpr int kHand = C::BM * BN * 2 / 16 / C::kThreads;
template <class C>
constexpr int kHandLds = C::BM / 2 * (BN * 2 + 16);
template <class C>
constexpr bool kStageAbove = C::kLds + kHandLds<C> <= 160 * 1024;

// half P of a handed-over tile (rows P BM / 2 ..+BM / 2) staged at hs and
// read back as the thread's chunks P kHand / 2 ..
template <class C, bool EPI, int P>
__device__ __forceinline__ void hand_half(uint8_t* hs, int rs, const f32x16 (&acc)[C::MT][C::NT], const Epilogue& ep,
                                          int n0, int N, int wave, int c, int h, int tid, u4 (&val)[kHand<C>]) {
    static_assert(C::MT % 2 == 0 && kHand<C> % 2 == 0, "halves of whole 32-row tiles and chunk rounds");
    constexpr int I0 = P * C::MT / 2, I1 = I0 + C::MT / 2, kHalf = kHand<C> / 2;
    if (ep.out_dt == DT_BF16) stage16<C, EPI, DT_BF16, I0, I1>(hs, rs, acc, ep, n0, N, wave, c, h);
    else stage16<C, EPI, DT_F16, I0, I1>(hs, rs, acc, ep, n0, N, wave, c, h);
    barrier();
#pragma unroll
    for (int i = 0; i < kHalf; i++) {
        const int q = tid + i * C::kThreads;
        val[P * kHalf + i] = *reinterpret_cast<const u4*>(hs + (q >> 5) * rs + (q & 31) * 16);
    }
}

// Grid: one block per unit (block b runs unit b), or fewer blocks than
// units: block b runs units b, b + grid, ... -- the launcher does so only
// for 16-bit outputs in 16-byte chunks (N % 8 == 0, y aligned) with 31-bit
// offsets, and with whole tiles before the halves (a half is always the
// last unit of its block)
template <class C, bool EPI>
__global__ __launch_bounds__(C::kThreads, 1) void qgemm_rw_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, Epilogue ep, int mtiles,
    int ntiles, int split_from, int nsplit, void* __restrict__ ws, uint32_t epoch, int units) {
    constexpr int NT = C::NT, MT = C::MT, BM = C::BM;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 31, h = lane >> 5;
    const int tiles = mtiles * ntiles;

    int u = blockIdx.x;
    Unit w = unit_of<C>(u, tiles, split_from, nsplit, mtiles, ntiles, K / BK);
    Ctx<C> t;
    setup_ctx<C>(t, w, lds, x, wq, scales, biases, M, K, N, wave, lane);
    // the next unit's context and its first D steps' transfers
    auto next_unit = [&](int un) {
        u = un;
        w = unit_of<C>(u, tiles, split_from, nsplit, mtiles, ntiles, K / BK);
        setup_ctx<C>(t, w, lds, x, wq, scales, biases, M, K, N, wave, lane);
        prologue_issue<C, 0>(t);
    };
    prologue_issue<C, 0>(t);
    f32x16 acc[MT][NT];
    bool handed = false;  // the previous unit's output stores follow this unit's first transfers
    for (;;) {
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
            for (int tt = 0; tt < NT; tt++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[i][tt][v] = 0.f;

        // prologue: the batches of steps 0 .. D - 1 are in flight; wait for
        // those of steps 0 .. BAR - 1 (vmcnt counts in issue order: the
        // younger batches and a handed-over tile's stores may still be in
        // flight).  The "previous sub-step 3" of step 0 is zeros (its MFMAs
        // add +0 to the +0 accumulators)
        Regs<C> r;
#pragma unroll
        for (int i = 0; i < MT; i++) r.a3[i] = u4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int tt = 0; tt < NT; tt++) r.b3[tt] = u4{0u, 0u, 0u, 0u};
        {
            constexpr int n = [] {
                int v = 0;
                for (int d = C::BAR; d < C::D; d++) v += C::batch(d);
                return v;
            }();
            if (handed) wait_vm<n + kHand<C>>();
            else wait_vm<n>();
        }
        barrier();
        {
            uint32_t rs[NT], rb[NT];
            read_step(t, 0, r.cw, rs, rb);
            factors<C::SB, NT>(rs, rb, r.f);
        }
        read_a(t, 0, 0, r.a);

        // KT is a multiple of kUnroll (the launcher's split rules keep it so)
        for (int kt = 0; kt < w.KT; kt += C::kUnroll) steps<C, 0>(t, r, acc, kt);
        // sub-step 3 of the last step
        mfmas<C::TX, MT, NT>(acc, r.a3, r.b3);
        // no transfer may still be landing when LDS is next written
        wait_vm<0>();
        const int un = u + (int)gridDim.x;
        if (un >= units || w.part >= 0) break;

        // ---- hand-over to unit un: every wave is past its K loop (the
        // rings are free after this barrier) ----
        barrier();
        const int mo = w.m0, no = w.n0;
        constexpr int rs = BN * 2 + 16;  // staging row stride: rows m and m + 4 in different banks
        u4 val[kHand<C>];
        if constexpr (kStageAbove<C>) {
            // the next unit's transfers first, then the tile above the
            // rings in two passes of BM / 2 rows
            next_unit(un);
            uint8_t* hs = lds + C::kLds;
            hand_half<C, EPI, 0>(hs, rs, acc, ep, no, N, wave, c, h, tid, val);
            barrier();
            hand_half<C, EPI, 1>(hs, rs, acc, ep, no, N, wave, c, h, tid, val);
        } else {
            // the tile in the rings in one pass, then the next unit's transfers
            if (ep.out_dt == DT_BF16) stage16<C, EPI, DT_BF16>(lds, rs, acc, ep, no, N, wave, c, h);
            else stage16<C, EPI, DT_F16>(lds, rs, acc, ep, no, N, wave, c, h);
            barrier();
#pragma unroll
            for (int i = 0; i < kHand<C>; i++) {
                const int q = tid + i * C::kThreads;
                val[i] = *reinterpret_cast<const u4*>(lds + (q >> 5) * rs + (q & 31) * 16);
            }
            barrier();
            next_unit(un);
        }
        // the stores: chunks past M or N (whole chunks, N % 8 == 0) get an
        // offset past the buffer's end, which the hardware drops, so every
        // thread issues exactly kHand stores after the next unit's transfers
        const __amdgpu_buffer_rsrc_t yr =
            __builtin_amdgcn_make_buffer_rsrc(y, 0, (int)((uint32_t)M * (uint32_t)N * 2u), 0x00020000);
#pragma unroll
        for (int j = 0; j < kHand<C>; j++) {
            const int m = mo + (tid >> 5) + C::kThreads / 32 * j, n = no + (tid & 31) * 8;
            const uint32_t off = m < M && n < N ? ((uint32_t)m * (uint32_t)N + (uint32_t)n) * 2u : 0x80000000u;
            __builtin_amdgcn_raw_buffer_store_b128(val[j], yr, off, 0, 0);
        }
        handed = true;
    }
    const int m0 = w.m0, n0 = w.n0;

    // a thread's sums as 16-byte vectors q (q = (i NT + tt) 4 + v / 4):
    // vector q of thread tid at byte (q threads + tid) 16 of a partial slot
    constexpr int kVec = MT * NT * 4;
    constexpr uint32_t kSlot = (uint32_t)(kVec * C::kThreads * 16);  // = BM BN 4
    const uint32_t voff = (uint32_t)tid * 16u;
    uint32_t* word = reinterpret_cast<uint32_t*>(lds);  // every transfer has landed
    if (nsplit > 1) {
        // ---- K parts: every part stores its sums; the last to count in adds
        // all nsplit of them in part order (the same bits whichever part is
        // last) and stores y; it also returns the tile's counter to zero ----
        const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
            static_cast<uint8_t*>(ws) + split::kPartOffset, 0, (int)((uint32_t)(tiles * nsplit) * kSlot), 0x00020000);
        const uint32_t slot = (uint32_t)(w.tile * nsplit + w.part) * kSlot;
#pragma unroll
        for (int q = 0; q < kVec; q++) {
            const f32x16& a = acc[q / (4 * NT)][(q / 4) % NT];
            const int v = 4 * (q % 4);
            __builtin_amdgcn_raw_buffer_store_b128(
                u4{__float_as_uint(a[v]), __float_as_uint(a[v + 1]), __float_as_uint(a[v + 2]), __float_as_uint(a[v + 3])},
                pr, voff, slot + (uint32_t)q * (C::kThreads * 16u), split::kCachePolicyDevice);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        barrier();
        if (tid == 0) *word = split::count_part(ws, w.tile, nsplit) ? 1u : 0u;
        barrier();
        if (*word == 0u) return;
        const uint32_t first = (uint32_t)(w.tile * nsplit) * kSlot;
#pragma unroll
        for (int q = 0; q < kVec; q++) {
            f32x16& a = acc[q / (4 * NT)][(q / 4) % NT];
            const int v = 4 * (q % 4);
            a[v] = a[v + 1] = a[v + 2] = a[v + 3] = 0.f;
        }
        // kPB parts' sums in flight together (32 vectors per thread: one
        // memory round trip per kPB parts, not per part); nsplit is a power
        // of two, so whole batches or a single one
        constexpr int kPB = kVec >= 32 ? 1 : 32 / kVec;
        for (int p0 = 0; p0 < nsplit; p0 += kPB) {
            u4 o[kPB][kVec];
#pragma unroll
            for (int pp = 0; pp < kPB; pp++)
#pragma unroll
                for (int q = 0; q < kVec; q++)
                    o[pp][q] = p0 + pp < nsplit
                                   ? __builtin_amdgcn_raw_buffer_load_b128(
                                         pr, voff, first + (uint32_t)(p0 + pp) * kSlot + (uint32_t)q * (C::kThreads * 16u),
                                         split::kCachePolicyDevice)
                                   : u4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int pp = 0; pp < kPB; pp++) {
                if (p0 + pp >= nsplit) break;
#pragma unroll
                for (int q = 0; q < kVec; q++) {
                    f32x16& a = acc[q / (4 * NT)][(q / 4) % NT];
                    const int v = 4 * (q % 4);
                    a[v] += __uint_as_float(o[pp][q].x);
                    a[v + 1] += __uint_as_float(o[pp][q].y);
                    a[v + 2] += __uint_as_float(o[pp][q].z);
                    a[v + 3] += __uint_as_float(o[pp][q].w);
                }
            }
        }
    } else if (w.part >= 0) {
        // ---- split last round: the two K halves meet (qsplit.h) ----
        const int st = w.tile - split_from;
        const uint32_t nslots = (uint32_t)(tiles - split_from);
        const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
            static_cast<uint8_t*>(ws) + split::kPartOffset, 0, (int)(nslots * kSlot), 0x00020000);
        barrier();
        if (tid == 0) *word = split::arrive_first(ws, st) ? 1u : 0u;
        barrier();
        const uint32_t slot = (uint32_t)st * kSlot;
        if (*word == 1u) {
#pragma unroll
            for (int q = 0; q < kVec; q++) {
                const f32x16& a = acc[q / (4 * NT)][(q / 4) % NT];
                const int v = 4 * (q % 4);
                __builtin_amdgcn_raw_buffer_store_b128(
                    u4{__float_as_uint(a[v]), __float_as_uint(a[v + 1]), __float_as_uint(a[v + 2]),
                       __float_as_uint(a[v + 3])},
                    pr, voff, slot + (uint32_t)q * (C::kThreads * 16u), split::kCachePolicyDevice);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            barrier();
            if (tid == 0) split::publish(ws, st, epoch);
            return;
        }
        if (tid == 0) *word = split::wait_partner(ws, st, epoch) ? 2u : 3u;
        barrier();
        const float fail = *word == 2u ? 0.f : __builtin_nanf("");
#pragma unroll
        for (int q = 0; q < kVec; q++) {
            const u4 o = __builtin_amdgcn_raw_buffer_load_b128(pr, voff, slot + (uint32_t)q * (C::kThreads * 16u),
                                                              split::kCachePolicyDevice);
            f32x16& a = acc[q / (4 * NT)][(q / 4) % NT];
            const int v = 4 * (q % 4);
            a[v] += __uint_as_float(o.x) + fail;
            a[v + 1] += __uint_as_float(o.y) + fail;
            a[v + 2] += __uint_as_float(o.z) + fail;
            a[v + 3] += __uint_as_float(o.w) + fail;
        }
    }

    // ---- output: lane holds column c of each 32 x 32 tile, VGPR v row
    // 8 (v / 4) + 4 h + v % 4.  The tile goes through LDS (free now: every
    // transfer has landed and every wave is past the K loop at the barrier)
    // so that the stores to y are whole 16-byte chunks of rows, in one pass
    // (two of half the rows for fp32 outputs of 128-row tiles).
    const bool f32_out = ep.out_dt == DT_F32;
    const int esz = f32_out ? 4 : 2;
    const int rs = BN * esz + 16;  // LDS row stride: rows m and m + 4 in different banks
    // vector stores need 16-byte aligned rows: N a multiple of 16 / esz, y aligned
    const bool vec = (((uintptr_t)y) & 15) == 0 && (N % (16 / esz)) == 0;
    const int passes = BM * rs > C::kLds ? 2 : 1, prow = BM / passes;
    for (int ps = 0; ps < passes; ps++) {
        barrier();
        if (!f32_out) {
            // one pass (prow = BM)
            if (ep.out_dt == DT_BF16) stage16<C, EPI, DT_BF16>(lds, rs, acc, ep, n0, N, wave, c, h);
            else stage16<C, EPI, DT_F16>(lds, rs, acc, ep, n0, N, wave, c, h);
        } else {
#pragma unroll
            for (int i = 0; i < MT; i++) {
                if (i * 32 / prow != ps) continue;
#pragma unroll
                for (int tt = 0; tt < NT; tt++) {
                    const int nl = wave * C::WN + 32 * tt + c;  // column within the tile
                    const int n = n0 + nl;
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int ml = 32 * i + 8 * (v >> 2) + 4 * h + (v & 3) - ps * prow;
                        float o = acc[i][tt][v];
                        if constexpr (EPI) {
                            if (n < N) o = apply_epilogue(ep, (size_t)n, o);
                        }
                        *reinterpret_cast<float*>(lds + ml * rs + nl * 4) = o;
                    }
                }
            }
        }
        barrier();
        // row r of the pass: BN * esz bytes = cpr 16-byte chunks
        const int cpr = BN * esz / 16;
        for (int q = tid; q < prow * cpr; q += C::kThreads) {
            const int rl = q / cpr, ch = q % cpr;
            const int m = m0 + ps * prow + rl, n = n0 + ch * (16 / esz);
            if (m >= M || n >= N) continue;
            const u4 val = *reinterpret_cast<const u4*>(lds + rl * rs + ch * 16);
            uint8_t* dst = static_cast<uint8_t*>(y) + ((size_t)m * N + n) * esz;
            if (vec && n + 16 / esz <= N) {
                *reinterpret_cast<u4*>(dst) = val;
            } else if (f32_out) {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (n + e < N) reinterpret_cast<uint32_t*>(dst)[e] = val[e];
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    if (n + e < N) reinterpret_cast<uint16_t*>(dst)[e] = (uint16_t)(val[e >> 1] >> (16 * (e & 1)));
            }
        }
    }
}

// the shapes this kernel takes: 4/8-bit codes, 16-bit x, K % 1024 == 0
// (whole scale windows, whole unrolled loops, group-aligned halves), x and W
// below 4 GiB (32-bit transfer offsets)
inline bool applies(int M, int K, int N, int bits, int x_dtype) {
    return (bits == 4 || bits == 8) && (x_dtype == DT_BF16 || x_dtype == DT_F16) && K % 1024 == 0 && M > 0 &&
           N > 0 && (size_t)M * K * 2 < (1ull << 32) && (size_t)N * K * bits / 8 < (1ull << 32);
}

// K parts for a shape with few tiles: the largest power of two (at most 16)
// that keeps the grid within one block per CU, every part a whole number of
// unrolled loops, and the parts' sums within the workspace; 1 for shapes
// with at least half a round of tiles (their last round splits instead)
template <class C>
inline int k_parts(int tiles, int KT, const QmmArgs& a) {
    if (a.ws == nullptr || 2 * tiles > kCUs || tiles > split::kMaxPartTiles) return 1;
    int S = 1;
    while (S < 16 && tiles * 2 * S <= kCUs && KT % (2 * S * C::kUnroll) == 0 &&
           split::kPartOffset + (size_t)tiles * 2 * S * C::BM * BN * 4 <= a.ws_bytes)
        S *= 2;
    return S;
}

template <class C, bool EPI>
LuxStatus launch_e(const QmmArgs& a, hipStream_t st) {
    if (planned(a, "qgemm_rw_kernel")) return LuxStatus::Ok;
    auto kern = qgemm_rw_kernel<C, EPI>;
    constexpr int kLdsMax = C::kLds + (kStageAbove<C> ? kHandLds<C> : 0);
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax);
    if (attr != hipSuccess) return LuxStatus::Internal;
    const int mtiles = (a.M + C::BM - 1) / C::BM, ntiles = (a.N + BN - 1) / BN;
    const int tiles = mtiles * ntiles, KT = a.K / BK;
    const int nsplit = k_parts<C>(tiles, KT, a);
    // with whole tiles: the last round's tiles in two K halves where that
    // round is at most half full (each half a whole number of unrolled loops)
    const int r = tiles % kCUs;
    const int split_from = nsplit == 1 && a.ws != nullptr && a.epoch != 0u && r > 0 && 2 * r <= kCUs &&
                                   r <= split::kMaxHalfTiles && (KT / 2) % C::kUnroll == 0 &&
                                   a.ws_bytes >= split::kPartOffset + (size_t)r * (C::BM * BN * 4)
                               ? tiles - r
                               : tiles;
    const int units = nsplit > 1 ? tiles * nsplit : tiles + (tiles - split_from);
    // one block per CU where there are more units than CUs and the
    // hand-over's stores apply: 16-bit output in whole 16-byte chunks at
    // 31-bit offsets (chunks past the end are dropped by offset)
    const bool persist = nsplit == 1 && units > kCUs && a.out_dtype != DT_F32 && (((uintptr_t)a.y) & 15) == 0 &&
                         a.N % 8 == 0 && (size_t)a.M * a.N * 2 < 0x80000000ull;
    const int blocks = persist ? kCUs : units;
    const int lds = persist ? kLdsMax : C::kLds;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(C::kThreads), lds, st, static_cast<const uint16_t*>(a.x), a.wq,
                       a.scales, a.biases, a.y, a.M, a.K, a.N, a.epi(), mtiles, ntiles, split_from, nsplit, a.ws,
                       a.epoch, units);
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

// the configuration the plugin runs: two waves per SIMD, a barrier every
// step, 3 K steps of transfers in flight (a K step of a 128-row block runs
// ~0.9 us, so 3 steps ahead cover the memory latency)
template <int TX, int BITS, int SB, int GS, int MT>
using PluginCfg = Cfg<TX, BITS, SB, GS, 8, 3, 1, MT>;

// M > 64 (128-row blocks).  The 32- and 64-row forms of this kernel
// (MT = 1, 2) measured slower than the small-M GEMMs at every M <= 64 shape
// tried (c2 25.6 against 21.5 us; M = 17, 32, 64 at N = 8192..14336 by
// 10-65 %): a K step of so few rows is short, so each CU's transfers in
// flight bound its stream, and the K-part reduction adds a serial tail.
template <int TX, int BITS, int SB, int GS>
LuxStatus launch_m(const QmmArgs& a, hipStream_t st) {
    if (a.M <= 64) return LuxStatus::NotSupported;
    return a.has_epilogue() ? launch_e<PluginCfg<TX, BITS, SB, GS, 4>, true>(a, st)
                            : launch_e<PluginCfg<TX, BITS, SB, GS, 4>, false>(a, st);
}

// one activation type and group size (one translation unit each): the code
// width and scale type
template <int TX, int GS>
LuxStatus launch_tg(const QmmArgs& a, hipStream_t st) {
    const bool b8 = a.bits == 8;
    switch (a.sb_dtype) {
    case DT_F32: return b8 ? launch_m<TX, 8, DT_F32, GS>(a, st) : launch_m<TX, 4, DT_F32, GS>(a, st);
    case DT_F16: return b8 ? launch_m<TX, 8, DT_F16, GS>(a, st) : launch_m<TX, 4, DT_F16, GS>(a, st);
    default: return b8 ? launch_m<TX, 8, DT_BF16, GS>(a, st) : launch_m<TX, 4, DT_BF16, GS>(a, st);
    }
}

extern template LuxStatus launch_tg<DT_BF16, 32>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_tg<DT_BF16, 64>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_tg<DT_BF16, 128>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_tg<DT_F16, 32>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_tg<DT_F16, 64>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_tg<DT_F16, 128>(const QmmArgs&, hipStream_t);

}  // namespace rw
}  // namespace lxq
