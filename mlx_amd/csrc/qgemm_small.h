// qgemm_small.h -- MFMA GEMM for 8 < M <= 64 (gfx950): the GEMM semantics
// (weights dequantized to the activation type T, fp32 accumulation) with W
// streamed once from HBM.
//
// A block owns 32 columns n (rows of W) and all of M; its 4 waves split K
// in four parts and meet in LDS at the end (no barrier in the main loop).
// v_mfma_f32_32x32x16_{bf16,f16}: A = x (rows m = lane % 32 of an M tile),
// B = W (column n = lane % 32).  Lane half h = lane / 32 owns the 32 codes
// [64q + 32h, +32) of step q; sub-step s takes codes 32h + 8s .. +8 from both
// halves, so a lane's codes of a step are one contiguous 4*BITS-byte slice,
// dequantized to T (RNE of fmaf(s, q, b)) in registers, and its x operand is
// the matching 16 bytes of row m.
//
// Operands reach the MFMA through LDS, each wave in its own rings (no
// barriers): a fragment load straight from global memory would touch 32
// rows = 32 cache lines per instruction, while a buffer->LDS DMA of 1 KB
// covers 8 lines.  x: one step (MT*32 rows x 128 B) per slot, 16-byte chunks
// XOR-swizzled by row through the DMA source address (conflict-free fragment
// reads); W and scales/biases: four steps per slot.  Each wave waits on a
// compile-time count of its own outstanding DMAs once per step.
#pragma once
#include "kernels.h"
#include "qcommon.h"

namespace lxq {
namespace small {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWaves = 4;
constexpr int kCUs = 256;      // compute units of the MI355X

template <int TX>
__device__ __forceinline__ f32x16 mfma(const u4& a, const u4& b, const f32x16& c) {
    if constexpr (TX == DT_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                      0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                     0, 0, 0);
}

// wait until at most N vector-memory instructions of this wave are in flight
template <int N>
__device__ __forceinline__ void wait_vmcnt_small() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// wait until this wave's LDS reads have returned.  A ring slot is refilled
// by a DMA one step after it was last read, and the compiler may leave one
// of those reads in flight across the refill's issue: an LDS DMA write can
// land before such a queued read executes (measured: stale operands in a
// few blocks per launch, with all 256 CUs busy), so every refill waits for
// the wave's outstanding reads first.
__device__ __forceinline__ void wait_lds_reads() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

template <int SB>
__device__ __forceinline__ float sb_val(uint32_t w) {
    if constexpr (SB == DT_F32) return __uint_as_float(w);
    else if constexpr (SB == DT_F16) return f16_to_f32(w & 0xffffu);
    else return bf16_to_f32(w & 0xffffu);
}
// two fp32 values -> a packed pair of T, RNE, as one packed conversion: a
// scalar (_Float16) cast of an fmaf result lets the compiler fuse both into
// v_fma_mixlo_f16, which rounds once (exact -> f16) where the format rounds
// twice (exact -> fp32 -> f16) and differs at f16 ties
template <int TX>
__device__ __forceinline__ uint32_t pack_t(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    if constexpr (TX == DT_BF16) {
        typedef __bf16 t2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, t2));
    } else {
        typedef _Float16 t2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, t2));
    }
}

// the f16 in the low / high half of a word, as fp32 (v_fma_mix_f32 reads it
// in place when the product feeds an FMA)
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float half_lo(uint32_t m) { return (float)__builtin_bit_cast(f16x2_t, m)[0]; }
__device__ __forceinline__ float half_hi(uint32_t m) { return (float)__builtin_bit_cast(f16x2_t, m)[1]; }

// the 24 bits at bit offset O of a lane's code words (a funnel shift where
// they straddle two words)
template <int O>
__device__ __forceinline__ uint32_t bits24(const uint32_t* c) {
    constexpr int wi = O / 32, sh = O % 32;
    if constexpr (sh + 24 <= 32) return c[wi] >> sh;
    else return __builtin_amdgcn_alignbit(c[wi + 1], c[wi], sh);
}
// a 24-bit group with its low 16 bits kept and bits 12..27 moved to the
// high half: the codes of the group's second half land at the bit positions
// of the first half's codes
__device__ __forceinline__ uint32_t fold24(uint32_t g) { return (g & 0x0000FFFFu) | ((g << 4) & 0xFFFF0000u); }

// codes 8s .. 8s+7 of the lane's 64 (held in 2 BITS words) dequantized to T:
// the B operand of sub-step s.
//
// 3/4/6/8-bit codes: masks leave pairs of codes in place in the two halves
// of a word, i.e. as the f16 subnormals q 2^(p-24) (p = the code's bit
// position within its half, p + BITS <= 10), and v_fma_mix_f32 computes
// fma(s 2^(24-p), q 2^(p-24), b) from them: the product is exactly s q, so
// each value is fmaf(s, q, b), bit for bit, in one instruction instead of a
// convert and an FMA.  (2^(24-p) s is exact for |s| < 2^103: any larger
// scale, from weights of range above ~1e32, would overflow it.)  Other
// widths: a bit-field extract, a convert and an FMA per code.
template <int BITS, int TX>
__device__ __forceinline__ u4 w_operand(const uint32_t* c, float sc, float bi, int s) {
    float q[8];
    if constexpr (BITS == 4) {
        const float s24 = sc * 0x1p24f, s20 = sc * 0x1p20f;
        const uint32_t w = c[s], w8 = w >> 8;
        const uint32_t m0 = w & 0x000F000Fu, m1 = w & 0x00F000F0u;  // codes 0, 4 at p = 0; 1, 5 at p = 4
        const uint32_t m2 = w8 & 0x000F000Fu, m3 = w8 & 0x00F000F0u;  // codes 2, 6; 3, 7
        q[0] = fmaf(s24, half_lo(m0), bi); q[4] = fmaf(s24, half_hi(m0), bi);
        q[1] = fmaf(s20, half_lo(m1), bi); q[5] = fmaf(s20, half_hi(m1), bi);
        q[2] = fmaf(s24, half_lo(m2), bi); q[6] = fmaf(s24, half_hi(m2), bi);
        q[3] = fmaf(s20, half_lo(m3), bi); q[7] = fmaf(s20, half_hi(m3), bi);
    } else if constexpr (BITS == 8) {
        const float s24 = sc * 0x1p24f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t w = c[2 * s + h];
            const uint32_t ma = w & 0x00FF00FFu, mb = (w >> 8) & 0x00FF00FFu;  // codes 0, 2; 1, 3
            q[4 * h] = fmaf(s24, half_lo(ma), bi);     q[4 * h + 2] = fmaf(s24, half_hi(ma), bi);
            q[4 * h + 1] = fmaf(s24, half_lo(mb), bi); q[4 * h + 3] = fmaf(s24, half_hi(mb), bi);
        }
    } else if constexpr (BITS == 3) {
        // one 24-bit group: codes j and 4 + j at p = 3 j (j = 3 shifted to 0)
        const float s24 = sc * 0x1p24f, s21 = sc * 0x1p21f, s18 = sc * 0x1p18f;
        uint32_t g;
        switch (s) {
        case 0: g = bits24<0>(c); break;    case 1: g = bits24<24>(c); break;
        case 2: g = bits24<48>(c); break;   case 3: g = bits24<72>(c); break;
        case 4: g = bits24<96>(c); break;   case 5: g = bits24<120>(c); break;
        case 6: g = bits24<144>(c); break;  default: g = bits24<168>(c); break;
        }
        const uint32_t t = fold24(g);
        const uint32_t m0 = t & 0x00070007u, m1 = t & 0x00380038u, m2 = t & 0x01C001C0u, m3 = (t >> 9) & 0x00070007u;
        q[0] = fmaf(s24, half_lo(m0), bi); q[4] = fmaf(s24, half_hi(m0), bi);
        q[1] = fmaf(s21, half_lo(m1), bi); q[5] = fmaf(s21, half_hi(m1), bi);
        q[2] = fmaf(s18, half_lo(m2), bi); q[6] = fmaf(s18, half_hi(m2), bi);
        q[3] = fmaf(s24, half_lo(m3), bi); q[7] = fmaf(s24, half_hi(m3), bi);
    } else if constexpr (BITS == 6) {
        // two 24-bit groups of 4 codes: codes 0, 2 and (shifted) 1, 3 at p = 0
        const float s24 = sc * 0x1p24f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint32_t g;
            switch (2 * s + h) {
            case 0: g = bits24<0>(c); break;     case 1: g = bits24<24>(c); break;
            case 2: g = bits24<48>(c); break;    case 3: g = bits24<72>(c); break;
            case 4: g = bits24<96>(c); break;    case 5: g = bits24<120>(c); break;
            case 6: g = bits24<144>(c); break;   case 7: g = bits24<168>(c); break;
            case 8: g = bits24<192>(c); break;   case 9: g = bits24<216>(c); break;
            case 10: g = bits24<240>(c); break;  case 11: g = bits24<264>(c); break;
            case 12: g = bits24<288>(c); break;  case 13: g = bits24<312>(c); break;
            case 14: g = bits24<336>(c); break;  default: g = bits24<360>(c); break;
            }
            const uint32_t t = fold24(g);
            const uint32_t ma = t & 0x003F003Fu, mb = (t >> 6) & 0x003F003Fu;
            q[4 * h] = fmaf(s24, half_lo(ma), bi);     q[4 * h + 2] = fmaf(s24, half_hi(ma), bi);
            q[4 * h + 1] = fmaf(s24, half_lo(mb), bi); q[4 * h + 3] = fmaf(s24, half_hi(mb), bi);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) q[e] = fmaf(sc, (float)unit_code<BITS>(c, 8 * s + e), bi);
    }
    u4 r;
    r.x = pack_t<TX>(q[0], q[1]);
    r.y = pack_t<TX>(q[2], q[3]);
    r.z = pack_t<TX>(q[4], q[5]);
    r.w = pack_t<TX>(q[6], q[7]);
    return r;
}

// buffer->LDS DMA, lane l copies E bytes to LDS address m0 + E l (global
// address = SGPR base + 32-bit lane offset; every offset here is in bounds)
__device__ __forceinline__ void dma16(uint32_t m0v, const void* sbase, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" : : "s"(m0v), "v"(voff), "s"(sbase) : "memory", "m0");
}
__device__ __forceinline__ void dma4(uint32_t m0v, const void* sbase, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" : : "s"(m0v), "v"(voff), "s"(sbase) : "memory", "m0");
}

__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// W rows of a super-step slot are 32*BITS bytes = 2*BITS 16-byte chunks
// (half that in a half slot).  Where that count kCpr is a power of two
// (BITS 2, 4, 8) chunk c of row r sits at position c ^ wswz(r) (through the
// DMA source address, like x): the row stride is a multiple of 64 B (256 B
// for 8-bit codes, a whole bank cycle), so without it the 32 lanes reading
// 32 rows' codes hit the same banks (measured at c2: 3.9M conflict cycles
// against 0.3M active LDS cycles).  16 consecutive rows reading one chunk
// then cover 16 distinct 16-byte slots of a 256-byte bank window.
template <int kCpr>
__device__ __forceinline__ int wswz(int r) {
    if constexpr ((kCpr & (kCpr - 1)) == 0 && kCpr <= 16) return (r / (16 / kCpr)) & (kCpr - 1);
    else return 0;
}

template <int BITS, int SB, int MT, int NT, int GS>
struct Lay {
    static constexpr int kSb = SB == DT_F32 ? 4 : 2;
    static constexpr int kXS = MT * 32 * 128;           // one x step
    static constexpr int kRX = MT == 1 ? 3 : 2;         // x steps resident (one being read)
    static constexpr int kSPR = (256 / GS) * kSb;       // scale bytes per row per super-step
    static constexpr int kDpr = kSPR / 4;               // ... in dwords (1..8)
    static constexpr int kNS = (32 * kDpr + 63) / 64;   // DMAs per column tile's scale super-step
    static constexpr int kST = 32 * kSPR;
    static constexpr int kSS = NT * kST;
    static constexpr int kNX = 4 * MT;                  // x DMAs per step
    // Part-super-step W slots (two 6- or 8-bit tiles, whose whole-super-step
    // W slots do not fit twice beside x's): W in a ring of kRWW slots of kSW
    // steps, half (3 slots of 2 steps) or, where that does not fit either,
    // quarter (5 slots of one step) super-steps, one refilled every kSW
    // steps and 4 steps ahead as with two whole slots; scales keep two
    // super-step slots
    static constexpr int kFull = kRX * kXS + 2 * (NT * 32 * 32 * BITS + 2 * kSS);
    static constexpr int kHalf = kRX * kXS + 3 * (NT * 32 * 16 * BITS) + 2 * 2 * kSS;
    static constexpr int kSW = NT != 2 || (BITS != 6 && BITS != 8) || 4 * kFull <= 160 * 1024 ? 4
                               : 4 * kHalf <= 160 * 1024 || BITS != 8                          ? 2
                                                                                               : 1;
    static constexpr bool kHW = kSW < 4;
    static constexpr int kWRow = 8 * BITS * kSW;        // W bytes of a row in a slot
    static constexpr int kWT = 32 * kWRow;              // one column tile's W slot
    static constexpr int kWS = NT * kWT;                // a W slot: the NT column tiles
    static constexpr int kNWI = BITS * kSW / 4;         // W DMAs per column tile and W issue
    static constexpr int kNSS = 2 * NT * kNS;           // scale + bias DMAs per super-step
    static constexpr int kNWS = NT * kNWI + kNSS;       // DMAs of the largest W issue
    // loads younger than X(q) when step q waits: the W DMAs issued in steps
    // q - kRX + 1 .. q and the x DMAs of steps q - kRX + 2 .. q: kRX - 1
    // x issues, a slot's W at most once per kSW steps, one scale super-step
    static constexpr int kMaxWait = (kRX - 1) * kNX + (kRX + kSW - 1) / kSW * NT * kNWI + kNSS;
    // W super-steps resident: 3 (two in flight) unless LDS or vmcnt say 2
    static constexpr int kWaveBytes3 = kRX * kXS + 3 * (kWS + 2 * kSS);
    static constexpr int kRW = (!kHW && 4 * kWaveBytes3 <= 160 * 1024) ? 3 : 2;  // scale slots (and W slots unless kHW)
    static constexpr int kRWW = kSW == 4 ? kRW : kSW == 2 ? 3 : 5;  // W slots
    static constexpr int kLead = kRWW - 1;              // part-super-step slots issued ahead
    static constexpr int kX0 = 0, kW0 = kRX * kXS, kS0 = kW0 + kRWW * kWS, kB0 = kS0 + kRW * kSS;
    static constexpr int kWaveBytes = kB0 + kRW * kSS;
    static constexpr int kRed = 4 * NT * MT * 16 * 64 * 4;  // final K-part reduction (reuses the rings)
    static constexpr int kBytes = (4 * kWaveBytes > kRed) ? 4 * kWaveBytes : kRed;
    static_assert(kMaxWait < 64, "vmcnt holds 6 bits");
    static_assert(kSPR % 4 == 0, "scale rows of a super-step are whole dwords");
    static_assert(BITS * kSW % 4 == 0, "part-super-step slots: whole DMAs per slot");
};

template <int BITS, int SB, int MT, int NT, int GS>
struct Ctx {
    uint32_t lds;                 // LDS address of this wave's rings
    const uint8_t* x;             // x + this wave's first k (bytes)
    const uint8_t* w;             // w_q + this wave's first code (bytes)
    const uint8_t* s;             // scales + this wave's first group (bytes)
    const uint8_t* b;
    uint32_t xoff[4 * MT];        // per x DMA: row (clamped) and swizzled chunk
    uint32_t woff[NT][BITS];      // per column tile and W DMA: row (clamped) and chunk
    uint32_t soff[NT][Lay<BITS, SB, MT, NT, GS>::kNS];
    bool sact[Lay<BITS, SB, MT, NT, GS>::kNS];
};

template <int BITS, int SB, int MT, int NT, int GS>
__device__ __forceinline__ void issue_x(const Ctx<BITS, SB, MT, NT, GS>& c, int qs) {  // qs: step within the part
    using L = Lay<BITS, SB, MT, NT, GS>;
    const uint32_t base = c.lds + L::kX0 + (uint32_t)(qs % L::kRX) * L::kXS;
    const uint8_t* src = c.x + (size_t)qs * 128;
#pragma unroll
    for (int i = 0; i < L::kNX; i++) dma16(base + 1024u * i, src, c.xoff[i]);
}
// part-super-step W (kHW): unit g (steps kSW g .. kSW g + kSW - 1 of the part) into slot g % kRWW
template <int BITS, int SB, int MT, int NT, int GS>
__device__ __forceinline__ void issue_wh(const Ctx<BITS, SB, MT, NT, GS>& c, int g) {
    using L = Lay<BITS, SB, MT, NT, GS>;
    const uint32_t slot = (uint32_t)(g % L::kRWW);
    const uint8_t* src = c.w + (size_t)g * L::kWRow;
#pragma unroll
    for (int ct = 0; ct < NT; ct++)
#pragma unroll
        for (int i = 0; i < L::kNWI; i++)
            dma16(c.lds + L::kW0 + slot * L::kWS + ct * L::kWT + 1024u * i, src, c.woff[ct][i]);
}
// W (unless kHW) and the scales and biases of super-step u into slot u % kRW
template <int BITS, int SB, int MT, int NT, int GS>
__device__ __forceinline__ void issue_w(const Ctx<BITS, SB, MT, NT, GS>& c, int u) {  // u: super-step within the part
    using L = Lay<BITS, SB, MT, NT, GS>;
    const uint32_t slot = (uint32_t)(u % L::kRW);
    if constexpr (!L::kHW) {
        const uint8_t* src = c.w + (size_t)u * 32 * BITS;
#pragma unroll
        for (int ct = 0; ct < NT; ct++)
#pragma unroll
            for (int i = 0; i < BITS; i++)
                dma16(c.lds + L::kW0 + slot * L::kWS + ct * L::kWT + 1024u * i, src, c.woff[ct][i]);
    }
    const uint8_t* ss = c.s + (size_t)u * L::kSPR;
    const uint8_t* bs = c.b + (size_t)u * L::kSPR;
#pragma unroll
    for (int ct = 0; ct < NT; ct++)
#pragma unroll
        for (int i = 0; i < L::kNS; i++) {
            if (c.sact[i]) dma4(c.lds + L::kS0 + slot * L::kSS + ct * L::kST + 256u * i, ss, c.soff[ct][i]);
        }
#pragma unroll
    for (int ct = 0; ct < NT; ct++)
#pragma unroll
        for (int i = 0; i < L::kNS; i++) {
            if (c.sact[i]) dma4(c.lds + L::kB0 + slot * L::kSS + ct * L::kST + 256u * i, bs, c.soff[ct][i]);
        }
}

// DMAs of the W and scale issues among steps q - kRX + 1 .. q (P = q % 4);
// steps before 0 count as the steady state would issue them, which the
// prologue follows
template <class L, int NT, int P>
constexpr int young_w() {
    int n = 0;
    for (int d = 0; d <= L::kRX - 1; d++) {
        const int p = ((P - d) % 4 + 4) % 4;
        if (p % L::kSW == 0) n += NT * L::kNWI;
        if (p == 0) n += L::kNSS;
    }
    return n;
}

// step q (P = q % 4, compile time) of a wave whose part has nq steps
template <int BITS, int TX, int SB, int MT, int NT, int GS, int P>
__device__ __forceinline__ void step(f32x16 (&acc)[NT][MT], const Ctx<BITS, SB, MT, NT, GS>& c, uint8_t* lw, int q,
                                     int nq) {
    using L = Lay<BITS, SB, MT, NT, GS>;
    const int u = q >> 2;
    // issue: x of step q + kRX - 1, then W/scales of super-step u + kRW - 1
    // (at P == 0) (past the part's end they repeat its last step / super-step:
    // counts stay fixed), once the previous step's reads of the refilled slots
    // are done.  x goes first: its wait comes kRX - 1 steps later, W's at
    // least 4 (M = 64, K = 4096, N = 11008, 3-bit: 17.80 -> 17.38 us; 1-2 %
    // on the other shapes measured)
    wait_lds_reads();
    {
        const int qx = q + L::kRX - 1;
        issue_x(c, qx < nq ? qx : nq - 1);
    }
    if constexpr (L::kHW) {
        // unit g + kLead into the slot unit g - 1 used, at the first step of
        // unit g; at P == 0 also the scales of super-step u + 1
        if constexpr (P % L::kSW == 0) {
            const int gw = u * (4 / L::kSW) + P / L::kSW + L::kLead, gl = (nq >> 2) * (4 / L::kSW) - 1;
            issue_wh(c, gw < gl ? gw : gl);
        }
        if constexpr (P == 0) {
            const int uw = u + 1, ul = (nq >> 2) - 1;
            issue_w(c, uw < ul ? uw : ul);
        }
    } else if constexpr (P == 0) {
        const int uw = u + L::kRW - 1, ul = (nq >> 2) - 1;
        issue_w(c, uw < ul ? uw : ul);
    }
    // X(q) (and the older W(u)) landed: younger are the W issues of steps
    // q - kRX + 1 .. q (X(q) went first in step q - kRX + 1) and the x
    // issues of steps q - kRX + 2 .. q
    static_assert(L::kRX >= 2 && L::kRX <= 4, "W issued 4 steps ahead: older than the x awaited");
    // the W issues of those steps: a slot's W at each step with P % kSW == 0,
    // the scales (and, for whole slots, the W) at the one with P == 0
    constexpr int kYoung = (L::kRX - 1) * L::kNX + young_w<L, NT, P>();
    wait_vmcnt_small<kYoung>();
    const int lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
    // x fragments
    const uint8_t* xs = lw + L::kX0 + (q % L::kRX) * L::kXS;
    u4 xf[MT][4];
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const int r = 32 * t + j;
#pragma unroll
        for (int s = 0; s < 4; s++) xf[t][s] = *reinterpret_cast<const u4*>(xs + r * 128 + (((4 * h + s) ^ swz(r)) * 16));
    }
    // codes and scale of this lane's 32 codes in each column tile
    const int slot = u % L::kRW;
    const int wslot = L::kHW ? (u * (4 / L::kSW) + P / L::kSW) % L::kRWW : slot;
    const int wz = wswz<L::kWRow / 16>(j);
    const int gi = (P * 64 + 32 * h) / GS;
    uint32_t cw[NT][BITS];
    float sc[NT], bi[NT];
#pragma unroll
    for (int ct = 0; ct < NT; ct++) {
        const uint8_t* wrow = lw + L::kW0 + wslot * L::kWS + ct * L::kWT + j * L::kWRow;
#pragma unroll
        for (int i = 0; i < BITS; i++) {
            // within the row, before the swizzle (a half slot holds steps 2 (P / 2), + 1)
            const int byte = (P % L::kSW) * 8 * BITS + 4 * BITS * h + 4 * i;
            cw[ct][i] = *reinterpret_cast<const uint32_t*>(wrow + ((((byte >> 4) ^ wz) << 4) | (byte & 15)));
        }
        const uint8_t* sp = lw + L::kS0 + slot * L::kSS + ct * L::kST + j * L::kSPR + gi * L::kSb;
        const uint8_t* bp = lw + L::kB0 + slot * L::kSS + ct * L::kST + j * L::kSPR + gi * L::kSb;
        if constexpr (SB == DT_F32) {
            sc[ct] = *reinterpret_cast<const float*>(sp);
            bi[ct] = *reinterpret_cast<const float*>(bp);
        } else if constexpr (SB == DT_F16) {
            sc[ct] = f16_to_f32(*reinterpret_cast<const uint16_t*>(sp));
            bi[ct] = f16_to_f32(*reinterpret_cast<const uint16_t*>(bp));
        } else {
            sc[ct] = bf16_to_f32(*reinterpret_cast<const uint16_t*>(sp));
            bi[ct] = bf16_to_f32(*reinterpret_cast<const uint16_t*>(bp));
        }
    }
#pragma unroll
    for (int s = 0; s < 4; s++)
#pragma unroll
        for (int ct = 0; ct < NT; ct++) {
            const u4 wop = w_operand<BITS, TX>(cw[ct], sc[ct], bi[ct], s);
#pragma unroll
            for (int t = 0; t < MT; t++) acc[ct][t] = mfma<TX>(xf[t][s], wop, acc[ct][t]);
        }
}

// NT column tiles of 32 per block.  One block per CU (the rings take most
// of the LDS), and a block's time hardly depends on how many blocks run
// beside it: a round of 64 blocks and one of 256 take about the same time
// (M = 64, K = 4096, one tile: 12.2 / 13.4 us), and a second, partial round
// costs a whole one (288 blocks: 23.0 us).  Two tiles per block double a
// block's dequant and MFMA work but halve the block count and x's
// re-reads: slower when one round of one-tile blocks covers N, faster when
// it takes two (the launcher picks).
template <int BITS, int TX, int SB, int MT, int NT, int GS, bool EPI>
__global__ __launch_bounds__(64 * kWaves) void qgemm_small_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, Epilogue ep) {
    using L = Lay<BITS, SB, MT, NT, GS>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 31, h = lane >> 5;
    const int n0 = blockIdx.x * 32 * NT;
    const int G = K / GS;
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    const int nq = K / 64 / kWaves;        // steps of this wave's K part (a multiple of 4)
    const int k0 = wave * nq * 64;         // first k of the part

    Ctx<BITS, SB, MT, NT, GS> c;
    c.lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds) + (uint32_t)wave * L::kWaveBytes;
    c.x = static_cast<const uint8_t*>(x) + (size_t)k0 * 2;
    c.w = reinterpret_cast<const uint8_t*>(wq) + (size_t)k0 * BITS / 8;
    c.s = static_cast<const uint8_t*>(scales) + (size_t)(k0 / GS) * L::kSb;
    c.b = static_cast<const uint8_t*>(biases) + (size_t)(k0 / GS) * L::kSb;
#pragma unroll
    for (int i = 0; i < L::kNX; i++) {
        const int r = 8 * i + (lane >> 3);                       // row within the MT*32 rows
        const int m = r < M ? r : M - 1;
        const int chunk = (lane & 7) ^ swz(r);                   // global chunk landing in slot lane & 7
        c.xoff[i] = ((uint32_t)m * K + 8 * chunk) * 2;
    }
#pragma unroll
    for (int ct = 0; ct < NT; ct++) {
#pragma unroll
        for (int i = 0; i < L::kNWI; i++) {
            constexpr int kCpr = L::kWRow / 16;                   // 16-byte chunks of a row in a slot
            const int v = 64 * i + lane, r = v / kCpr, ch = v % kCpr;
            const int n = n0 + 32 * ct + r < N ? n0 + 32 * ct + r : N - 1;
            c.woff[ct][i] = (uint32_t)n * row_bytes + 16u * (ch ^ wswz<kCpr>(r));  // lands at position ch
        }
#pragma unroll
        for (int i = 0; i < L::kNS; i++) {
            const int v = 64 * i + lane, r = v / L::kDpr, d = v % L::kDpr;
            const int n = n0 + 32 * ct + r < N ? n0 + 32 * ct + r : N - 1;
            c.sact[i] = v < 32 * L::kDpr;
            c.soff[ct][i] = (uint32_t)n * G * L::kSb + 4u * d;
        }
    }
    uint8_t* lw = lds + (size_t)wave * L::kWaveBytes;

    // prologue: the issues of steps -kRX+1 .. -1 and super-steps up to kRW - 2
    // in the order the steady state keeps, which the waits of steps 0 ..
    // kRX - 2 count on: first what it issues before step -kRX + 1 (the W and
    // scale slots, the part-super-step units g with (g - kLead) kSW < 1 - kRX),
    // then step s = -kRX + 1 .. -1: x of step s + kRX - 1, then the unit of s
    // where s % kSW == 0.  (All units issued ahead of x once let step 0 of
    // 8-bit, f32-scale, group-32 tiles read x before it landed.)
    if constexpr (L::kHW) {
#pragma unroll
        for (int g = 0; g < L::kLead; g++)  // a part has at least one super-step: 4 / kSW units
            if ((g - L::kLead) * L::kSW < 1 - L::kRX) issue_wh(c, g);
    }
#pragma unroll
    for (int uu = 0; uu < L::kRW - 1; uu++) issue_w(c, uu < (nq >> 2) - 1 ? uu : (nq >> 2) - 1);
#pragma unroll
    for (int qq = 0; qq < L::kRX - 1; qq++) {
        issue_x(c, qq < nq - 1 ? qq : nq - 1);
        if constexpr (L::kHW) {
            constexpr int s0 = 1 - L::kRX;  // step of x(qq) is s0 + qq
            if ((s0 + qq) % L::kSW == 0) issue_wh(c, (s0 + qq) / L::kSW + L::kLead);
        }
    }
    // the steady state's W issue of super-step kRW - 1 happens in step 0

    f32x16 acc[NT][MT];
#pragma unroll
    for (int ct = 0; ct < NT; ct++)
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[ct][t][v] = 0.f;
    for (int q = 0; q < nq; q += 4) {
        step<BITS, TX, SB, MT, NT, GS, 0>(acc, c, lw, q, nq);
        step<BITS, TX, SB, MT, NT, GS, 1>(acc, c, lw, q + 1, nq);
        step<BITS, TX, SB, MT, NT, GS, 2>(acc, c, lw, q + 2, nq);
        step<BITS, TX, SB, MT, NT, GS, 3>(acc, c, lw, q + 3, nq);
    }
    wait_vmcnt_small<0>();
    __syncthreads();

    // ---- the four K parts meet in LDS; wave w stores accumulator VGPRs 4w..4w+3 ----
    constexpr int kAcc = NT * MT * 16;            // accumulator VGPRs per lane
    float* red = reinterpret_cast<float*>(lds);   // [wave][kAcc][64]
#pragma unroll
    for (int ct = 0; ct < NT; ct++)
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int v = 0; v < 16; v++)
                red[((size_t)wave * kAcc + (ct * MT + t) * 16 + v) * 64 + lane] = acc[ct][t][v];
    __syncthreads();
#pragma unroll
    for (int ct = 0; ct < NT; ct++) {
        const int nn = n0 + 32 * ct + j;
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int vv = 0; vv < 4; vv++) {
                const int v = 4 * wave + vv;
                float sum = 0.f;
#pragma unroll
                for (int w2 = 0; w2 < kWaves; w2++)
                    sum += red[((size_t)w2 * kAcc + (ct * MT + t) * 16 + v) * 64 + lane];
                // 32x32 accumulator layout: column lane % 32, row 8 (v / 4) + 4 (lane / 32) + v % 4
                const int m = 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
                if (m < M && nn < N) store_out<EPI>(y, (size_t)m * N + nn, nn, ep, sum);
            }
    }
}

// whether two column tiles per block fit: both tiles' W rings beside x's
template <int BITS, int SB, int MT, int GS>
constexpr bool small_nt2_fits() {
    return 4 * Lay<BITS, SB, MT, 2, GS>::kWaveBytes <= 160 * 1024;
}

template <int BITS, int TX, int SB, int MT, int NT, int GS, bool EPI>
LuxStatus launch_e(const QmmArgs& a, hipStream_t st) {
    using L = Lay<BITS, SB, MT, NT, GS>;
    static_assert(L::kBytes <= 160 * 1024, "LDS");
    if (planned(a, "qgemm_small_kernel")) return LuxStatus::Ok;
    auto kern = qgemm_small_kernel<BITS, TX, SB, MT, NT, GS, EPI>;
    // once per instantiation; a function-local static initializes exactly once
    // even when several threads make the first call together
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes);
    if (attr != hipSuccess) return LuxStatus::Internal;
    hipLaunchKernelGGL(kern, dim3((a.N + 32 * NT - 1) / (32 * NT)), dim3(64 * kWaves), L::kBytes, st, a.x, a.wq,
                       a.scales, a.biases, a.y, a.M, a.K, a.N, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

template <int BITS, int TX, int SB, int MT, int NT, int GS>
LuxStatus launch_nt(const QmmArgs& a, hipStream_t st) {
    return a.has_epilogue() ? launch_e<BITS, TX, SB, MT, NT, GS, true>(a, st)
                            : launch_e<BITS, TX, SB, MT, NT, GS, false>(a, st);
}

// two tiles per block where one-tile blocks would need a second round on the
// kCUs CUs (M = 64, K = 4096, 4-bit: N = 11008 17.3 us against 22.6, N =
// 16384 22.8 against 26.9; N = 8192 16.0 against 13.1 stays one tile)
template <int BITS, int TX, int SB, int MT, int GS>
LuxStatus launch(const QmmArgs& a, hipStream_t st) {
    if constexpr (small_nt2_fits<BITS, SB, MT, GS>()) {
        if ((a.N + 31) / 32 > kCUs) return launch_nt<BITS, TX, SB, MT, 2, GS>(a, st);
    }
    return launch_nt<BITS, TX, SB, MT, 1, GS>(a, st);
}

template <int BITS, int TX, int SB, int MT>
LuxStatus launch_gs(const QmmArgs& a, hipStream_t st) {
    switch (a.group_size) {
    case 32: return launch<BITS, TX, SB, MT, 32>(a, st);
    case 64: return launch<BITS, TX, SB, MT, 64>(a, st);
    default: return launch<BITS, TX, SB, MT, 128>(a, st);
    }
}

template <int BITS, int TX, int SB>
LuxStatus launch_mt(const QmmArgs& a, hipStream_t st) {
    return a.M <= 32 ? launch_gs<BITS, TX, SB, 1>(a, st) : launch_gs<BITS, TX, SB, 2>(a, st);
}

template <int BITS, int TX>
LuxStatus launch_sb(const QmmArgs& a, hipStream_t st) {
    switch (a.sb_dtype) {
    case DT_F32: return launch_mt<BITS, TX, DT_F32>(a, st);
    case DT_F16: return launch_mt<BITS, TX, DT_F16>(a, st);
    default: return launch_mt<BITS, TX, DT_BF16>(a, st);
    }
}

// one explicit instantiation per code width, each in its own translation
// unit (qgemm_small_b{2,3,4,5,6,8}.hip)
template <int BITS>
LuxStatus launch_tx(const QmmArgs& a, hipStream_t st) {
    return a.x_dtype == DT_F16 ? launch_sb<BITS, DT_F16>(a, st) : launch_sb<BITS, DT_BF16>(a, st);
}

}  // namespace small

// launcher (qgemm_small.hip): NotSupported unless 8 < M <= 64, f16/bf16 x, K % 1024 == 0
LuxStatus launch_qgemm_small(const QmmArgs& a, hipStream_t st);

}  // namespace lxq
