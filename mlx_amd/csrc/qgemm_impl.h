// qgemm_impl.h -- compute-bound dequant GEMM for large M (gfx950, MFMA): kernel templates.
//
// y[M, N] = x[M, K] . T(w_hat)[N, K]^T,  T = the activation type (bf16/f16):
// each K step of 64 codes, the block dequantizes its W tile exactly
// (w_hat = fmaf(scale, q, bias) in fp32, rounded RNE to T) into LDS and runs
// v_mfma_f32_32x32x16_{bf16,f16} with fp32 accumulation.  This is the
// "dequantize to the activation type, then matmul" semantics.
//
// Block tile 256 (M) x 128 (N), 8 waves (two per SIMD) as 4 x 2, wave tile
// 64 x 64 = 2 x 2 MFMA tiles of 32 x 32.  Every wave also dequantizes 16
// codes of one W row per K step.
//
// All operands reach LDS by direct global->LDS transfers (global_load_lds):
// x tiles (all waves), packed W (waves 0..3) and scale/bias windows (waves
// 4..7).  No vector-memory load lands in registers inside the K loop, so the
// compiler adds no waits of its own and the explicit per-step waits count
// every transfer in flight; the two wave roles are separate compile-time
// code paths with their own constant waits.
//
// LDS: three x stages (256 rows x 64 k, 32 KB each), two dequantized W
// stages (128 rows x 64 k, 16 KB each), three packed W slots (one K step
// each) and two scale windows (4 K steps each).  x and dequantized-W rows
// are 128 B; 16-byte chunk c of row r sits at position c ^ swz(r), which
// makes the fragment reads (16 lanes = 16 consecutive rows, one chunk), the
// dequant writes (same shape) and the direct x writes (contiguous) free of
// bank conflicts for 8- and 16-lane LDS passes alike.
//
// Pipeline: x and packed W run two K steps ahead (x(k+2) and W(k+3) are
// issued at step k), scale windows one window ahead; GS = group size is a
// template parameter so a window is a compile-time shape (K must be a
// multiple of 256).  While the MFMAs of step k run, step k+1 is
// dequantized into the other W stage in two halves between them: one
// barrier per K step.
//
// Grid: one block per tile, M-tile fastest.  Blocks are dealt round-robin to
// the 8 XCDs, so with 8 M-tiles (M = 2048) every XCD owns one 256-row slab of
// x and keeps it in its own L2 while it walks the N-tiles.  When the tiles
// leave a last round at most half full (tiles % 256 in 1..128, e.g. 896
// tiles at M = 2048, N = 14336: 3.5 rounds), each tile of that round is run
// by two blocks over the two halves of K, so the last round fills the CUs
// and takes half as long; the two halves' fp32 sums meet in the workspace
// (the second block to finish adds the first's partial tile to its own --
// one fp32 addition per value, the same whichever finishes first -- and
// stores y).
#pragma once
#include "kernels.h"
#include "qcommon.h"
#include "qsplit.h"

namespace lxq {
namespace gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
// 16-byte aligned vector for LDS and buffer loads
typedef uint32_t v4 __attribute__((ext_vector_type(4), aligned(16)));
typedef uint32_t v3 __attribute__((ext_vector_type(3)));
typedef uint32_t v2 __attribute__((ext_vector_type(2)));

constexpr int BM = 256, BN = 128, BK = 64;
constexpr int kThreads = 512;  // 8 waves: two per SIMD
constexpr int kXStageBytes = BM * BK * 2;  // 32768
constexpr int kXStages = 3;
constexpr int kWStageBytes = BN * BK * 2;  // 16384
// tail split: CUs of the target (MI355X: 256); the workspace layout and the
// protocol of the split tiles are qsplit.h's
constexpr int kCUs = 256;
constexpr uint32_t kSplitSlotBytes = BM * BN * 4;  // one K half of one tile, fp32
static_assert(split::kPartOffset + (size_t)kCUs / 2 * kSplitSlotBytes <= kSplitWorkspaceBytes, "workspace size");
static_assert(kCUs / 2 <= split::kMaxHalfTiles, "split tiles within the workspace's counter words");

// chunk position permutation of LDS row r (bijective on the 8 chunks; rows
// r and r + 8 get different permutations)
__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// two fp32 values -> packed pair of T, RNE (one v_cvt_pk_{bf16,f16}_f32)
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <int TX>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (TX == DT_BF16)
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2_t));
    else
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), f16x2_t));
}

// 8 codes (8c .. 8c+7) of a 32-code half unit held in BITS words, as fp32.
// 4-bit and 8-bit codes are spread to bytes for v_cvt_f32_ubyte{0..3};
// other widths extract each code with a bitfield op.
template <int BITS>
__device__ __forceinline__ void codes8(const uint32_t* w, int c, float* q) {
    if constexpr (BITS == 4) {
        const uint32_t lo = w[c] & 0x0F0F0F0Fu, hi = (w[c] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            q[2 * j] = (float)((lo >> (8 * j)) & 0xffu);
            q[2 * j + 1] = (float)((hi >> (8 * j)) & 0xffu);
        }
    } else if constexpr (BITS == 8) {
#pragma unroll
        for (int j = 0; j < 8; j++) q[j] = (float)((w[2 * c + (j >> 2)] >> (8 * (j & 3))) & 0xffu);
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int i = 8 * c + j, bit = i * BITS, wi = bit >> 5, sh = bit & 31;
            const uint32_t mask = (1u << BITS) - 1u;
            // a code straddling two words: funnel shift (v_alignbit_b32), which
            // keeps the words in registers (a 64-bit shift invites the
            // compiler to combine them into a 64-bit access of a memory copy)
            const uint32_t v = (sh + BITS <= 32) ? (w[wi] >> sh) & mask
                                                 : __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & mask;
            q[j] = (float)v;
        }
    }
}

template <int TX>
__device__ __forceinline__ f32x16 mfma(const v4& a, const v4& b, const f32x16& c) {
    if constexpr (TX == DT_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// buffer resource over [p, p + bytes): 32-bit offsets, reads past the end return 0
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}

// ---- LDS layout ----------------------------------------------------------
//
// [x stage 0..2: 256 rows x 128 B][dequantized W stage 0..1: 128 rows x 128 B]
// [packed W slot 0..2: one K step, 128 rows x 8 BITS B, rows contiguous]
// [scale window slot 0..1: 4 K steps; per 32-row quarter q: scales of its
//  32 rows, then biases, each row kRowBytes]

template <int BITS>
constexpr int pack_row_bytes() { return 8 * BITS; }  // 64 codes
template <int BITS>
constexpr int pack_slot_bytes() { return BN * pack_row_bytes<BITS>(); }
constexpr int kPackSlots = 3;

template <int GS, int SB>
struct Win {
    static constexpr int kSb = SB == DT_F32 ? 4 : 2;
    static constexpr int kGroups = 256 / GS;          // groups in 4 K steps
    static constexpr int kRowBytes = kGroups * kSb;   // 4 .. 32
    static constexpr int kWords = kRowBytes / 4;      // 1 .. 8
    static constexpr int kSlotBytes = 2 * BN * kRowBytes;
};

template <int BITS, int GS, int SB>
constexpr size_t lds_bytes() {
    return (size_t)kXStages * kXStageBytes + 2 * (size_t)kWStageBytes +
           (size_t)kPackSlots * pack_slot_bytes<BITS>() + 2 * (size_t)Win<GS, SB>::kSlotBytes;
}
constexpr size_t kMaxLds = 160 * 1024;

// the combinations whose buffers fit one CU's LDS (all but f32 scales at
// group size 32 with 6- or 8-bit codes)
template <int BITS, int GS, int SB>
constexpr bool lds_fits() { return lds_bytes<BITS, GS, SB>() <= kMaxLds; }

// ---- direct-to-LDS transfers (global_load_lds) ----------------------------
//
// Lane l copies E bytes to LDS address m0 + E l.  Issued through inline asm:
// the compiler's wait-count pass would otherwise wait for these LDS writes
// before every LDS read, prefetch included.  No other vector-memory load is
// issued inside the K loop, so the explicit waits (wait_vmcnt) are the only
// ones, and they count exactly.

__device__ __forceinline__ void dma16(uint32_t m0v, const void* sbase, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(m0v), "v"(voff), "s"(sbase)
                 : "memory", "m0");
}

__device__ __forceinline__ void dma4(uint32_t m0v, const void* sbase, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2"
                 :
                 : "s"(m0v), "v"(voff), "s"(sbase)
                 : "memory", "m0");
}

// per-lane 64-bit address
__device__ __forceinline__ void dma4a(uint32_t m0v, const void* addr) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off"
                 :
                 : "s"(m0v), "v"(addr)
                 : "memory", "m0");
}

// wait until at most N vector-memory instructions of this wave are in flight
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N < 64, "vmcnt has 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// packed W of one K step by waves 0..3: wave w copies rows 32 w .. 32 w + 31
// (32 x 8 BITS contiguous bytes of LDS) in kInstr transfers of E bytes/lane
template <int BITS>
struct WDma {
    static constexpr int E = (BITS % 4 == 0) ? 16 : 4;
    static constexpr int kWaveBytes = 32 * pack_row_bytes<BITS>();
    static constexpr int kInstr = kWaveBytes / (64 * E);  // 2 3 1 5 6 2 for BITS 2 3 4 5 6 8
    static_assert(kWaveBytes % (64 * E) == 0 && pack_row_bytes<BITS>() % E == 0, "W transfer shape");
};

// ---- fragments and MFMA ----------------------------------------------------

struct Frags {
    v4 a[2], b[2];
};

// fragments of k sub-step ks: A from x stage X (rows a_row + 32 i), B from W
// stage Wt (rows b_row + 32 j); lane reads 16-byte chunk 2 ks + kh at byte
// offset chk within the row (all rows a lane reads share swz)
__device__ __forceinline__ void read_frags(Frags& f, const uint8_t* X, const uint8_t* Wt, int a_row,
                                           int b_row, int chk) {
#pragma unroll
    for (int i = 0; i < 2; i++) f.a[i] = *reinterpret_cast<const v4*>(X + (a_row + 32 * i) * 128 + chk);
#pragma unroll
    for (int j = 0; j < 2; j++) f.b[j] = *reinterpret_cast<const v4*>(Wt + (b_row + 32 * j) * 128 + chk);
}

template <int TX>
__device__ __forceinline__ void mfmas(f32x16 (&acc)[2][2], const Frags& f) {
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = mfma<TX>(f.a[i], f.b[j], acc[i][j]);
}

// ---- dequantization: every thread, 16 codes of one row per K step --------
//
// Thread (wave w, lane l) takes row r = 16 w + l % 16 and codes
// [16 cp, 16 cp + 16), cp = l / 16, i.e. 16-byte chunks 2 cp and 2 cp + 1 of
// the dequantized row: 16 consecutive lanes write 16 consecutive rows.

// LDS words holding the 16 codes (a 16-bit shift aligns them for odd BITS)
template <int BITS>
constexpr int raw_words() {
    return BITS == 2 ? 1 : BITS == 3 ? 2 : BITS == 4 ? 2 : BITS == 5 ? 3 : BITS == 6 ? 3 : 4;
}

template <int BITS>
__device__ __forceinline__ void read_raw(const uint8_t* pk, int r, int cp, uint32_t (&w)[raw_words<BITS>()]) {
    // bit offset of the codes in the row: 16 cp BITS; dword aligned for even BITS
    const uint32_t* row = reinterpret_cast<const uint32_t*>(pk + r * pack_row_bytes<BITS>());
    const int d0 = (16 * cp * BITS) >> 5;
#pragma unroll
    for (int i = 0; i < raw_words<BITS>(); i++) w[i] = row[d0 + i];
}

// 16 codes as fp32, from the raw words (shifted right by 16 for odd BITS and odd cp)
template <int BITS>
__device__ __forceinline__ void decode16(const uint32_t (&raw)[raw_words<BITS>()], int cp, float (&q)[16]) {
    constexpr int NR = raw_words<BITS>();
    uint32_t w[NR];
    if constexpr (BITS & 1) {
        const int sh = (cp & 1) << 4;
#pragma unroll
        for (int i = 0; i + 1 < NR; i++) w[i] = __builtin_amdgcn_alignbit(raw[i + 1], raw[i], sh);
        w[NR - 1] = raw[NR - 1] >> sh;
    } else {
#pragma unroll
        for (int i = 0; i < NR; i++) w[i] = raw[i];
    }
    if constexpr (BITS == 4) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                q[8 * i + 2 * j] = (float)((lo >> (8 * j)) & 0xffu);
                q[8 * i + 2 * j + 1] = (float)((hi >> (8 * j)) & 0xffu);
            }
        }
    } else if constexpr (BITS == 8) {
#pragma unroll
        for (int j = 0; j < 16; j++) q[j] = (float)((w[j >> 2] >> (8 * (j & 3))) & 0xffu);
    } else {
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int bit = j * BITS, wi = bit >> 5, s = bit & 31;
            constexpr uint32_t mask = (1u << BITS) - 1u;
            // a code straddling two words: funnel shift (v_alignbit_b32)
            const uint32_t v = (s + BITS <= 32) ? (w[wi] >> s) & mask
                                                : __builtin_amdgcn_alignbit(w[wi + 1], w[wi], s) & mask;
            q[j] = (float)v;
        }
    }
}

template <int SB>
__device__ __forceinline__ float sb_load(const uint8_t* p) {
    if constexpr (SB == DT_F32) return *reinterpret_cast<const float*>(p);
    else if constexpr (SB == DT_F16) return f16_to_f32(*reinterpret_cast<const uint16_t*>(p));
    else return bf16_to_f32(*reinterpret_cast<const uint16_t*>(p));
}

// scale and bias of the thread's codes in window step J
template <int GS, int SB, int J>
__device__ __forceinline__ void read_sb(const uint8_t* win, int r, int cp, float& s, float& b) {
    using Wn = Win<GS, SB>;
    const int i = (J * 64 + 16 * cp) / GS;  // group within the window
    const uint8_t* p = win + (r >> 5) * (2 * 32 * Wn::kRowBytes) + (r & 31) * Wn::kRowBytes + i * Wn::kSb;
    s = sb_load<SB>(p);
    b = sb_load<SB>(p + 32 * Wn::kRowBytes);
}

// half h: chunk 2 cp + h of row r = codes 8 h .. 8 h + 7 of the 16, as
// fmaf(s, q, b) rounded RNE to TX, into W stage D
template <int TX>
__device__ __forceinline__ void deq_half(const float (&q)[16], float s, float b, uint8_t* D, int r, int cp,
                                         int h) {
    v4 o;
    o.x = pack2<TX>(fmaf(s, q[8 * h + 0], b), fmaf(s, q[8 * h + 1], b));
    o.y = pack2<TX>(fmaf(s, q[8 * h + 2], b), fmaf(s, q[8 * h + 3], b));
    o.z = pack2<TX>(fmaf(s, q[8 * h + 4], b), fmaf(s, q[8 * h + 5], b));
    o.w = pack2<TX>(fmaf(s, q[8 * h + 6], b), fmaf(s, q[8 * h + 7], b));
    *reinterpret_cast<v4*>(D + r * 128 + (((2 * cp + h) ^ swz(r)) << 4)) = o;
}

// ---- the K loop ------------------------------------------------------------

// everything a K step needs besides the accumulators
struct Ctx {
    uint8_t* lds;
    uint32_t lds_addr;  // LDS address of lds (low 32 bits of the flat address)
    const uint16_t* x;
    const uint32_t* wq;
    uint32_t xoff[4];   // byte offset (in x) of this lane's 4 x chunks, K step 0
    int wave, lane, KT, n0, N, G;
    int k0;             // the block's first K step (K steps k0 .. k0 + KT - 1)
    uint32_t row_bytes;
    int a_row, b_row;
    int chk[4];         // byte offset of this lane's fragment chunk, per k sub-step
    int dr, dcp;        // dequantization: row and code quarter
};

template <int BITS, int GS, int SB>
struct Off {
    static constexpr int kX = 0;
    static constexpr int kW = kXStages * kXStageBytes;
    static constexpr int kPack = kW + 2 * kWStageBytes;
    static constexpr int kWin = kPack + kPackSlots * pack_slot_bytes<BITS>();
};

// x tile of K step kt into x stage xs: wave w, instruction i fills the 1 KB
// block of rows 8 (4 w + i) .. +8
__device__ __forceinline__ void load_x(const Ctx& t, int xs, int kt) {
    const uint32_t base = t.lds_addr + (uint32_t)xs * kXStageBytes + (uint32_t)t.wave * 4096u;
#pragma unroll
    for (int i = 0; i < 4; i++) dma16(base + 1024u * i, t.x, t.xoff[i] + (uint32_t)kt * BK * 2);
}

// K step kt (P = kt % 4).  x stage kt % 3 and W stage kt % 2 hold step kt;
// packed slot (kt+1) % 3 and window slot ((kt+1) / 4) % 2 hold the codes and
// scales of step kt+1.  Issue x(kt+2) into x stage (kt+2) % 3; waves 0..3
// (ROLE 0) issue the packed W of step kt+3 into slot kt % 3, waves 4..7
// (ROLE 1) at P = 0 the scale window of steps kt+4 .. kt+7.  Then the MFMAs
// of step kt with the dequantization of step kt+1 into W stage (kt+1) % 2,
// the wait, the barrier.  At the wait, ROLE 0 needs x(kt+1) and W(kt+2)
// (issued at step kt-1) landed: in flight may stay x(kt+2), W(kt+3).  ROLE 1
// needs x(kt+1): in flight may stay x(kt+2), the window of step kt (P = 0)
// and the one of step kt-1 (P = 1), which is first read at step kt+3 after
// the barrier of step kt+2.  Loads past the last step re-read the last step
// or window (never used), so every step issues the same loads.
template <int TX, int BITS, int SB, int GS, int ROLE, int P>
__device__ __forceinline__ void ring_step(f32x16 (&acc)[2][2], const Ctx& t, const uint32_t* wv,
                                          const uint8_t* const* sp, int kt) {
    using Lo = Off<BITS, GS, SB>;
    using Wn = Win<GS, SB>;
    const int xi = kt % 3;
    load_x(t, xi == 0 ? 2 : xi - 1, min(kt + 2, t.KT - 1));
    if constexpr (ROLE == 0) {
        // packed W of step kt+3 into slot kt % 3
        using WD = WDma<BITS>;
        const uint32_t base = t.lds_addr + Lo::kPack + (uint32_t)xi * pack_slot_bytes<BITS>() +
                              (uint32_t)t.wave * WD::kWaveBytes;
        const uint32_t koff = (uint32_t)min(kt + 3, t.KT - 1) * pack_row_bytes<BITS>();
#pragma unroll
        for (int j = 0; j < WD::kInstr; j++) {
            if constexpr (WD::E == 16) dma16(base + 64u * 16u * j, t.wq, wv[j] + koff);
            else dma4(base + 64u * 4u * j, t.wq, wv[j] + koff);
        }
    } else if constexpr (P == 0) {
        // scale window of steps kt+4 .. kt+7 into window slot (kt/4 + 1) % 2
        const int wi = min(kt / 4 + 1, t.KT / 4 - 1);
        const uint32_t base = t.lds_addr + Lo::kWin + (uint32_t)(((kt >> 2) + 1) & 1) * Wn::kSlotBytes +
                              (uint32_t)(t.wave - 4) * (2 * 32 * Wn::kRowBytes);
        const size_t goff = (size_t)wi * Wn::kRowBytes;
#pragma unroll
        for (int j = 0; j < Wn::kWords; j++) dma4a(base + 256u * j, sp[j] + goff);
    }
    const uint8_t* X = t.lds + Lo::kX + xi * kXStageBytes;
    const uint8_t* Wt = t.lds + Lo::kW + (P & 1) * kWStageBytes;
    uint8_t* D = t.lds + Lo::kW + ((P + 1) & 1) * kWStageBytes;
    const uint8_t* pk = t.lds + Lo::kPack + ((kt + 1) % 3) * pack_slot_bytes<BITS>();
    const uint8_t* win = t.lds + Lo::kWin + (((kt + 1) >> 2) & 1) * Wn::kSlotBytes;

    // MFMAs of step kt (fragments of sub-step ks+1 read while ks runs); the
    // dequantization of step kt+1 in two halves between them
    Frags f0, f1;
    read_frags(f0, X, Wt, t.a_row, t.b_row, t.chk[0]);
    uint32_t raw[raw_words<BITS>()];
    read_raw<BITS>(pk, t.dr, t.dcp, raw);
    float s, b;
    read_sb<GS, SB, (P + 1) & 3>(win, t.dr, t.dcp, s, b);
    read_frags(f1, X, Wt, t.a_row, t.b_row, t.chk[1]);
    mfmas<TX>(acc, f0);
    read_frags(f0, X, Wt, t.a_row, t.b_row, t.chk[2]);
    float q[16];
    decode16<BITS>(raw, t.dcp, q);
    mfmas<TX>(acc, f1);
    deq_half<TX>(q, s, b, D, t.dr, t.dcp, 0);
    read_frags(f1, X, Wt, t.a_row, t.b_row, t.chk[3]);
    mfmas<TX>(acc, f0);
    deq_half<TX>(q, s, b, D, t.dr, t.dcp, 1);
    mfmas<TX>(acc, f1);

    if constexpr (ROLE == 0) wait_vmcnt<4 + WDma<BITS>::kInstr>();
    else wait_vmcnt<4 + Wn::kWords * ((P == 0) + (P == 1))>();
    __syncthreads();
}

// prologue and K loop of one wave role
template <int TX, int BITS, int SB, int GS, int ROLE>
__device__ __forceinline__ void main_loop(f32x16 (&acc)[2][2], const Ctx& t, const void* scales,
                                          const void* biases) {
    using Lo = Off<BITS, GS, SB>;
    using Wn = Win<GS, SB>;
    using WD = WDma<BITS>;
    // per-lane global offsets of this role's transfers
    uint32_t wv[ROLE == 0 ? WD::kInstr : 1];
    const uint8_t* sp[ROLE == 1 ? Wn::kWords : 1];
    if constexpr (ROLE == 0) {
#pragma unroll
        for (int j = 0; j < WD::kInstr; j++) {
            const int off = 64 * WD::E * j + WD::E * t.lane;  // byte in the wave's 32 rows
            const int row = off / pack_row_bytes<BITS>(), byte = off % pack_row_bytes<BITS>();
            const int n = min(t.n0 + 32 * t.wave + row, t.N - 1);  // rows past N: valid data, never stored
            wv[j] = (uint32_t)n * t.row_bytes + (uint32_t)t.k0 * pack_row_bytes<BITS>() + (uint32_t)byte;
        }
    } else {
#pragma unroll
        for (int j = 0; j < Wn::kWords; j++) {
            const int d = 64 * j + t.lane;  // dword of the quarter's window part
            const int a = d / (32 * Wn::kWords), rem = d % (32 * Wn::kWords);
            const int row = rem / Wn::kWords, word = rem % Wn::kWords;
            const int n = min(t.n0 + 32 * (t.wave - 4) + row, t.N - 1);
            sp[j] = static_cast<const uint8_t*>(a ? biases : scales) + (size_t)n * t.G * Wn::kSb +
                    (size_t)(t.k0 / 4) * Wn::kRowBytes + 4 * word;
        }
    }

    // prologue: x of steps 0, 1; packed W of steps 0..2 (slots 0..2); scale
    // window 0 (slot 0); then step 0 dequantized into W stage 0
    load_x(t, 0, 0);
    load_x(t, 1, 1);
    if constexpr (ROLE == 0) {
#pragma unroll
        for (int st = 0; st < 3; st++) {
            const uint32_t base = t.lds_addr + Lo::kPack + (uint32_t)st * pack_slot_bytes<BITS>() +
                                  (uint32_t)t.wave * WD::kWaveBytes;
#pragma unroll
            for (int j = 0; j < WD::kInstr; j++) {
                const uint32_t v = wv[j] + (uint32_t)st * pack_row_bytes<BITS>();
                if constexpr (WD::E == 16) dma16(base + 64u * 16u * j, t.wq, v);
                else dma4(base + 64u * 4u * j, t.wq, v);
            }
        }
    } else {
        const uint32_t base = t.lds_addr + Lo::kWin + (uint32_t)(t.wave - 4) * (2 * 32 * Wn::kRowBytes);
#pragma unroll
        for (int j = 0; j < Wn::kWords; j++) dma4a(base + 256u * j, sp[j]);
    }
    wait_vmcnt<0>();
    __syncthreads();
    {
        uint32_t raw[raw_words<BITS>()];
        read_raw<BITS>(t.lds + Lo::kPack, t.dr, t.dcp, raw);
        float s, b, q[16];
        read_sb<GS, SB, 0>(t.lds + Lo::kWin, t.dr, t.dcp, s, b);
        decode16<BITS>(raw, t.dcp, q);
        deq_half<TX>(q, s, b, t.lds + Lo::kW, t.dr, t.dcp, 0);
        deq_half<TX>(q, s, b, t.lds + Lo::kW, t.dr, t.dcp, 1);
    }
    __syncthreads();

    // KT is a multiple of 4 (K % 256 == 0)
    for (int kt = 0; kt < t.KT; kt += 4) {
        ring_step<TX, BITS, SB, GS, ROLE, 0>(acc, t, wv, sp, kt);
        ring_step<TX, BITS, SB, GS, ROLE, 1>(acc, t, wv, sp, kt + 1);
        ring_step<TX, BITS, SB, GS, ROLE, 2>(acc, t, wv, sp, kt + 2);
        ring_step<TX, BITS, SB, GS, ROLE, 3>(acc, t, wv, sp, kt + 3);
    }
    // no LDS transfer may still be landing when the block's LDS is released
    wait_vmcnt<0>();
}

template <int TX, int BITS, int SB, int GS, bool EPI>
__global__ __launch_bounds__(kThreads, 2) void qgemm_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, Epilogue ep,
    int mtiles, int split_from, void* __restrict__ ws, uint32_t epoch) {
    static_assert(lds_fits<BITS, GS, SB>(), "LDS budget");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int wm = wave >> 1, wn = wave & 1;  // 4 x 2 waves, 64 x 64 each
    // blocks below split_from own a whole tile; the rest are the two K
    // halves (part 0: all first halves, then part 1) of tiles split_from ..
    int tile = blockIdx.x, part = -1, KT = K / BK;
    if (tile >= split_from) {
        const int r = (int)((gridDim.x - (unsigned)split_from) >> 1), i = tile - split_from;
        part = i >= r;
        tile = split_from + i - part * r;
        KT >>= 1;
    }
    const int mt = tile % mtiles, nt = tile / mtiles;
    const int m0 = mt * BM;

    Ctx t;
    t.lds = lds;
    t.lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    t.x = x;
    t.wq = wq;
    t.wave = wave;
    t.lane = lane;
    t.KT = KT;
    t.k0 = part > 0 ? KT : 0;
    t.n0 = nt * BN;
    t.N = N;
    t.G = K / GS;
    t.row_bytes = (uint32_t)K * BITS / 8;
    // x tile: lane writes chunk position lane%8 of row r = 8 (4 wave + i) +
    // lane/8, so it reads global chunk (lane%8) ^ swz(r) of that row
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 8 * (4 * wave + i) + (lane >> 3);
        const int rg = min(m0 + r, M - 1);  // rows past M: valid data, never stored
        t.xoff[i] = ((uint32_t)rg * K + (uint32_t)t.k0 * BK + (((lane & 7) ^ swz(r)) << 3)) * 2;
    }
    // fragment addressing: lane reads row (lane % 32), k block 8 (lane / 32)
    const int fr_row = lane & 31, kh = lane >> 5;
    t.a_row = wm * 64 + fr_row;
    t.b_row = wn * 64 + fr_row;
#pragma unroll
    for (int ks = 0; ks < 4; ks++) t.chk[ks] = ((2 * ks + kh) ^ swz(fr_row)) << 4;
    t.dr = 16 * wave + (lane & 15);
    t.dcp = lane >> 4;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

    if (wave < 4)
        main_loop<TX, BITS, SB, GS, 0>(acc, t, scales, biases);
    else
        main_loop<TX, BITS, SB, GS, 1>(acc, t, scales, biases);

    if (part >= 0) {
        // A K half of a split tile: the halves meet in the workspace by the
        // protocol of qsplit.h.  The first to arrive stores its fp32 sums --
        // vector q of thread tid at byte ((slot * 16 + q) * 512 + tid) * 16
        // -- and publishes; the second waits, adds them to its own and
        // stores y.  The count's outcome goes through the first LDS word:
        // every wave's transfers have landed (the K loop ends waiting for
        // them all), so nothing writes the x stages any more (a static LDS
        // variable would push the buffers that fill the 160 KB exactly past
        // the limit).
        const int st = tile - split_from;
        const __amdgpu_buffer_rsrc_t pr = make_rsrc(static_cast<uint8_t*>(ws) + split::kPartOffset,
                                                    (uint32_t)((gridDim.x - (unsigned)split_from) >> 1) * kSplitSlotBytes);
        const uint32_t voff = (uint32_t)tid * 16u;
        uint32_t* word = reinterpret_cast<uint32_t*>(lds);
        __syncthreads();
        if (tid == 0) *word = split::arrive_first(ws, st) ? 1u : 0u;
        __syncthreads();
        if (*word == 1u) {
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const f32x16& a = acc[q >> 3][(q >> 2) & 1];
                const int v = 4 * (q & 3);
                __builtin_amdgcn_raw_buffer_store_b128(
                    v4{__float_as_uint(a[v]), __float_as_uint(a[v + 1]), __float_as_uint(a[v + 2]),
                       __float_as_uint(a[v + 3])},
                    pr, voff, (uint32_t)(st * 16 + q) * (kThreads * 16u), split::kCachePolicyDevice);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (tid == 0) split::publish(ws, st, epoch);
            return;
        }
        // the second half: the first's sums, or NaN for a tile whose partner
        // never published (bounded wait)
        if (tid == 0) *word = split::wait_partner(ws, st, epoch) ? 2u : 3u;
        __syncthreads();
        const float fail = *word == 2u ? 0.f : __builtin_nanf("");
        v4 o[16];
#pragma unroll
        for (int q = 0; q < 16; q++)
            o[q] = __builtin_amdgcn_raw_buffer_load_b128(pr, voff, (uint32_t)(st * 16 + q) * (kThreads * 16u),
                                                         split::kCachePolicyDevice);
#pragma unroll
        for (int q = 0; q < 16; q++) {
            f32x16& a = acc[q >> 3][(q >> 2) & 1];
            const int v = 4 * (q & 3);
            a[v] += __uint_as_float(o[q].x) + fail;
            a[v + 1] += __uint_as_float(o[q].y) + fail;
            a[v + 2] += __uint_as_float(o[q].z) + fail;
            a[v + 3] += __uint_as_float(o[q].w) + fail;
        }
    }

    // ---- epilogue: 32x32 accumulator layout: lane holds column (lane % 32),
    // VGPR v holds row 8 (v / 4) + 4 (lane / 32) + v % 4 ----
    const int ncol = t.n0 + wn * 64 + (lane & 31);
    const int mrow = m0 + wm * 64 + 4 * (lane >> 5);
    if (ep.out_dt == DT_BF16 || ep.out_dt == DT_F16) {
        uint16_t* yo = static_cast<uint16_t*>(y);
        const bool bf = ep.out_dt == DT_BF16;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int n = ncol + j * 32;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int m = mrow + i * 32 + 8 * (v >> 2) + (v & 3);
                    if (m < M && n < N) {
                        const float o = EPI ? apply_epilogue(ep, n, acc[i][j][v]) : acc[i][j][v];
                        yo[(size_t)m * N + n] = bf ? f32_to_bf16(o) : f32_to_f16(o);
                    }
                }
            }
    } else {
        float* yo = static_cast<float*>(y);
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int n = ncol + j * 32;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int m = mrow + i * 32 + 8 * (v >> 2) + (v & 3);
                    if (m < M && n < N) yo[(size_t)m * N + n] = EPI ? apply_epilogue(ep, n, acc[i][j][v]) : acc[i][j][v];
                }
            }
    }
}

template <int TX, int BITS, int SB, int GS, bool EPI>
LuxStatus launch4_e(const QmmArgs& a, hipStream_t st) {
    if constexpr (!lds_fits<BITS, GS, SB>()) {
        return LuxStatus::NotSupported;
    } else {
        if (planned(a, "qgemm_kernel")) return LuxStatus::Ok;
        auto kern = qgemm_kernel<TX, BITS, SB, GS, EPI>;
        constexpr size_t lds = lds_bytes<BITS, GS, SB>();
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (attr != hipSuccess) return LuxStatus::Internal;
        const int mtiles = (a.M + BM - 1) / BM, ntiles = (a.N + BN - 1) / BN;
        const int tiles = mtiles * ntiles;
        // the last round's tiles in two K halves where that round is at most
        // half full (each half a whole number of 4-step scale windows)
        const int r = tiles % kCUs;
        const int split_from =
            r > 0 && 2 * r <= kCUs && (a.K / BK) % 8 == 0 && a.ws != nullptr && a.epoch != 0u &&
                    a.ws_bytes >= split::kPartOffset + (size_t)r * kSplitSlotBytes
                ? tiles - r
                : tiles;
        hipLaunchKernelGGL(kern, dim3(tiles + (tiles - split_from)), dim3(kThreads), lds, st,
                           static_cast<const uint16_t*>(a.x), a.wq, a.scales, a.biases, a.y, a.M, a.K,
                           a.N, a.epi(), mtiles, split_from, a.ws, a.epoch);
        return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
    }
}

template <int TX, int BITS, int SB, int GS>
LuxStatus launch4(const QmmArgs& a, hipStream_t st) {
    return a.has_epilogue() ? launch4_e<TX, BITS, SB, GS, true>(a, st) : launch4_e<TX, BITS, SB, GS, false>(a, st);
}

template <int TX, int BITS, int GS>
LuxStatus launch3(const QmmArgs& a, hipStream_t st) {
    switch (a.sb_dtype) {
    case DT_F32: return launch4<TX, BITS, DT_F32, GS>(a, st);
    case DT_F16: return launch4<TX, BITS, DT_F16, GS>(a, st);
    default: return launch4<TX, BITS, DT_BF16, GS>(a, st);
    }
}

template <int TX, int GS>
LuxStatus launch2(const QmmArgs& a, hipStream_t st) {
    switch (a.bits) {
    case 2: return launch3<TX, 2, GS>(a, st);
    case 3: return launch3<TX, 3, GS>(a, st);
    case 4: return launch3<TX, 4, GS>(a, st);
    case 5: return launch3<TX, 5, GS>(a, st);
    case 6: return launch3<TX, 6, GS>(a, st);
    case 8: return launch3<TX, 8, GS>(a, st);
    default: return LuxStatus::NotSupported;
    }
}

// one group size, both activation types (one translation unit per group size)
template <int GS>
LuxStatus launch_g(const QmmArgs& a, hipStream_t st) {
    if (a.x_dtype == DT_BF16) return launch2<DT_BF16, GS>(a, st);
    if (a.x_dtype == DT_F16) return launch2<DT_F16, GS>(a, st);
    return LuxStatus::NotSupported;
}

extern template LuxStatus launch_g<32>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_g<64>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_g<128>(const QmmArgs&, hipStream_t);

}  // namespace gemm
}  // namespace lxq
