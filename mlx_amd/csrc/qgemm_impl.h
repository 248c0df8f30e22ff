// qgemm_impl.h -- compute-bound dequant GEMM for large M (gfx950, MFMA): kernel templates.
//
// y[M, N] = x[M, K] . T(w_hat)[N, K]^T,  T = the activation type (bf16/f16):
// each K step of 64 codes, the block dequantizes its W tile exactly
// (w_hat = fmaf(scale, q, bias) in fp32, rounded RNE to T) into LDS and runs
// v_mfma_f32_32x32x16_{bf16,f16} with fp32 accumulation.  This is the
// "dequantize to the activation type, then matmul" semantics.
//
// Block tile 256 (M) x 128 (N), 8 waves (two per SIMD) as 4 x 2, wave tile
// 64 x 64 = 2 x 2 MFMA tiles of 32 x 32.  Waves 0..3 (one per SIMD) also
// load and dequantize W; waves 4..7 only load x and run MFMAs.  The two
// roles are separate compile-time code paths, so each keeps a fixed number
// of loads in flight and its waits are constants.
//
// LDS: three x stages (256 rows x 64 k, 32 KB each, filled straight from
// global memory by global_load_lds_dwordx4) and two dequantized W stages
// (128 rows x 64 k, 16 KB each).  Rows are 128 B; 16-byte chunk c of row r
// sits at position c ^ swz(r), which makes the fragment reads (16 lanes =
// 16 consecutive rows, one chunk), the dequant writes (same shape) and the
// direct x writes (contiguous) free of bank conflicts for 8- and 16-lane
// LDS passes alike.
//
// Pipeline: x runs two K steps ahead; packed W runs four steps ahead in
// registers; scales and biases are loaded once per 4 K steps as one aligned
// window per row (GS = group size is a template parameter so the window is
// a compile-time shape; K must be a multiple of 256).  While the MFMAs of
// step k run, step k+1 is dequantized into the other W stage in two halves
// between them: one barrier per K step.
//
// Grid: one block per tile, M-tile fastest.  Blocks are dealt round-robin to
// the 8 XCDs, so with 8 M-tiles (M = 2048) every XCD owns one 256-row slab of
// x and keeps it in its own L2 while it walks the N-tiles.
#pragma once
#include "kernels.h"
#include "qcommon.h"

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
constexpr size_t kLdsBytes = (size_t)kXStages * kXStageBytes + 2 * (size_t)kWStageBytes;

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

// ---- packed W: 32 codes (one row half of a K step) = BITS words ----------

template <int BITS>
struct WRegs {
    uint32_t w[BITS];
};

// vector-memory instructions one load_words issues
template <int BITS>
constexpr int w_loads() {
    return (BITS == 5 || BITS == 6 || BITS == 8) ? 2 : 1;
}

template <int BITS>
__device__ __forceinline__ void load_words(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                           uint32_t* w) {
    if constexpr (BITS == 2) {
        v2 t = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
        w[0] = t.x; w[1] = t.y;
    } else if constexpr (BITS == 3) {
        v3 t = __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, 0);
        w[0] = t.x; w[1] = t.y; w[2] = t.z;
    } else {
        v4 t = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
        w[0] = t.x; w[1] = t.y; w[2] = t.z; w[3] = t.w;
        if constexpr (BITS == 5) {
            w[4] = __builtin_amdgcn_raw_buffer_load_b32(r, voff + 16, soff, 0);
        } else if constexpr (BITS == 6) {
            v2 u = __builtin_amdgcn_raw_buffer_load_b64(r, voff + 16, soff, 0);
            w[4] = u.x; w[5] = u.y;
        } else if constexpr (BITS == 8) {
            v4 u = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, soff, 0);
            w[4] = u.x; w[5] = u.y; w[6] = u.z; w[7] = u.w;
        }
    }
}

// ---- scales / biases of 4 K steps (256 codes) of one row ------------------

template <int GS, int SB>
struct SWin {
    static constexpr int kGroups = 256 / GS;                     // 8, 4, 2
    static constexpr int kWords = kGroups * (SB == DT_F32 ? 4 : 2) / 4;
    uint32_t s[kWords], b[kWords];
};

// loads of one window: one for scales and one for biases (two each for f32
// scales at group size 32)
template <int GS, int SB>
constexpr int s_loads() {
    return SWin<GS, SB>::kWords > 4 ? 4 : 2;
}

template <int NW>
__device__ __forceinline__ void load_win_words(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t* w) {
    if constexpr (NW == 1) {
        w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    } else if constexpr (NW == 2) {
        v2 t = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
        w[0] = t.x; w[1] = t.y;
    } else {
#pragma unroll
        for (int i = 0; i < NW; i += 4) {
            v4 t = __builtin_amdgcn_raw_buffer_load_b128(r, off + 4 * i, 0, 0);
            w[i] = t.x; w[i + 1] = t.y; w[i + 2] = t.z; w[i + 3] = t.w;
        }
    }
}

// scale/bias value of group i (compile-time) of a window
template <int SB, int NW>
__device__ __forceinline__ float win_value(const uint32_t (&w)[NW], int i) {
    if constexpr (SB == DT_F32) return __uint_as_float(w[i]);
    else {
        const uint32_t h = (i & 1) ? (w[i >> 1] >> 16) : (w[i >> 1] & 0xffffu);
        return SB == DT_F16 ? f16_to_f32(h) : bf16_to_f32(h);
    }
}

// ---- per-thread staging coordinates -------------------------------------

struct StageCoord {
    uint32_t xoff[4];  // byte offset (in x) of this lane's 4 direct-to-LDS chunks, K step 0
    uint32_t w_voff;   // byte offset of its 32 codes in W, K step 0 (dequantizing waves)
    uint32_t sb_off;   // element index of its row's first scale
    int w_row;         // W tile row it dequantizes
    int w_half;        // which 32 codes of the K step
};

// x tile of K step kt straight into an LDS x stage: 4 x 16 B per lane; wave
// w, instruction i fills the 1 KB block of rows 8 (4 w + i) .. +8 (lane l
// writes stage + block + 16 l).  Issued through inline asm: the compiler's
// wait-count pass would otherwise wait for these LDS writes before every LDS
// read, prefetch included.  The caller waits for them explicitly
// (wait_vmcnt) before the barrier that publishes the stage.
__device__ __forceinline__ void load_x_lds(uint32_t stage_lds, const uint16_t* x, const StageCoord& c,
                                           int wave, int kt) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t m0v = stage_lds + (uint32_t)(4 * wave + i) * 1024u;
        asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                     :
                     : "s"(m0v), "v"(c.xoff[i] + (uint32_t)kt * BK * 2), "s"(x)
                     : "memory", "m0");
    }
}

// wait until at most N vector-memory instructions of this wave are in flight
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N < 64, "vmcnt has 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// half h (0..1) of dequantizing K step j (0..3 within the scale window) into
// W stage D: 16 codes, w_hat = fmaf(s, q, b) rounded RNE to TX
template <int TX, int BITS, int SB, int GS, int J>
__device__ __forceinline__ void store_half(const WRegs<BITS>& ws, const SWin<GS, SB>& sw,
                                           uint8_t* D, const StageCoord& c, int h) {
    float sv, bv;
    if constexpr (GS == 32) {
        // the thread's 32 codes are group 2J + w_half
        const float s0 = win_value<SB>(sw.s, 2 * J), s1 = win_value<SB>(sw.s, 2 * J + 1);
        const float b0 = win_value<SB>(sw.b, 2 * J), b1 = win_value<SB>(sw.b, 2 * J + 1);
        sv = c.w_half ? s1 : s0;
        bv = c.w_half ? b1 : b0;
    } else {
        sv = win_value<SB>(sw.s, J * 64 / GS);
        bv = win_value<SB>(sw.b, J * 64 / GS);
    }
    const int sz = swz(c.w_row);
#pragma unroll
    for (int q = 2 * h; q < 2 * h + 2; q++) {
        float f[8];
        codes8<BITS>(ws.w, q, f);
        v4 o;
        o.x = pack2<TX>(fmaf(sv, f[0], bv), fmaf(sv, f[1], bv));
        o.y = pack2<TX>(fmaf(sv, f[2], bv), fmaf(sv, f[3], bv));
        o.z = pack2<TX>(fmaf(sv, f[4], bv), fmaf(sv, f[5], bv));
        o.w = pack2<TX>(fmaf(sv, f[6], bv), fmaf(sv, f[7], bv));
        *reinterpret_cast<v4*>(D + c.w_row * 128 + (((4 * c.w_half + q) ^ sz) << 4)) = o;
    }
}

struct Frags {
    v4 a[2], b[2];
};

// fragments of k sub-step ks: A from x stage X (rows a_row + 32 i), B from W
// stage Wt (rows b_row + 32 j); lane reads 16-byte chunk 2 ks + kh, whose
// position is ch[ks] (all rows a lane reads share swz)
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

// everything a K step needs besides the accumulators and register rings
struct Ctx {
    uint8_t* xl;        // x stages
    uint32_t xl_lds;    // their LDS address
    uint8_t* wl;        // W stages
    const uint16_t* x;
    __amdgpu_buffer_rsrc_t wr, sr, br;
    StageCoord c;
    int wave, KT, a_row, b_row;
    int chk[4];         // byte offset of this lane's fragment chunk, per k sub-step
};

// MFMAs of one K step (fragments of sub-step ks+1 are read while those of ks
// are used); dequantizing waves write the next K step (ws, window step J)
// into W stage D in two halves between them (after the last step this
// writes a stage nobody reads)
template <int TX, int BITS, int SB, int GS, bool DEQ, int J>
__device__ __forceinline__ void kstep(f32x16 (&acc)[2][2], const Ctx& t, const uint8_t* X,
                                      const uint8_t* Wt, uint8_t* D, const WRegs<BITS>& ws,
                                      const SWin<GS, SB>& sw) {
    Frags f0, f1;
    read_frags(f0, X, Wt, t.a_row, t.b_row, t.chk[0]);
    read_frags(f1, X, Wt, t.a_row, t.b_row, t.chk[1]);
    mfmas<TX>(acc, f0);
    read_frags(f0, X, Wt, t.a_row, t.b_row, t.chk[2]);
    mfmas<TX>(acc, f1);
    if constexpr (DEQ) store_half<TX, BITS, SB, GS, J>(ws, sw, D, t.c, 0);
    read_frags(f1, X, Wt, t.a_row, t.b_row, t.chk[3]);
    mfmas<TX>(acc, f0);
    mfmas<TX>(acc, f1);
    if constexpr (DEQ) store_half<TX, BITS, SB, GS, J>(ws, sw, D, t.c, 1);
}

// K step kt (P = kt % 4).  x stage kt % 3 and W stage kt % 2 hold step kt;
// W of step kt+1 is in register slot ws[(P+1) % 4], its scales in window
// cur.  Dequantizing waves issue the W loads of step kt+4 (slot ws[P]) and
// at P = 0 the scale window of steps kt+4 .. kt+7 (nxt); at P = 3 the next
// window becomes current.  Then the MFMAs with the dequantization of step
// kt+1, the x load of step kt+2, a wait until x of step kt+1 and everything
// issued before it has landed, and the barrier.  Loads past the last step
// re-read the last step (never used), so every step issues the same loads.
// In flight at the wait, after x(kt+1) [end of step kt-1]: W(kt+4) and, at
// P = 0, the new window, then x(kt+2) [step kt].
template <int TX, int BITS, int SB, int GS, bool DEQ, int P>
__device__ __forceinline__ void ring_step(f32x16 (&acc)[2][2], const Ctx& t, WRegs<BITS> (&ws)[4],
                                          SWin<GS, SB>& cur, SWin<GS, SB>& nxt, int kt) {
    const int xi = kt % 3;
    const uint8_t* X = t.xl + xi * kXStageBytes;
    const uint8_t* Wt = t.wl + (P & 1) * kWStageBytes;
    uint8_t* D = t.wl + ((P + 1) & 1) * kWStageBytes;
    if constexpr (DEQ) {
        load_words<BITS>(t.wr, t.c.w_voff, (uint32_t)min(kt + 4, t.KT - 1) * 8 * BITS, ws[P].w);
        if constexpr (P == 0) {
            constexpr int kG = SWin<GS, SB>::kGroups, kW = SWin<GS, SB>::kWords;
            const uint32_t g0 = t.c.sb_off + (uint32_t)min(kt + 4, t.KT - 4) / 4 * kG;
            load_win_words<kW>(t.sr, g0 * (SB == DT_F32 ? 4 : 2), nxt.s);
            load_win_words<kW>(t.br, g0 * (SB == DT_F32 ? 4 : 2), nxt.b);
        }
        if constexpr (P == 3) cur = nxt;
    }
    kstep<TX, BITS, SB, GS, DEQ, (P + 1) & 3>(acc, t, X, Wt, D, ws[(P + 1) & 3], cur);
    // x is issued last: the compiler does not see these loads, so the waits
    // it adds before using W registers count only its own loads; issued
    // earlier, x(kt+2) would sit inside those waits and be drained at once
    load_x_lds(t.xl_lds + (uint32_t)(xi == 0 ? 2 : xi - 1) * kXStageBytes, t.x, t.c, t.wave,
               min(kt + 2, t.KT - 1));
    if constexpr (DEQ)
        wait_vmcnt<4 + w_loads<BITS>() + s_loads<GS, SB>() * (P == 0)>();
    else
        wait_vmcnt<4>();
    __syncthreads();
}

// prologue and main loop of one wave role
template <int TX, int BITS, int SB, int GS, bool DEQ>
__device__ __forceinline__ void main_loop(f32x16 (&acc)[2][2], const Ctx& t) {
    WRegs<BITS> ws[4];
    SWin<GS, SB> cur, nxt;
    // prologue: x of steps 0, 1 into x stages 0, 1; W of steps 0..3 and the
    // scale window of steps 0..3 into registers; step 0 dequantized into W
    // stage 0
    load_x_lds(t.xl_lds, t.x, t.c, t.wave, 0);
    load_x_lds(t.xl_lds + kXStageBytes, t.x, t.c, t.wave, min(1, t.KT - 1));
    if constexpr (DEQ) {
#pragma unroll
        for (int j = 0; j < 4; j++)
            load_words<BITS>(t.wr, t.c.w_voff, (uint32_t)min(j, t.KT - 1) * 8 * BITS, ws[j].w);
        constexpr int kW = SWin<GS, SB>::kWords;
        load_win_words<kW>(t.sr, t.c.sb_off * (SB == DT_F32 ? 4 : 2), cur.s);
        load_win_words<kW>(t.br, t.c.sb_off * (SB == DT_F32 ? 4 : 2), cur.b);
    }
    wait_vmcnt<0>();
    if constexpr (DEQ) {
        store_half<TX, BITS, SB, GS, 0>(ws[0], cur, t.wl, t.c, 0);
        store_half<TX, BITS, SB, GS, 0>(ws[0], cur, t.wl, t.c, 1);
    }
    __syncthreads();

    // KT is a multiple of 4 (K % 256 == 0)
    for (int kt = 0; kt < t.KT; kt += 4) {
        ring_step<TX, BITS, SB, GS, DEQ, 0>(acc, t, ws, cur, nxt, kt);
        ring_step<TX, BITS, SB, GS, DEQ, 1>(acc, t, ws, cur, nxt, kt + 1);
        ring_step<TX, BITS, SB, GS, DEQ, 2>(acc, t, ws, cur, nxt, kt + 2);
        ring_step<TX, BITS, SB, GS, DEQ, 3>(acc, t, ws, cur, nxt, kt + 3);
    }
    // no LDS transfer may still be landing when the block's LDS is released
    wait_vmcnt<0>();
}

template <int TX, int BITS, int SB, int GS>
__global__ __launch_bounds__(kThreads, 2) void qgemm_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, int out_dt,
    int mtiles) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int wm = wave >> 1, wn = wave & 1;  // 4 x 2 waves, 64 x 64 each
    const int mt = blockIdx.x % mtiles, nt = blockIdx.x / mtiles;
    const int m0 = mt * BM, n0 = nt * BN;
    const int G = K / GS;
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    const uint32_t sbsz = SB == DT_F32 ? 4 : 2;

    Ctx t;
    t.x = x;
    t.wave = wave;
    t.KT = K / BK;
    t.wr = make_rsrc(wq, (uint32_t)((size_t)N * row_bytes));
    t.sr = make_rsrc(scales, (uint32_t)((size_t)N * G * sbsz));
    t.br = make_rsrc(biases, (uint32_t)((size_t)N * G * sbsz));
    // staging.  x tile (load_x_lds): lane writes chunk position lane%8 of
    // row r = 8 (4 wave + i) + lane/8 and so reads global chunk
    // (lane%8) ^ swz(r) of that row.  W tile (waves 0..3, tid < 256): row
    // (tid % 16) + 16 (tid / 32), codes [32 ((tid / 16) % 2), +32) of the K
    // step, so 16 consecutive lanes write 16 consecutive rows.
    {
        const int w_row = (tid & 15) | ((tid >> 5) << 4);
        t.c.w_row = w_row & (BN - 1);
        t.c.w_half = (tid >> 4) & 1;
        const int wn_glob = min(n0 + t.c.w_row, N - 1);  // rows past N: valid data, never stored
        t.c.w_voff = (uint32_t)wn_glob * row_bytes + t.c.w_half * 4 * BITS;
        t.c.sb_off = (uint32_t)wn_glob * G;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 8 * (4 * wave + i) + (lane >> 3);
            const int rg = min(m0 + r, M - 1);  // rows past M: valid data, never stored
            t.c.xoff[i] = ((uint32_t)rg * K + (((lane & 7) ^ swz(r)) << 3)) * 2;
        }
    }
    // fragment addressing: lane reads row (lane % 32), k block 8 (lane / 32)
    const int fr_row = lane & 31, kh = lane >> 5;
    t.a_row = wm * 64 + fr_row;
    t.b_row = wn * 64 + fr_row;
#pragma unroll
    for (int ks = 0; ks < 4; ks++) t.chk[ks] = ((2 * ks + kh) ^ swz(fr_row)) << 4;
    t.xl = lds;
    t.wl = lds + kXStages * kXStageBytes;
    // LDS address of the x stages (low 32 bits of the flat address)
    t.xl_lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)t.xl);

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

    if (wave < 4)
        main_loop<TX, BITS, SB, GS, true>(acc, t);
    else
        main_loop<TX, BITS, SB, GS, false>(acc, t);

    // ---- epilogue: 32x32 accumulator layout: lane holds column (lane % 32),
    // VGPR v holds row 8 (v / 4) + 4 (lane / 32) + v % 4 ----
    const int ncol = n0 + wn * 64 + (lane & 31);
    const int mrow = m0 + wm * 64 + 4 * (lane >> 5);
    if (out_dt == DT_BF16 || out_dt == DT_F16) {
        uint16_t* yo = static_cast<uint16_t*>(y);
        const bool bf = out_dt == DT_BF16;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int n = ncol + j * 32;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int m = mrow + i * 32 + 8 * (v >> 2) + (v & 3);
                    if (m < M && n < N)
                        yo[(size_t)m * N + n] = bf ? f32_to_bf16(acc[i][j][v]) : f32_to_f16(acc[i][j][v]);
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
                    if (m < M && n < N) yo[(size_t)m * N + n] = acc[i][j][v];
                }
            }
    }
}

template <int TX, int BITS, int SB, int GS>
LuxStatus launch4(const QmmArgs& a, hipStream_t st) {
    auto kern = qgemm_kernel<TX, BITS, SB, GS>;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsBytes);
    if (attr != hipSuccess) return LuxStatus::Internal;
    const int mtiles = (a.M + BM - 1) / BM, ntiles = (a.N + BN - 1) / BN;
    hipLaunchKernelGGL(kern, dim3(mtiles * ntiles), dim3(kThreads), kLdsBytes, st,
                       static_cast<const uint16_t*>(a.x), a.wq, a.scales, a.biases, a.y, a.M, a.K,
                       a.N, a.out_dtype, mtiles);
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
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
