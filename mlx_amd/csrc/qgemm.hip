// qgemm.hip -- compute-bound dequant GEMM for large M (gfx950, MFMA).
//
// y[M, N] = x[M, K] . T(w_hat)[N, K]^T,  T = the activation type (bf16/f16):
// each K step of 64 codes, the block dequantizes its W tile exactly
// (w_hat = fmaf(scale, q, bias) in fp32, rounded RNE to T) into LDS and runs
// v_mfma_f32_32x32x16_{bf16,f16} with fp32 accumulation.  This is the
// "dequantize to the activation type, then matmul" semantics.
//
// Block tile 256 (M) x 128 (N), 8 waves (two per SIMD, so one wave's MFMAs
// overlap the other's loads and dequantization) as 4 x 2, wave tile 64 x 64
// = 2 x 2 MFMA tiles of 32 x 32.
//
// LDS holds three x stages (256 rows x 64 k, 32 KB each, filled straight from
// global memory by global_load_lds_dwordx4, 16-byte chunks XOR-swizzled by
// row) and two dequantized W stages (128 rows x 64 k, rows padded to 144 B).
// x runs two K steps ahead; the packed W runs four steps ahead in registers
// (its 32-byte row pieces miss L2 more often than the x slab).  While the
// MFMAs of step k run, step k+1 is dequantized into the other W stage in two
// halves between them: one barrier per K step.
//
// Grid: one block per tile, M-tile fastest.  Blocks are dealt round-robin to
// the 8 XCDs, so with 8 M-tiles (M = 2048) every XCD owns one 256-row slab of
// x and keeps it in its own L2 while it walks the N-tiles.
#include "kernels.h"
#include "qcommon.h"

namespace lxq {
namespace gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
// 16-byte aligned vector for LDS and buffer loads
typedef uint32_t v4 __attribute__((ext_vector_type(4), aligned(16)));

constexpr int BM = 256, BN = 128, BK = 64;
constexpr int kThreads = 512;                  // 8 waves: two per SIMD
// x stages: 256 rows x 128 B, unpadded; 16-byte chunk c of row r sits at
// chunk position c ^ (r & 7), so fragment reads of 8 consecutive rows hit
// distinct banks
constexpr int kXStageBytes = BM * BK * 2;      // 32768
constexpr int kXStages = 3;
// dequantized W stages: 128 rows x 64 codes, rows padded 128 -> 144 B
constexpr int kStride = 72;                    // 16-bit elements per W row
constexpr int kWStageElems = BN * kStride;     // 9216
constexpr size_t kLdsBytes = (size_t)kXStages * kXStageBytes + 2 * (size_t)kWStageElems * 2;

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
            uint32_t v;
            if (sh + BITS <= 32) v = (w[wi] >> sh) & mask;
            else v = (uint32_t)((((uint64_t)w[wi + 1] << 32) | w[wi]) >> sh) & mask;
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

// packed W operands of one K step, held in registers (raw: converted only
// when dequantized, so nothing waits on a load right after it is issued)
template <int BITS, int SB>
struct WStage {
    uint32_t w[BITS];  // 32 codes of one W row half
    uint32_t s, b;     // raw scale and bias bits
};

// vector-memory instructions one load_w issues
template <int BITS>
constexpr int w_loads() {
    return (BITS == 4 ? 1 : BITS == 8 ? 2 : BITS) + 2;
}

template <int BITS>
__device__ __forceinline__ void load_words(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                           uint32_t* w) {
    if constexpr (BITS == 4) {
        v4 t = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
        w[0] = t.x; w[1] = t.y; w[2] = t.z; w[3] = t.w;
    } else if constexpr (BITS == 8) {
        v4 t = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
        v4 u = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, soff, 0);
        w[0] = t.x; w[1] = t.y; w[2] = t.z; w[3] = t.w;
        w[4] = u.x; w[5] = u.y; w[6] = u.z; w[7] = u.w;
    } else {
#pragma unroll
        for (int i = 0; i < BITS; i++) w[i] = __builtin_amdgcn_raw_buffer_load_b32(r, voff + 4 * i, soff, 0);
    }
}

template <int SB>
__device__ __forceinline__ uint32_t load_sb_raw(__amdgpu_buffer_rsrc_t r, uint32_t idx) {
    if constexpr (SB == DT_F32) return __builtin_amdgcn_raw_buffer_load_b32(r, idx * 4, 0, 0);
    else return __builtin_amdgcn_raw_buffer_load_b16(r, idx * 2, 0, 0);
}

template <int SB>
__device__ __forceinline__ float sb_value(uint32_t raw) {
    if constexpr (SB == DT_F32) return __uint_as_float(raw);
    else if constexpr (SB == DT_F16) return f16_to_f32(raw);
    else return bf16_to_f32(raw);
}

// per-thread staging coordinates
struct StageCoord {
    uint32_t xoff[4];       // byte offset (in x) of this lane's 4 direct-to-LDS chunks, K step 0
    uint32_t w_voff;        // byte offset of its 32 codes in W, K step 0
    uint32_t sb_row;        // index of its W row's first scale
    int w_lds;              // LDS element offset of its dequantized codes
    int w_half;
    bool deq;               // this thread dequantizes a W row half
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

// every thread issues the same loads (threads 256..511 read the same rows as
// their partner and never use them), so the number of loads in flight is the
// same on every path and the compiler's wait counts stay exact
template <int BITS, int SB>
__device__ __forceinline__ void load_w(WStage<BITS, SB>& st, __amdgpu_buffer_rsrc_t wr,
                                       __amdgpu_buffer_rsrc_t sr, __amdgpu_buffer_rsrc_t br,
                                       const StageCoord& c, int kt, int gsize) {
    load_words<BITS>(wr, c.w_voff, (uint32_t)kt * 8 * BITS, st.w);
    const uint32_t gi = c.sb_row + (uint32_t)(kt * BK + c.w_half * 32) / gsize;
    st.s = load_sb_raw<SB>(sr, gi);
    st.b = load_sb_raw<SB>(br, gi);
}

// wait until at most N vector-memory instructions of this wave are in flight
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N < 64, "vmcnt has 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// half h (0..1) of dequantizing a staged K step into a W stage (16 codes,
// w_hat = fmaf(s, q, b) rounded RNE to TX), dequantizing threads only
template <int TX, int BITS, int SB>
__device__ __forceinline__ void store_half(const WStage<BITS, SB>& ws, uint16_t* D, const StageCoord& c,
                                           int h) {
    if (c.deq) {
        const float sv = sb_value<SB>(ws.s), bv = sb_value<SB>(ws.b);
#pragma unroll
        for (int q = 2 * h; q < 2 * h + 2; q++) {
            float f[8];
            codes8<BITS>(ws.w, q, f);
            v4 o;
            o.x = pack2<TX>(fmaf(sv, f[0], bv), fmaf(sv, f[1], bv));
            o.y = pack2<TX>(fmaf(sv, f[2], bv), fmaf(sv, f[3], bv));
            o.z = pack2<TX>(fmaf(sv, f[4], bv), fmaf(sv, f[5], bv));
            o.w = pack2<TX>(fmaf(sv, f[6], bv), fmaf(sv, f[7], bv));
            *reinterpret_cast<v4*>(D + c.w_lds + 8 * q) = o;
        }
    }
}

struct Frags {
    v4 a[2], b[2];
};

// fragments of k sub-step ks: A from x stage X (row a_row + 32 i, 16-byte
// chunk 2 ks + kh, swizzled), B from W stage Wt (row b_row + 32 j)
__device__ __forceinline__ void read_frags(Frags& f, const uint8_t* X, const uint16_t* Wt, int a_row,
                                           int b0, int kh, int ks) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int r = a_row + 32 * i;
        f.a[i] = *reinterpret_cast<const v4*>(X + r * 128 + (((2 * ks + kh) ^ (r & 7)) << 4));
    }
#pragma unroll
    for (int j = 0; j < 2; j++) f.b[j] = *reinterpret_cast<const v4*>(Wt + b0 + j * 32 * kStride + ks * 16);
}

template <int TX>
__device__ __forceinline__ void mfmas(f32x16 (&acc)[2][2], const Frags& f) {
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = mfma<TX>(f.a[i], f.b[j], acc[i][j]);
}

// MFMAs of one K step (fragments of sub-step ks+1 are read while those of ks
// are used); the next K step (ws) is dequantized into W stage D in two halves
// between them (after the last step this writes a stage nobody reads)
template <int TX, int BITS, int SB>
__device__ __forceinline__ void kstep(f32x16 (&acc)[2][2], const uint8_t* X, const uint16_t* Wt,
                                      uint16_t* D, const WStage<BITS, SB>& ws, const StageCoord& c,
                                      int a_row, int b0, int kh) {
    Frags f0, f1;
    read_frags(f0, X, Wt, a_row, b0, kh, 0);
    read_frags(f1, X, Wt, a_row, b0, kh, 1);
    mfmas<TX>(acc, f0);
    read_frags(f0, X, Wt, a_row, b0, kh, 2);
    mfmas<TX>(acc, f1);
    store_half<TX, BITS, SB>(ws, D, c, 0);
    read_frags(f1, X, Wt, a_row, b0, kh, 3);
    mfmas<TX>(acc, f0);
    mfmas<TX>(acc, f1);
    store_half<TX, BITS, SB>(ws, D, c, 1);
}

// K step kt.  x stage kt % 3 and W stage kt % 2 hold step kt; W of step
// kt+1 is in register slot ws[(kt+1) % 4].  Issue the x load of step kt+2
// (x stage (kt+2) % 3) and the W loads of step kt+4 (slot ws[kt % 4]), run
// the MFMAs, dequantize step kt+1 into W stage (kt+1) % 2, wait until x of
// step kt+1 (issued one step earlier) has landed, then barrier.  Loads past
// the last step re-read step KT-1 (never used), so every step issues the
// same loads and keeps the same number in flight.  P = kt % 4 gives
// compile-time register slots.
template <int TX, int BITS, int SB, int P>
__device__ __forceinline__ void ring_step(f32x16 (&acc)[2][2], WStage<BITS, SB> (&ws)[4],
                                          uint8_t* xl, uint32_t xl_lds, const uint16_t* x,
                                          uint16_t* wl, __amdgpu_buffer_rsrc_t wr,
                                          __amdgpu_buffer_rsrc_t sr, __amdgpu_buffer_rsrc_t br,
                                          const StageCoord& c, int wave, int kt, int KT, int gsize,
                                          int a_row, int b0, int kh) {
    const int xi = kt % 3;
    const uint8_t* X = xl + xi * kXStageBytes;
    const uint16_t* Wt = wl + (P & 1) * kWStageElems;
    uint16_t* D = wl + ((P + 1) & 1) * kWStageElems;
    load_x_lds(xl_lds + (uint32_t)(xi == 0 ? 2 : xi - 1) * kXStageBytes, x, c, wave, min(kt + 2, KT - 1));
    load_w<BITS, SB>(ws[P], wr, sr, br, c, min(kt + 4, KT - 1), gsize);
    kstep<TX, BITS, SB>(acc, X, Wt, D, ws[(P + 1) & 3], c, a_row, b0, kh);
    // in flight after x(kt+1) of this wave: W(kt+3) [issued at step kt-1],
    // x(kt+2) and W(kt+4) [this step]
    wait_vmcnt<4 + 2 * w_loads<BITS>()>();
    __syncthreads();
}

template <int TX, int BITS, int SB>
__global__ __launch_bounds__(kThreads, 2) void qgemm_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, int gsize,
    int out_dt, int mtiles) {
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int wm = wave >> 1, wn = wave & 1;  // 4 x 2 waves, 64 x 64 each
    const int mt = blockIdx.x % mtiles, nt = blockIdx.x / mtiles;
    const int m0 = mt * BM, n0 = nt * BN;
    const int KT = K / BK;
    const int G = K / gsize;
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    const uint32_t sbsz = SB == DT_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wq, (uint32_t)((size_t)N * row_bytes));
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(scales, (uint32_t)((size_t)N * G * sbsz));
    const __amdgpu_buffer_rsrc_t br = make_rsrc(biases, (uint32_t)((size_t)N * G * sbsz));

    // staging.  x tile (load_x_lds): lane writes chunk position lane%8 of
    // row 8 (4 wave + i) + lane/8 and so reads global chunk (lane%8) ^ (row&7)
    // of that row.  W tile (threads 0..255): row tid/2, codes
    // [32 (tid%2), +32) of the K step.
    StageCoord c;
    {
        const int wt = tid & 255, w_row = wt >> 1;
        c.deq = tid < 256;
        c.w_half = wt & 1;
        const int wn_glob = min(n0 + w_row, N - 1);  // rows past N: valid data, never stored
        c.w_voff = (uint32_t)wn_glob * row_bytes + c.w_half * 4 * BITS;
        c.sb_row = (uint32_t)wn_glob * G;
        c.w_lds = w_row * kStride + c.w_half * 32;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 8 * (4 * wave + i) + (lane >> 3);
            const int rg = min(m0 + r, M - 1);  // rows past M: valid data, never stored
            c.xoff[i] = ((uint32_t)rg * K + (((lane & 7) ^ (r & 7)) << 3)) * 2;
        }
    }

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

    // fragment addressing: lane reads row (lane % 32), k block 8 (lane / 32)
    const int fr_row = lane & 31, kh = lane >> 5;
    const int a_row = wm * 64 + fr_row;
    const int b0 = (wn * 64 + fr_row) * kStride + kh * 8;
    uint8_t* xl = reinterpret_cast<uint8_t*>(lds);
    uint16_t* wl = reinterpret_cast<uint16_t*>(xl + kXStages * kXStageBytes);
    // LDS address of the x stages (low 32 bits of the flat address)
    const uint32_t xl_lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)xl);

    // prologue: x of steps 0, 1 into x stages 0, 1; W of steps 0..3 into
    // registers; step 0 dequantized into W stage 0
    WStage<BITS, SB> ws[4];
    load_x_lds(xl_lds, x, c, wave, 0);
    load_x_lds(xl_lds + kXStageBytes, x, c, wave, min(1, KT - 1));
#pragma unroll
    for (int j = 0; j < 4; j++) load_w<BITS, SB>(ws[j], wr, sr, br, c, min(j, KT - 1), gsize);
    wait_vmcnt<0>();
    store_half<TX, BITS, SB>(ws[0], wl, c, 0);
    store_half<TX, BITS, SB>(ws[0], wl, c, 1);
    __syncthreads();

    int kt = 0;
    for (; kt + 4 <= KT; kt += 4) {
        ring_step<TX, BITS, SB, 0>(acc, ws, xl, xl_lds, x, wl, wr, sr, br, c, wave, kt, KT, gsize, a_row, b0, kh);
        ring_step<TX, BITS, SB, 1>(acc, ws, xl, xl_lds, x, wl, wr, sr, br, c, wave, kt + 1, KT, gsize, a_row, b0, kh);
        ring_step<TX, BITS, SB, 2>(acc, ws, xl, xl_lds, x, wl, wr, sr, br, c, wave, kt + 2, KT, gsize, a_row, b0, kh);
        ring_step<TX, BITS, SB, 3>(acc, ws, xl, xl_lds, x, wl, wr, sr, br, c, wave, kt + 3, KT, gsize, a_row, b0, kh);
    }
    // the last KT % 4 steps
    if (kt < KT)
        ring_step<TX, BITS, SB, 0>(acc, ws, xl, xl_lds, x, wl, wr, sr, br, c, wave, kt, KT, gsize, a_row, b0, kh);
    if (kt + 1 < KT)
        ring_step<TX, BITS, SB, 1>(acc, ws, xl, xl_lds, x, wl, wr, sr, br, c, wave, kt + 1, KT, gsize, a_row, b0, kh);
    if (kt + 2 < KT)
        ring_step<TX, BITS, SB, 2>(acc, ws, xl, xl_lds, x, wl, wr, sr, br, c, wave, kt + 2, KT, gsize, a_row, b0, kh);
    // no LDS transfer may still be landing when the block's LDS is released
    wait_vmcnt<0>();

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

template <int TX, int BITS, int SB>
LuxStatus launch3(const QmmArgs& a, hipStream_t st) {
    auto kern = qgemm_kernel<TX, BITS, SB>;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsBytes);
    if (attr != hipSuccess) return LuxStatus::Internal;
    const int mtiles = (a.M + BM - 1) / BM, ntiles = (a.N + BN - 1) / BN;
    hipLaunchKernelGGL(kern, dim3(mtiles * ntiles), dim3(kThreads), kLdsBytes, st,
                       static_cast<const uint16_t*>(a.x), a.wq, a.scales, a.biases, a.y, a.M, a.K,
                       a.N, a.group_size, a.out_dtype, mtiles);
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

template <int TX, int BITS>
LuxStatus launch2(const QmmArgs& a, hipStream_t st) {
    switch (a.sb_dtype) {
    case DT_F32: return launch3<TX, BITS, DT_F32>(a, st);
    case DT_F16: return launch3<TX, BITS, DT_F16>(a, st);
    default: return launch3<TX, BITS, DT_BF16>(a, st);
    }
}

template <int TX>
LuxStatus launch1(const QmmArgs& a, hipStream_t st) {
    switch (a.bits) {
    case 2: return launch2<TX, 2>(a, st);
    case 3: return launch2<TX, 3>(a, st);
    case 4: return launch2<TX, 4>(a, st);
    case 5: return launch2<TX, 5>(a, st);
    case 6: return launch2<TX, 6>(a, st);
    case 8: return launch2<TX, 8>(a, st);
    default: return LuxStatus::NotSupported;
    }
}

}  // namespace gemm

LuxStatus launch_qgemm(const QmmArgs& a, hipStream_t st) {
    if (a.K % gemm::BK != 0) return LuxStatus::NotSupported;
    // x and W offsets are 32-bit: each must stay below 4 GiB
    if ((size_t)a.M * a.K * 2 >= (1ull << 32) || (size_t)a.N * a.K * a.bits / 8 >= (1ull << 32))
        return LuxStatus::NotSupported;
    if (a.x_dtype == DT_BF16) return gemm::launch1<DT_BF16>(a, st);
    if (a.x_dtype == DT_F16) return gemm::launch1<DT_F16>(a, st);
    return LuxStatus::NotSupported;
}

}  // namespace lxq
