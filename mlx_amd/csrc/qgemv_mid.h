// qgemv_mid.h -- exact-form MFMA kernel for 2 <= M <= 16 rows of x, 4- and
// 8-bit codes, f16/bf16 activations, K % 1024 == 0 (gfx950).
//
// y[m, n] = sum_g s[n,g] * sum_{k in g} q[n,k] x[m,k] + b[n,g] * sum_{k in g} x[m,k]
//
// Same skeleton as the small-M GEMM (qgemm_small.h): a block owns 32 rows n
// of W, its 4 waves split K in four parts and meet in LDS at the end, and
// every wave stages its operands in LDS rings of its own by buffer->LDS DMA
// (x: the M rows of one 64-code step; W, scales, biases: four steps), with
// one compile-time vmcnt wait per step and no barrier in the main loop.
//
// Arithmetic is the exact form of the skinny kernel (qmm_skinny.h):
// v_mfma_f32_16x16x32 with A = x (row m = lane % 16; rows past M repeat row
// M-1 and are never stored) and B = the codes as operands v = A0 + q U
// (column = W row 16 t + lane % 16 of the wave's tile t).  Every MFMA covers
// 32 codes of one group, so a group's D = sum v x is complete after GS/32
// MFMAs and is scaled by s in fp32 at once; an MFMA with an all-ones B
// operand gives sx = sum_{k in g} x for the term (b/kPow - A0 s) sx.
//
// Code slices: for GS = 32 slice t of a step is codes 32t .. 32t+31 (lane
// group c = lane / 16 takes 32t + 8c .. +8); for GS >= 64 a step lies in one
// group and lane group c takes codes 16c .. 16c+15 (slice t: 16c + 8t .. +8),
// one contiguous read per tile.  W chunks (16 B) are XOR-swizzled by row
// through the DMA source address, so the 16 rows a read touches spread over
// the LDS banks.
#pragma once
#include "kernels.h"
#include "qcommon.h"
#include "qgemm_small.h"
#include "qmm_skinny.h"

namespace lxq {
namespace mid {

using small::u4;
using small::dma16;
using small::dma4;
using small::swz;
using small::wait_vmcnt_small;
using small::wait_lds_reads;
using skinny::Form;
using skinny::code_operand;
using skinny::x_operand;
using skinny::mfma32;
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;

template <int BITS, int SB, int GS, int XR>
struct Lay {
    static constexpr int kSb = SB == DT_F32 ? 4 : 2;
    static constexpr int kXS = XR * 1024;               // one x step: 8 XR rows x 128 B
    static constexpr int kRX = 3;                       // x steps resident
    static constexpr int kCPR = 2 * BITS;               // 16-B chunks per W row per super-step
    static constexpr int kWS = 32 * 32 * BITS;          // one W super-step (4 steps)
    static constexpr int kRW = 3;                       // W super-steps resident
    static constexpr int kSPR = (256 / GS) * kSb;       // scale bytes per row per super-step
    static constexpr int kDpr = kSPR / 4;
    static constexpr int kNS = (32 * kDpr + 63) / 64;
    static constexpr int kSS = 32 * kSPR;
    static constexpr int kNWS = BITS + 2 * kNS;         // W + scale + bias DMAs per super-step
    static constexpr int kX0 = 0, kW0 = kRX * kXS, kS0 = kW0 + kRW * kWS, kB0 = kS0 + kRW * kSS;
    static constexpr int kWaveBytes = kB0 + kRW * kSS;
    static constexpr int kRed = 4 * 2 * 4 * 64 * 4;     // final K-part reduction (reuses the rings)
    static constexpr int kBytes = (4 * kWaveBytes > kRed) ? 4 * kWaveBytes : kRed;
    static_assert(2 * XR + 2 * kNWS < 64, "vmcnt holds 6 bits");
    static_assert(kSPR % 4 == 0, "scale rows of a super-step are whole dwords");
};

template <int BITS, int SB, int GS, int XR>
struct Ctx {
    uint32_t lds;
    const uint8_t *x, *w, *s, *b;
    uint32_t xoff[XR];
    uint32_t woff[BITS];
    uint32_t soff[Lay<BITS, SB, GS, XR>::kNS];
    bool sact[Lay<BITS, SB, GS, XR>::kNS];
};

template <int BITS, int SB, int GS, int XR>
__device__ __forceinline__ void issue_x(const Ctx<BITS, SB, GS, XR>& c, int qs) {
    using L = Lay<BITS, SB, GS, XR>;
    const uint32_t base = c.lds + L::kX0 + (uint32_t)(qs % L::kRX) * L::kXS;
    const uint8_t* src = c.x + (size_t)qs * 128;
#pragma unroll
    for (int i = 0; i < XR; i++) dma16(base + 1024u * i, src, c.xoff[i]);
}
template <int BITS, int SB, int GS, int XR>
__device__ __forceinline__ void issue_w(const Ctx<BITS, SB, GS, XR>& c, int u) {
    using L = Lay<BITS, SB, GS, XR>;
    const uint32_t slot = (uint32_t)(u % L::kRW);
    const uint8_t* src = c.w + (size_t)u * 32 * BITS;
#pragma unroll
    for (int i = 0; i < BITS; i++) dma16(c.lds + L::kW0 + slot * L::kWS + 1024u * i, src, c.woff[i]);
    const uint8_t* ss = c.s + (size_t)u * L::kSPR;
    const uint8_t* bs = c.b + (size_t)u * L::kSPR;
#pragma unroll
    for (int i = 0; i < L::kNS; i++)
        if (c.sact[i]) dma4(c.lds + L::kS0 + slot * L::kSS + 256u * i, ss, c.soff[i]);
#pragma unroll
    for (int i = 0; i < L::kNS; i++)
        if (c.sact[i]) dma4(c.lds + L::kB0 + slot * L::kSS + 256u * i, bs, c.soff[i]);
}

template <int SB>
__device__ __forceinline__ float ld_sb(const uint8_t* p) {
    if constexpr (SB == DT_F32) return *reinterpret_cast<const float*>(p);
    else if constexpr (SB == DT_F16) return f16_to_f32(*reinterpret_cast<const uint16_t*>(p));
    else return bf16_to_f32(*reinterpret_cast<const uint16_t*>(p));
}

// first code (within the step) of lane group cg in slice t
template <int GS>
__device__ __forceinline__ int slice_code(int t, int cg) {
    return GS == 32 ? 32 * t + 8 * cg : 16 * cg + 8 * t;
}

// step q (P = q % 4): issues W of super-step u + 2 (at P == 0) and x of step
// q + 2, waits for x(q) (the W of super-step u is older), then two slices
template <int BITS, int TX, int SB, int GS, int XR, int P>
__device__ __forceinline__ void step(f32x4 (&acc)[2], f32x4 (&dg)[2], f32x4& dx, const Ctx<BITS, SB, GS, XR>& c,
                                     const uint8_t* lw, int q, int nq, int M, uint32_t vm, uint32_t vmagic) {
    using L = Lay<BITS, SB, GS, XR>;
    using F = Form<BITS, TX>;
    constexpr int NMG = GS / 32;  // slices per group
    const int u = q >> 2;
    wait_lds_reads();  // the previous step's reads of the slots refilled here are done
    if constexpr (P == 0) {
        const int uw = u + L::kRW - 1, ul = (nq >> 2) - 1;
        issue_w(c, uw < ul ? uw : ul);
    }
    {
        const int qx = q + L::kRX - 1;
        issue_x(c, qx < nq ? qx : nq - 1);
    }
    // younger than x(q): x(q+1), x(q+2) and the W issues of steps q-1, q
    constexpr int kYoung = 2 * XR + L::kNWS * ((P == 0 ? 1 : 0) + (P == 1 ? 1 : 0));
    wait_vmcnt_small<kYoung>();
    const int lane = threadIdx.x & 63, j = lane & 15, cg = lane >> 4;
    const uint8_t* xs = lw + L::kX0 + (q % L::kRX) * L::kXS;
    const int m = j < M ? j : M - 1;
    const int slot = u % L::kRW;
    const u4 ones = {F::kOne2, F::kOne2, F::kOne2, F::kOne2};
    // codes of both slices for both tiles (BITS/4 words per slice)
    uint32_t cw[2][2][BITS / 4];
#pragma unroll
    for (int tile = 0; tile < 2; tile++) {
        const int r = 16 * tile + j;
        const uint8_t* row = lw + L::kW0 + slot * L::kWS + r * L::kCPR * 16;
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int byte = P * 8 * BITS + slice_code<GS>(t, cg) * BITS / 8;  // within the row's super-step
            const int ch = (byte >> 4) ^ (r & (L::kCPR - 1));
            const uint32_t* wp = reinterpret_cast<const uint32_t*>(row + ch * 16 + (byte & 15));
#pragma unroll
            for (int i = 0; i < BITS / 4; i++) cw[tile][t][i] = wp[i];
        }
    }
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int chunk = slice_code<GS>(t, cg) >> 3;  // 16-B x chunk of the step
        const u4 xn = *reinterpret_cast<const u4*>(xs + m * 128 + ((chunk ^ swz(m)) * 16));
        const u4 xa = x_operand<BITS, TX>(xn);
#pragma unroll
        for (int tile = 0; tile < 2; tile++)
            dg[tile] = mfma32<TX>(xa, code_operand<BITS, TX>(cw[tile][t], vm, vmagic), dg[tile]);
        dx = mfma32<TX>(xn, ones, dx);
        const int slice = 2 * P + t;
        if ((slice + 1) % NMG == 0) {  // a group ends: scale it and restart the group sums
            const int gi = (P * 64 + 32 * t) / GS;
#pragma unroll
            for (int tile = 0; tile < 2; tile++) {
                const int r = 16 * tile + j;
                const float sc = ld_sb<SB>(lw + L::kS0 + slot * L::kSS + r * L::kSPR + gi * L::kSb);
                const float bi = ld_sb<SB>(lw + L::kB0 + slot * L::kSS + r * L::kSPR + gi * L::kSb);
                const float cc = fmaf(-F::kA0, sc, bi * (1.f / F::kPow));
#pragma unroll
                for (int e = 0; e < 4; e++) acc[tile][e] = fmaf(sc, dg[tile][e], fmaf(cc, dx[e], acc[tile][e]));
                dg[tile] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
            dx = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
}

template <int BITS, int TX, int SB, int GS, int XR, bool EPI>
__global__ __launch_bounds__(64 * kWaves) void qgemv_mid_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, Epilogue ep) {
    using L = Lay<BITS, SB, GS, XR>;
    using F = Form<BITS, TX>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * 32;
    const int G = K / GS;
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    const int nq = K / 64 / kWaves;  // steps of this wave's part (a multiple of 4)
    const int k0 = wave * nq * 64;

    Ctx<BITS, SB, GS, XR> c;
    c.lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds) + (uint32_t)wave * L::kWaveBytes;
    c.x = static_cast<const uint8_t*>(x) + (size_t)k0 * 2;
    c.w = reinterpret_cast<const uint8_t*>(wq) + (size_t)k0 * BITS / 8;
    c.s = static_cast<const uint8_t*>(scales) + (size_t)(k0 / GS) * L::kSb;
    c.b = static_cast<const uint8_t*>(biases) + (size_t)(k0 / GS) * L::kSb;
#pragma unroll
    for (int i = 0; i < XR; i++) {
        const int r = 8 * i + (lane >> 3);  // LDS row of the step
        const int mr = r < M ? r : M - 1;   // rows past M repeat row M-1
        c.xoff[i] = ((uint32_t)mr * K + 8 * ((lane & 7) ^ swz(r))) * 2;
    }
#pragma unroll
    for (int i = 0; i < BITS; i++) {
        // LDS slot v of the super-step: row r, physical chunk p, holding logical chunk p ^ (r % kCPR)
        const int v = 64 * i + lane, r = v / L::kCPR, p = v % L::kCPR;
        const int n = n0 + r < N ? n0 + r : N - 1;
        c.woff[i] = (uint32_t)n * row_bytes + 16u * (p ^ (r & (L::kCPR - 1)));
    }
#pragma unroll
    for (int i = 0; i < L::kNS; i++) {
        const int v = 64 * i + lane, r = v / L::kDpr, d = v % L::kDpr;
        const int n = n0 + r < N ? n0 + r : N - 1;
        c.sact[i] = v < 32 * L::kDpr;
        c.soff[i] = (uint32_t)n * G * L::kSb + 4u * d;
    }
    const uint8_t* lw = lds + (size_t)wave * L::kWaveBytes;
    const uint32_t vm = vconst(F::kMask), vmagic = vconst(F::kMagic);

    // prologue: W of super-steps 0 .. kRW-2, x of steps 0 .. kRX-2 (the steady-state order)
#pragma unroll
    for (int uu = 0; uu < L::kRW - 1; uu++) issue_w(c, uu < (nq >> 2) - 1 ? uu : (nq >> 2) - 1);
#pragma unroll
    for (int qq = 0; qq < L::kRX - 1; qq++) issue_x(c, qq < nq - 1 ? qq : nq - 1);

    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    f32x4 dg[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    f32x4 dx = {0.f, 0.f, 0.f, 0.f};
    for (int q = 0; q < nq; q += 4) {
        step<BITS, TX, SB, GS, XR, 0>(acc, dg, dx, c, lw, q, nq, M, vm, vmagic);
        step<BITS, TX, SB, GS, XR, 1>(acc, dg, dx, c, lw, q + 1, nq, M, vm, vmagic);
        step<BITS, TX, SB, GS, XR, 2>(acc, dg, dx, c, lw, q + 2, nq, M, vm, vmagic);
        step<BITS, TX, SB, GS, XR, 3>(acc, dg, dx, c, lw, q + 3, nq, M, vm, vmagic);
    }
    wait_vmcnt_small<0>();
    __syncthreads();

    // K parts meet in LDS: wave w sums accumulator element w of both tiles
    float* red = reinterpret_cast<float*>(lds);  // [wave][tile][4][64]
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int e = 0; e < 4; e++) red[((wave * 2 + t) * 4 + e) * 64 + lane] = acc[t][e];
    __syncthreads();
    const int j = lane & 15, cg = lane >> 4;
#pragma unroll
    for (int t = 0; t < 2; t++) {
        float sum = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < kWaves; w2++) sum += red[((w2 * 2 + t) * 4 + wave) * 64 + lane];
        // 16x16 accumulator: lane holds D[4 (lane / 16) + e][lane % 16] (rows m of x, columns n of W)
        const int mm = 4 * cg + wave, nn = n0 + 16 * t + j;
        if (mm < M && nn < N) store_out<EPI>(y, (size_t)mm * N + nn, nn, ep, sum * F::kPow);
    }
}

}  // namespace mid

// launcher (qgemv_mid.hip): NotSupported unless 2 <= M <= 16, bits 4 or 8,
// f16/bf16 x, K % 1024 == 0 and 32-bit DMA offsets
LuxStatus launch_qgemv_mid(const QmmArgs& a, hipStream_t st);

}  // namespace lxq
