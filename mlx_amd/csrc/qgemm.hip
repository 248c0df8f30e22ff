// qgemm.hip -- compute-bound dequant GEMM for large M (gfx950, MFMA).
//
// y[M, N] = x[M, K] . T(w_hat)[N, K]^T,  T = the activation type (bf16/f16):
// each K step of 64 codes, the block dequantizes its W tile exactly
// (w_hat = fmaf(scale, q, bias) in fp32, rounded RNE to T) into LDS and runs
// v_mfma_f32_32x32x16_{bf16,f16} with fp32 accumulation.  This is the
// "dequantize to the activation type, then matmul" semantics.
//
// Block tile 256 (M) x 128 (N), 4 waves as 2 x 2, wave tile 128 x 64 =
// 4 x 2 MFMA tiles of 32 x 32.  LDS holds two stages of
//   A: 256 rows x 64 k (x tile, copied)       36 KB with padding
//   B: 128 rows x 64 k (dequantized W tile)   18 KB with padding
// Rows are padded from 128 B to 144 B so that the 16-byte fragment reads of
// 32 consecutive rows spread over the LDS banks.  Global loads of stage k+1
// are issued before the MFMAs of stage k and written to the other LDS buffer
// after them: one barrier per K step.
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
// 16-byte aligned vector for LDS and for the 16-byte aligned x rows
typedef uint32_t v4 __attribute__((ext_vector_type(4), aligned(16)));

constexpr int BM = 256, BN = 128, BK = 64;
constexpr int kThreads = 256;
constexpr int kStride = 72;                    // 16-bit elements per LDS row (64 + 8 pad)
constexpr int kAElems = BM * kStride;
constexpr int kBElems = BN * kStride;
constexpr int kStageElems = kAElems + kBElems;
constexpr size_t kLdsBytes = 2 * kStageElems * 2;  // 110592

template <int DT>
__device__ __forceinline__ float load_c(const void* __restrict__ p, size_t i) {
    if constexpr (DT == DT_F32) return reinterpret_cast<const float*>(p)[i];
    else if constexpr (DT == DT_F16) return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    else return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

// two fp32 values -> packed pair of T (RNE)
template <int TX>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (TX == DT_BF16) {
        return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
    } else {
        return (uint32_t)f32_to_f16(a) | ((uint32_t)f32_to_f16(b) << 16);
    }
}

// code i (0..31) of a 32-code half unit held in BITS words
template <int BITS>
__device__ __forceinline__ uint32_t half_code(const uint32_t* w, int i) {
    const int bit = i * BITS, wi = bit >> 5, sh = bit & 31;
    const uint32_t mask = (1u << BITS) - 1u;
    if (sh + BITS <= 32) return (w[wi] >> sh) & mask;
    return (uint32_t)((((uint64_t)w[wi + 1] << 32) | w[wi]) >> sh) & mask;
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

template <int TX, int BITS, int SB>
__global__ __launch_bounds__(kThreads, 1) void qgemm_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, int gsize,
    int out_dt, int mtiles) {
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int mt = blockIdx.x % mtiles, nt = blockIdx.x / mtiles;
    const int m0 = mt * BM, n0 = nt * BN;
    const int KT = K / BK;
    const int G = K / gsize;
    const int row_words = (K * BITS) >> 5;

    // ---- global -> register staging ----
    // A: thread loads 16 B (8 elements) of 8 rows: row tid/8 + 32 i, chunk tid%8
    // W: thread handles row tid/2, codes [32 (tid%2), +32) of the K step
    const int a_chunk = tid & 7, a_row0 = tid >> 3;
    const int w_row = tid >> 1, w_half = tid & 1;
    const int wn_glob = min(n0 + w_row, N - 1);
    const uint32_t* wrow = wq + (size_t)wn_glob * row_words;
    size_t a_off[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = min(m0 + a_row0 + 32 * i, M - 1);  // rows past M: valid reads, never stored
        a_off[i] = (size_t)r * K + a_chunk * 8;
    }
    v4 a_reg[8];
    uint32_t w_reg[BITS];
    float s_reg = 0.f, b_reg = 0.f;

    auto load_stage = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 8; i++) a_reg[i] = *reinterpret_cast<const v4*>(x + a_off[i] + kt * BK);
        const int kc = kt * BK + w_half * 32;  // first code of this thread's half unit
        const uint32_t* p = wrow + ((kc * BITS) >> 5);
#pragma unroll
        for (int i = 0; i < BITS; i++) w_reg[i] = p[i];
        const size_t gi = (size_t)wn_glob * G + kc / gsize;
        s_reg = load_c<SB>(scales, gi);
        b_reg = load_c<SB>(biases, gi);
    };

    auto store_stage = [&](int buf) {
        uint16_t* A = lds + buf * kStageElems;
        uint16_t* Bt = A + kAElems;
#pragma unroll
        for (int i = 0; i < 8; i++)
            *reinterpret_cast<v4*>(A + (a_row0 + 32 * i) * kStride + a_chunk * 8) = a_reg[i];
        uint32_t pk[16];
#pragma unroll
        for (int c = 0; c < 16; c++) {
            const float v0 = fmaf(s_reg, (float)half_code<BITS>(w_reg, 2 * c), b_reg);
            const float v1 = fmaf(s_reg, (float)half_code<BITS>(w_reg, 2 * c + 1), b_reg);
            pk[c] = pack2<TX>(v0, v1);
        }
        v4* dst = reinterpret_cast<v4*>(Bt + w_row * kStride + w_half * 32);
#pragma unroll
        for (int i = 0; i < 4; i++) dst[i] = v4{pk[4 * i], pk[4 * i + 1], pk[4 * i + 2], pk[4 * i + 3]};
    };

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

    // fragment addressing: lane reads row (lane % 32), k block 8 (lane / 32)
    const int fr_row = lane & 31, fr_k = (lane >> 5) * 8;

    load_stage(0);
    store_stage(0);
    __syncthreads();

    for (int kt = 0; kt < KT; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < KT) load_stage(kt + 1);
        const uint16_t* A = lds + buf * kStageElems;
        const uint16_t* Bt = A + kAElems;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            v4 af[4], bfr[2];
#pragma unroll
            for (int i = 0; i < 4; i++)
                af[i] = *reinterpret_cast<const v4*>(A + (wm * 128 + i * 32 + fr_row) * kStride +
                                                        ks * 16 + fr_k);
#pragma unroll
            for (int j = 0; j < 2; j++)
                bfr[j] = *reinterpret_cast<const v4*>(Bt + (wn * 64 + j * 32 + fr_row) * kStride +
                                                         ks * 16 + fr_k);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) acc[i][j] = mfma<TX>(af[i], bfr[j], acc[i][j]);
        }
        if (kt + 1 < KT) store_stage(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue: 32x32 accumulator layout: lane holds column (lane % 32),
    // VGPR v holds row 8 (v / 4) + 4 (lane / 32) + v % 4 ----
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wn * 64 + j * 32 + (lane & 31);
            if (n >= N) continue;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = m0 + wm * 128 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (m < M) store_f(y, (size_t)m * N + n, out_dt, acc[i][j][v]);
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
    if (a.x_dtype == DT_BF16) return gemm::launch1<DT_BF16>(a, st);
    if (a.x_dtype == DT_F16) return gemm::launch1<DT_F16>(a, st);
    return LuxStatus::NotSupported;
}

}  // namespace lxq
