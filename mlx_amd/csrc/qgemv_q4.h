// qgemv_q4.h -- 2 <= M <= 8 rows of x, 4-bit codes, f16/bf16 x: the
// dequant-GEMV on v_mfma_f32_4x4x4_16b (gfx950), with 256-byte row segments
// per load instruction.
//
// A block is KW waves and owns RB = 4 RG consecutive rows of W; wave w owns
// CH chunks of 512 codes, codes 512 CH w .. 512 CH (w + 1) - 1 of K (K = 512
// CH KW with one chunk; with two, K <= 1024 KW and codes past K idle).  Lane l = 4 b + j of a wave is MFMA block b (b = l / 4) and column
// j (j = l % 4): for each 4-row group of the block and each chunk h it loads
// the 32 codes 512 (CH w + h) + 32 b .. + 31 of the group's row j with one
// 128-bit load.  So one wave load reads 4 rows x 16 lanes x 16 bytes, 256
// contiguous bytes of each row, where the 16-row MFMA decode kernel reads 64
// and the whole-line kernels 512 or 1024.  CH = 2 lets K up to 16384 run on
// at most 16 waves (long-K down projections at M <= 4); with CH = 1 the
// kernel is the one-chunk form used up to K = 8192.
//
// MFMA: v_mfma_f32_4x4x4_16b_{f16,bf16} runs 16 independent 4x4x4 products,
// block b on lanes 4 b .. 4 b + 3.  A = x (row i of block b on lane 4 b + i:
// rows 4 s + i of x for set s, the lane's 32 codes of K), B = the codes as
// the exact operands v = 1 + q / kPow of the MFMA decode kernel (column j on
// lane 4 b + j), D = the 4 x 4 block (lane 4 b + j, VGPR i: x row i, W row
// j).  A lane's 32 codes lie in one group (group sizes 32, 64, 128), so per
// 4-row group and set
//   D = sum v x = sx + sum q x / kPow over the lane's 32 codes,
//   s sum q x + b sx = kPow (s D + (b / kPow - s) sx),
// with sx = sum x over the lane's codes (of each row of the set: the lane's
// own row i = j, the others from its quad by DPP).  A lane's CH chunks each
// get their own factors (their groups differ) and are added, and then the
// 16 blocks' values are summed in registers (lane-half and row swaps, then
// row rotations by 4 and 8 lanes), parked in LDS, and after the last
// barrier thread t adds the KW waves' parts of value t in wave order and
// stores kPow times it.
//
// Load order, as in the whole-line kernels: x and the block's scale rows
// first (scale rows as 16-byte chunks over the block's threads), a block
// barrier, then the codes (non-temporal), groups in order; the scale rows go
// through LDS (a second barrier) to each lane's (row, group).
#pragma once
#include "qgemv_dec.h"
#include "qgemv_mx.h"

namespace lxq {
namespace q4 {

using dec::dec_code_operand;
using dec::DForm;
using gemv::buf_rsrc;
using gemv::kCachePolicyNT;
using gemv::kZeroOff;
using gemv::mx_sb_loads;
using gemv::sb_value;
using gemv::swap16_sum;
using gemv::swap32_sum;
using gemv::v4u32;

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

template <int TX>
__device__ __forceinline__ f4 mfma4(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, f4 c) {
    const u2 a = {a0, a1}, b = {b0, b1};
    if constexpr (TX == DT_F16)
        return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(h4, a), __builtin_bit_cast(h4, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s4, a), __builtin_bit_cast(s4, b), c, 0, 0,
                                                      0);
}

// LDS of the block: scale rows, bias rows (SBQ passes of the block's
// threads, 16 bytes each), then the waves' reduced values
template <int RG, int XS, int SBQ, int KW>
struct Q4Lds {
    static constexpr int kSbBytes = SBQ * KW * 64 * 16;
    static constexpr int kSb = 0, kBi = kSbBytes, kRed = 2 * kSbBytes;
    static constexpr int kBytes = kRed + KW * RG * XS * 16 * 4;
};

// XS: sets of 4 rows of x (M <= 4 XS)
template <int TX, int SB, int XS, int RG, int SBQ, int KW, bool EPI, int CH>
__global__ __launch_bounds__(64 * KW) void qgemv_q4_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, int gshift, Epilogue ep) {
    using L = Q4Lds<RG, XS, SBQ, KW>;
    using F = DForm<TX>;
    constexpr int kThreads = 64 * KW;
    constexpr int RB = 4 * RG;
    constexpr int kSb = SB == DT_F32 ? 4 : 2;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 3, blk = lane >> 2;
    const uint32_t kc = (uint32_t)(wave * 512 * CH + 32 * blk);  // the lane's first code; chunk h at kc + 512 h
    const uint32_t row_bytes = (uint32_t)K / 2;
    const int G = K >> gshift;
    const int n0 = blockIdx.x * RB;
    // with two chunks, K need not fill the waves (part of a chunk, a whole
    // chunk or whole waves idle): a lane's 32-code block past K (K % 32 =
    // 0) loads no x and no codes and gets zero factors, so it adds exactly 0
    bool in_k[CH];
#pragma unroll
    for (int h = 0; h < CH; h++) in_k[h] = CH == 1 || kc + 512u * h < (uint32_t)K;

    // ---- 1. x: rows 4 s + j, the lane's 32 codes (rows past M re-read row
    // M - 1; they are never stored) ----
    v4u32 xn[XS][CH][4];
    {
        const auto xr = buf_rsrc(x, (uint32_t)M * K * 2);
#pragma unroll
        for (int s = 0; s < XS; s++) {
            const int m = 4 * s + j < M ? 4 * s + j : M - 1;
            const uint32_t off = ((uint32_t)m * K + kc) * 2u;
#pragma unroll
            for (int h = 0; h < CH; h++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    xn[s][h][q] = __builtin_amdgcn_raw_buffer_load_b128(
                        xr, in_k[h] ? off + 1024u * h + 16 * q : kZeroOff, 0, 0);
        }
    }
    // ---- 2. the block's scale and bias rows, from the 16-byte chunk holding
    // the first: thread t loads chunks t, t + 64 KW, ... ----
    uint32_t sraw[SBQ][4], braw[SBQ][4];
    uint32_t s_lead;
    {
        const size_t sb_row = (size_t)G * kSb;
        const size_t sb_first = (size_t)n0 * sb_row;
        s_lead = (uint32_t)(sb_first & 15u);
        const size_t sb_base = sb_first - s_lead;
        const size_t stotal = (size_t)N * sb_row;
        // rows past N read zeros (never stored)
        const size_t sleft = sb_base < stotal ? ((stotal - sb_base + 15u) & ~(size_t)15u) : 0;
        const uint32_t sbytes = (uint32_t)(sleft < 0x7fffffffu ? sleft : 0x7fffffffu);
        const auto sr = buf_rsrc(static_cast<const uint8_t*>(scales) + sb_base, sbytes);
        const auto br = buf_rsrc(static_cast<const uint8_t*>(biases) + sb_base, sbytes);
        const uint32_t nch = (s_lead + (uint32_t)(RB * sb_row) + 15u) >> 4;
#pragma unroll
        for (int q = 0; q < SBQ; q++) {
            const uint32_t c = (uint32_t)(q * kThreads + tid);
            const uint32_t off = c < nch ? c * 16u : kZeroOff;
            const v4u32 a = __builtin_amdgcn_raw_buffer_load_b128(sr, off, 0, 0);
            const v4u32 b = __builtin_amdgcn_raw_buffer_load_b128(br, off, 0, 0);
            sraw[q][0] = a.x; sraw[q][1] = a.y; sraw[q][2] = a.z; sraw[q][3] = a.w;
            braw[q][0] = b.x; braw[q][1] = b.y; braw[q][2] = b.z; braw[q][3] = b.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // ---- 3. every wave's x and scale requests ahead of any code request ----
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // ---- 4. codes: row j of each 4-row group, 16 bytes per lane, groups in
    // order (rows past N re-read row N - 1, never stored) ----
    v4u32 w[RG][CH];
    {
        const size_t wleft = (size_t)(N - n0) * row_bytes;
        const auto wr = buf_rsrc(reinterpret_cast<const uint8_t*>(wq) + (size_t)n0 * row_bytes,
                                 (uint32_t)(wleft < 0x7fffffffu ? wleft : 0x7fffffffu));
#pragma unroll
        for (int rg = 0; rg < RG; rg++) {
            const int n = n0 + 4 * rg + j < N ? n0 + 4 * rg + j : N - 1;
            const uint32_t off = (uint32_t)(n - n0) * row_bytes + kc / 2;
#pragma unroll
            for (int h = 0; h < CH; h++)
                w[rg][h] = __builtin_amdgcn_raw_buffer_load_b128(wr, in_k[h] ? off + 256u * h : kZeroOff, 0,
                                                                 kCachePolicyNT);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 5. scale rows into LDS (every thread writes its chunks), published
    // by a barrier; then the lane's factors for each group ----
#pragma unroll
    for (int q = 0; q < SBQ; q++) {
        const int c = q * kThreads + tid;
        *reinterpret_cast<v4u32*>(lds + L::kSb + c * 16) = v4u32{sraw[q][0], sraw[q][1], sraw[q][2], sraw[q][3]};
        *reinterpret_cast<v4u32*>(lds + L::kBi + c * 16) = v4u32{braw[q][0], braw[q][1], braw[q][2], braw[q][3]};
    }
    __syncthreads();
    // c0 multiplies D, c1 multiplies sx: s and b / kPow - s
    float c0[RG][CH], c1[RG][CH];
#pragma unroll
    for (int hh = 0; hh < CH; hh++) {
        const uint32_t g = in_k[hh] ? (kc + 512u * hh) >> gshift : 0u;
#pragma unroll
        for (int rg = 0; rg < RG; rg++) {
            const uint32_t off = s_lead + ((uint32_t)(4 * rg + j) * G + g) * kSb;
            float s, b;
            if constexpr (SB == DT_F32) {
                s = *reinterpret_cast<const float*>(lds + L::kSb + off);
                b = *reinterpret_cast<const float*>(lds + L::kBi + off);
            } else {
                s = sb_value<SB>(*reinterpret_cast<const uint16_t*>(lds + L::kSb + off));
                b = sb_value<SB>(*reinterpret_cast<const uint16_t*>(lds + L::kBi + off));
            }
            c0[rg][hh] = in_k[hh] ? s : 0.f;
            c1[rg][hh] = in_k[hh] ? fmaf(b, 1.f / F::kPow, -s) : 0.f;
        }
    }

    // ---- 6. x operands (the code operands' order) and sums of x: the
    // lane's own row 4 s + j, then rows 4 s + i from lane 4 b + i ----
    v4u32 xo[XS][CH][4];
    float sxq[XS][CH][4];
    {
        const uint32_t one2 = TX == DT_F16 ? 0x3C003C00u : 0x3F803F80u;
#pragma unroll
        for (int s = 0; s < XS; s++)
#pragma unroll
            for (int h = 0; h < CH; h++) {
                float sx = 0.f;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    xo[s][h][q] = skinny::x_operand<4, TX>(xn[s][h][q]);
                    sx = dot2(xn[s][h][q].x, one2, sx, TX);
                    sx = dot2(xn[s][h][q].y, one2, sx, TX);
                    sx = dot2(xn[s][h][q].z, one2, sx, TX);
                    sx = dot2(xn[s][h][q].w, one2, sx, TX);
                }
                sxq[s][h][0] = dpp_f<0x00>(sx);  // quad_perm [0,0,0,0]
                sxq[s][h][1] = dpp_f<0x55>(sx);  // quad_perm [1,1,1,1]
                sxq[s][h][2] = dpp_f<0xAA>(sx);  // quad_perm [2,2,2,2]
                sxq[s][h][3] = dpp_f<0xFF>(sx);  // quad_perm [3,3,3,3]
            }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 7. groups in arrival order: 8 MFMAs per set over the lane's 32
    // codes, the factors, then the 16 blocks' sum; lanes 16 r + c (c < 4)
    // hold value (x row 4 s + pi(r), W row 4 rg + c), pi = 0 2 1 3 ----
    float* red = reinterpret_cast<float*>(lds + L::kRed);
    uint32_t vm = F::kMask, vmagic = F::kMagic;
    asm volatile("" : "+v"(vm), "+v"(vmagic));
#pragma unroll
    for (int rg = 0; rg < RG; rg++) {
        v4u32 bop[CH][4];
#pragma unroll
        for (int h = 0; h < CH; h++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const auto o = dec_code_operand<TX>(w[rg][h][q], vm, vmagic);
                bop[h][q] = v4u32{o.x, o.y, o.z, o.w};
            }
#pragma unroll
        for (int s = 0; s < XS; s++) {
            f4 d[CH];
#pragma unroll
            for (int h = 0; h < CH; h++) {
                d[h] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    d[h] = mfma4<TX>(xo[s][h][q].x, xo[s][h][q].y, bop[h][q].x, bop[h][q].y, d[h]);
                    d[h] = mfma4<TX>(xo[s][h][q].z, xo[s][h][q].w, bop[h][q].z, bop[h][q].w, d[h]);
                }
            }
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[i] = fmaf(c0[rg][0], d[0][i], c1[rg][0] * sxq[s][0][i]);
#pragma unroll
                for (int h = 1; h < CH; h++) v[i] += fmaf(c0[rg][h], d[h][i], c1[rg][h] * sxq[s][h][i]);
            }
            // the 4 rows of 16 lanes (lane-half and row swaps: row r then
            // holds value pi(r)), then the 4 quads of each row
            float z = swap16_sum(swap32_sum(v[0], v[1]), swap32_sum(v[2], v[3]));
            z += dpp_f<0x124>(z);  // row_ror:4
            z += dpp_f<0x128>(z);  // row_ror:8
            if ((lane & 15) < 4) {
                const int r = lane >> 4, i = ((r & 1) << 1) | (r >> 1);
                red[((wave * RG + rg) * XS + s) * 16 + 4 * i + (lane & 3)] = z;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- 8. the KW waves' parts of each value, in wave order; store ----
    __syncthreads();
    if (tid < RG * XS * 16) {
        const int rg = tid / (XS * 16), s = (tid / 16) % XS, i = (tid >> 2) & 3, jj = tid & 3;
        float z = red[tid];
#pragma unroll
        for (int v = 1; v < KW; v++) z += red[v * RG * XS * 16 + tid];
        z *= F::kPow;
        const int m = 4 * s + i, n = n0 + 4 * rg + jj;
        if (m < M && n < N) store_out<EPI>(y, (size_t)m * N + n, n, ep, z);
    }
}

// Rows per block: 28 where that spreads the blocks over the 256 CUs more
// evenly than 16 (as the K-split whole-line kernel)
template <int TX, int SB, int XS, int RG, int SBQ, int KW, int CH>
LuxStatus launch_k(const QmmArgs& a, hipStream_t st) {
    using L = Q4Lds<RG, XS, SBQ, KW>;
    static_assert(L::kBytes <= 160 * 1024, "LDS");
    if (planned(a, "qgemv_q4_kernel")) return LuxStatus::Ok;
    if constexpr (L::kBytes > 64 * 1024) {
        // once per instantiation (a function-local static initializes once)
        static const hipError_t attr[2] = {
            hipFuncSetAttribute(reinterpret_cast<const void*>(qgemv_q4_kernel<TX, SB, XS, RG, SBQ, KW, true, CH>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes),
            hipFuncSetAttribute(reinterpret_cast<const void*>(qgemv_q4_kernel<TX, SB, XS, RG, SBQ, KW, false, CH>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes)};
        if (attr[0] != hipSuccess || attr[1] != hipSuccess) return LuxStatus::Internal;
    }
    const int gshift = a.group_size == 32 ? 5 : a.group_size == 64 ? 6 : 7;
    const int blocks = (a.N + 4 * RG - 1) / (4 * RG);
    if (a.has_epilogue())
        hipLaunchKernelGGL((qgemv_q4_kernel<TX, SB, XS, RG, SBQ, KW, true, CH>), dim3(blocks), dim3(64 * KW), L::kBytes,
                           st, a.x, a.wq, a.scales, a.biases, a.y, a.M, a.K, a.N, gshift, a.epi());
    else
        hipLaunchKernelGGL((qgemv_q4_kernel<TX, SB, XS, RG, SBQ, KW, false, CH>), dim3(blocks), dim3(64 * KW), L::kBytes,
                           st, a.x, a.wq, a.scales, a.biases, a.y, a.M, a.K, a.N, gshift, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

}  // namespace q4
}  // namespace lxq
