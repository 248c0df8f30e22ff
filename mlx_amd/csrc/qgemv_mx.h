// qgemv_mx.h -- 2..4 rows of x, K <= 16384: the dequant-GEMV that streams
// whole cache lines with the waves of a block splitting K (gfx950).
//
// Included after qgemv_line.h (it uses the whole-line kernel's operand forms
// and partials on 16-code chunks) by the per-bit-width translation units.
//
// A block is KW waves (4, 8 or 16: each covers at most 1024 codes) and owns
// RB consecutive rows of W; wave w owns part w of K (K / KW codes) for all
// RB rows, and lane l the 16 codes 16 l .. 16 l + 15 of that part.  So one
// wave load per row reads 64 lanes x 16 codes, contiguous (512 B at 4-bit
// codes: whole 128-byte lines), and a lane holds the x operands of its 16
// codes for each of the MX rows of x (8 words per row at 16-bit x, 16 at f32
// x, where a wave covering all of K = 4096 would need 32 or 64).
// Every load is issued at the start, straight into registers:
//   1. x: the lane's 16 x values of each of the MX rows;
//   2. the block's RB scale rows and RB bias rows (contiguous in the scale
//      arrays), as 16-byte chunks split over the block's threads;
//   3. a block barrier, so the x and scale requests of all the waves enter
//      the CU's vector-memory queue ahead of every code request;
//   4. the codes: one non-temporal wave load per row, rows in order.
// The scale rows are written to LDS (a second barrier publishes them: the
// scale loads were issued before the codes, so waiting for them leaves the
// codes in flight) and each lane reads the scale and bias of its group in
// each row.  Rows are computed in arrival order, MX partials per row from
// the same code words; every 8 partials (8 / MX rows) are reduced across the
// wave together (sum8) and parked in LDS; after a last barrier, thread t
// adds the KW waves' parts of value t in wave order and stores it.
#pragma once
#include "qgemv_line.h"

namespace lxq {
namespace gemv {

template <int BITS>
struct MxCfg {
    static constexpr bool kOk = BITS == 2 || BITS == 4 || BITS == 8;
    static constexpr int NC = 16;                 // codes per lane per row
    static constexpr int WPL = NC * BITS / 32;    // code words per lane per row
};

// LDS of the block: scale rows, bias rows (SBQ passes of the block's
// threads, 16 bytes each), then the waves' reduced partials
template <int RB, int MX, int SBQ, int KW>
struct MxLds {
    static constexpr int kSbBytes = SBQ * KW * 64 * 16;
    static constexpr int kSb = 0, kBi = kSbBytes, kRed = 2 * kSbBytes;
    static constexpr int kBytes = kRed + KW * RB * MX * 4;
};

// passes of KW * 64 threads x 16 bytes that cover RB scale rows of G groups
// plus the lead of the first row within its 16-byte chunk
inline int mx_sb_loads(int RB, int G, int sb_dtype, int KW) {
    const int pass = KW * 64 * 16;
    const int q = (RB * G * (sb_dtype == DT_F32 ? 4 : 2) + 15 + pass - 1) / pass;
    return q <= 1 ? 1 : q <= 2 ? 2 : 4;
}

template <int BITS, int TX, int SB, int MX, int RB, int SBQ, int KW, bool EPI>
__global__ __launch_bounds__(64 * KW) void qgemv_mx_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, int gshift, Epilogue ep) {
    using C = MxCfg<BITS>;
    using L = MxLds<RB, MX, SBQ, KW>;
    constexpr int kThreads = 64 * KW;
    constexpr int OP = op_kind<BITS, TX>();
    constexpr int NC = C::NC, WPL = C::WPL;
    constexpr int XE = TX == DT_F32 ? 4 : 2;
    constexpr int XW = NC * XE / 4;  // 32-bit words of x per row of x
    constexpr int kSb = SB == DT_F32 ? 4 : 2;
    constexpr int VPB = 8 / MX;  // rows per reduction batch
    static_assert(MX == 2 || MX == 4, "rows of x");
    static_assert(RB % VPB == 0, "whole reduction batches");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kq = K / KW;                                        // codes per wave part
    const bool ok = lane * NC < kq;                               // lanes past the part read zeros
    const uint32_t kc = (uint32_t)(wave * kq + lane * NC);        // the lane's first code
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    const int G = K >> gshift;
    const int n0 = blockIdx.x * RB;

    // ---- 1. x of the lane's 16 codes, each row of x (rows past M re-read
    // row M-1; they are never stored) ----
    uint32_t xn[MX][XW];
    {
        const auto xr = buf_rsrc(x, (uint32_t)M * K * XE);
#pragma unroll
        for (int m = 0; m < MX; m++) {
            const int mr = m < M ? m : M - 1;
            const uint32_t off = ok ? ((uint32_t)mr * K + kc) * XE : kZeroOff;
#pragma unroll
            for (int j = 0; j < XW / 4; j++) {
                const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16 * j, 0, 0);
                xn[m][4 * j] = v.x; xn[m][4 * j + 1] = v.y; xn[m][4 * j + 2] = v.z; xn[m][4 * j + 3] = v.w;
            }
        }
    }
    // ---- 2. the block's scale and bias rows, from the 16-byte chunk
    // holding the first: thread t loads chunks t, t + 64 KW, ... ----
    constexpr int kSbQ = SBQ;  // chunks per thread
    uint32_t sraw[kSbQ][4], braw[kSbQ][4];
    uint32_t s_lead, nch;
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
        nch = (s_lead + (uint32_t)(RB * sb_row) + 15u) >> 4;
#pragma unroll
        for (int q = 0; q < kSbQ; q++) {
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
    // ---- 4. codes: a quarter row per wave load, non-temporal, rows in order ----
    uint32_t w[RB][WPL];
    {
        const size_t wleft = (size_t)(N - n0) * row_bytes;
        const auto wr = buf_rsrc(reinterpret_cast<const uint8_t*>(wq) + (size_t)n0 * row_bytes,
                                 (uint32_t)(wleft < 0x7fffffffu ? wleft : 0x7fffffffu));
        const uint32_t voff = ok ? kc * BITS / 8 : kZeroOff;
#pragma unroll
        for (int r = 0; r < RB; r++) {
            const int n = n0 + r < N ? n0 + r : N - 1;
            const uint32_t soff = (uint32_t)(n - n0) * row_bytes;
            if constexpr (WPL == 4) {
                const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(wr, voff, soff, kCachePolicyNT);
                w[r][0] = v.x; w[r][1] = v.y; w[r][2] = v.z; w[r][3] = v.w;
            } else if constexpr (WPL == 2) {
                const v2u32 v = __builtin_amdgcn_raw_buffer_load_b64(wr, voff, soff, kCachePolicyNT);
                w[r][0] = v.x; w[r][1] = v.y;
            } else {
                w[r][0] = __builtin_amdgcn_raw_buffer_load_b32(wr, voff, soff, kCachePolicyNT);
            }
            // rows issued in order: they are computed in this order
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 5. scale rows into LDS (every thread writes its chunks, so no
    // lane-dependent use can pull the loads past the codes), published by a
    // barrier; then the lane's scale and bias in each row ----
#pragma unroll
    for (int q = 0; q < kSbQ; q++) {
        const int c = q * kThreads + tid;
        *reinterpret_cast<v4u32*>(lds + L::kSb + c * 16) = v4u32{sraw[q][0], sraw[q][1], sraw[q][2], sraw[q][3]};
        *reinterpret_cast<v4u32*>(lds + L::kBi + c * 16) = v4u32{braw[q][0], braw[q][1], braw[q][2], braw[q][3]};
    }
    __syncthreads();
    float sc[RB], bi[RB];
    {
        const uint32_t g = ok ? kc >> gshift : 0u;  // a 16-code chunk lies in one group (g >= 32)
#pragma unroll
        for (int r = 0; r < RB; r++) {
            const uint32_t off = s_lead + ((uint32_t)r * G + g) * kSb;
            if constexpr (SB == DT_F32) {
                sc[r] = *reinterpret_cast<const float*>(lds + L::kSb + off);
                bi[r] = *reinterpret_cast<const float*>(lds + L::kBi + off);
            } else {
                sc[r] = sb_value<SB>(*reinterpret_cast<const uint16_t*>(lds + L::kSb + off));
                bi[r] = sb_value<SB>(*reinterpret_cast<const uint16_t*>(lds + L::kBi + off));
            }
            // lanes past the part hold zero codes and x: their partial is exactly 0
            if (!ok) { sc[r] = 0.f; bi[r] = 0.f; }
        }
    }

    // ---- 6. x operands ----
    LineX<BITS, TX, OP, NC> xo[MX];
#pragma unroll
    for (int m = 0; m < MX; m++) prep_line_x<BITS, TX, OP, NC>(xn[m], xo[m]);
    __builtin_amdgcn_sched_barrier(0);

    // ---- 7. rows in arrival order; every VPB rows, their 8 partials are
    // reduced across the wave and parked in LDS ----
    float* red = reinterpret_cast<float*>(lds + L::kRed);
#pragma unroll
    for (int rb = 0; rb < RB; rb += VPB) {
        float acc[8];
#pragma unroll
        for (int rr = 0; rr < VPB; rr++) {
#pragma unroll
            for (int m = 0; m < MX; m++)
                acc[rr * MX + m] = line_partial<BITS, TX, OP, false, NC>(w[rb + rr], xo[m], sc[rb + rr], bi[rb + rr],
                                                                        0.f, 0.f);
            __builtin_amdgcn_sched_barrier(0);
        }
        const float z = sum8(acc, lane);
        if ((lane & 7) == 0) red[wave * RB * MX + rb * MX + sum8_index(lane)] = z;
    }

    // ---- 8. the KW waves' parts of each value, in wave order; store ----
    __syncthreads();
    if (tid < RB * MX) {
        const int r = tid / MX, m = tid % MX, n = n0 + r;
        float z = red[tid];
#pragma unroll
        for (int v = 1; v < KW; v++) z += red[v * RB * MX + tid];
        z *= out_scale<OP>();
        if (m < M && n < N) store_out<EPI>(y, (size_t)m * N + n, n, ep, z);
    }
}

// Rows per block: 28 where that spreads the blocks over the 256 CUs more
// evenly than 16 (N = 14336: 512 blocks, 2 per CU, against 896), else 16.
inline int mx_rows(int N) {
    auto balance = [](int blocks) {
        const int rounds = (blocks + 255) / 256;
        return (double)blocks / (256.0 * rounds);
    };
    return balance((N + 27) / 28) > balance((N + 15) / 16) + 0.05 ? 28 : 16;
}

template <int BITS, int TX, int SB, int MX, int RB, int SBQ, int KW>
LuxStatus launch_mx_k(const QmmArgs& a, hipStream_t st) {
    using L = MxLds<RB, MX, SBQ, KW>;
    static_assert(L::kBytes <= 160 * 1024, "LDS");
    if (planned(a, "qgemv_mx_kernel")) return LuxStatus::Ok;
    if constexpr (L::kBytes > 64 * 1024) {
        // once per instantiation (a function-local static initializes once)
        static const hipError_t attr[2] = {
            hipFuncSetAttribute(reinterpret_cast<const void*>(qgemv_mx_kernel<BITS, TX, SB, MX, RB, SBQ, KW, true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes),
            hipFuncSetAttribute(reinterpret_cast<const void*>(qgemv_mx_kernel<BITS, TX, SB, MX, RB, SBQ, KW, false>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes)};
        if (attr[0] != hipSuccess || attr[1] != hipSuccess) return LuxStatus::Internal;
    }
    const int gshift = a.group_size == 32 ? 5 : a.group_size == 64 ? 6 : 7;
    const int blocks = (a.N + RB - 1) / RB;
    if (a.has_epilogue())
        hipLaunchKernelGGL((qgemv_mx_kernel<BITS, TX, SB, MX, RB, SBQ, KW, true>), dim3(blocks), dim3(64 * KW),
                           L::kBytes, st,
                           a.x, a.wq, a.scales, a.biases, a.y, a.M, a.K, a.N, gshift, a.epi());
    else
        hipLaunchKernelGGL((qgemv_mx_kernel<BITS, TX, SB, MX, RB, SBQ, KW, false>), dim3(blocks), dim3(64 * KW),
                           L::kBytes, st,
                           a.x, a.wq, a.scales, a.biases, a.y, a.M, a.K, a.N, gshift, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

template <int BITS, int TX, int SB, int MX, int RB, int KW>
LuxStatus launch_mx_q(const QmmArgs& a, hipStream_t st) {
    switch (mx_sb_loads(RB, a.K / a.group_size, SB, KW)) {
    case 1: return launch_mx_k<BITS, TX, SB, MX, RB, 1, KW>(a, st);
    case 2: return launch_mx_k<BITS, TX, SB, MX, RB, 2, KW>(a, st);
    default: return launch_mx_k<BITS, TX, SB, MX, RB, 4, KW>(a, st);
    }
}

// waves per block: each covers at most 1024 codes of K; 8 waves (2 per
// SIMD, 256 VGPRs) take 16-row blocks, 16 waves (4 per SIMD, 128 VGPRs) 16
// rows of codes up to 4 bits and 8 rows of 8-bit codes (16 rows of 8-bit
// codes are 64 VGPRs of code words alone and spilled to scratch), half that
// with f32 x (16 VGPRs of x per row of x)
template <int BITS, int TX, int SB, int MX>
LuxStatus launch_mx_r(const QmmArgs& a, hipStream_t st) {
    constexpr int RB16 = (BITS == 8 ? 8 : 16) / (TX == DT_F32 ? 2 : 1);
    if (a.K > 8192) return launch_mx_q<BITS, TX, SB, MX, RB16, 16>(a, st);
    if (a.K > 4096) return launch_mx_q<BITS, TX, SB, MX, 16, 8>(a, st);
    return mx_rows(a.N) == 28 ? launch_mx_q<BITS, TX, SB, MX, 28, 4>(a, st) : launch_mx_q<BITS, TX, SB, MX, 16, 4>(a, st);
}

template <int BITS, int TX, int SB>
LuxStatus launch_mx_m(const QmmArgs& a, hipStream_t st) {
    return a.M <= 2 ? launch_mx_r<BITS, TX, SB, 2>(a, st) : launch_mx_r<BITS, TX, SB, 4>(a, st);
}

// Where this kernel runs (f16 x unless noted, µs per launch against the
// kernels AUTO picked before it, same box):
//  * K = 4096, N = 14336: 8-bit codes M = 2 / 3 / 4 13.75 / 16.51 / 17.04
//    against 14.17 / 18.71 / 19.58 (stream kernel); 2-bit M = 3 / 4 13.17 /
//    13.64 against 14.54 / 14.76 (stream); 4-bit M = 2 10.11 against 10.91
//    (stream).  Elsewhere at K <= 4096 it loses: its v_dot2 arithmetic (about
//    3.6 VALU instructions per code at M = 4) no longer hides under the
//    stream, and the MFMA decode kernel wins (4-bit M = 3 / 4: 14.0 / 14.1
//    against 11.9 / 13.0; bf16 x 4-bit M = 4: 15.8 against 12.7), as does the
//    stream kernel at 2-bit M = 2 (9.35 against 8.95) and bf16 4-bit M = 2
//    (11.29 against 10.95).
//  * K > 8192 (down projections, where the decode kernel stops and the
//    LDS-ring kernel took M >= 3): K = 14336, N = 4096, 4-bit M = 2 / 3 / 4
//    12.6 / 17.3 / 17.4 against 15.7 / 25.2 / 25.3, bf16 x M = 4 18.2 against
//    25.6, 8-bit M = 4 22.3 against 27.5; K = 16384 g128 M = 4 18.7 against
//    24.5.
//  * 4096 < K <= 8192: M = 2 (K = N = 8192, 4-bit: 12.0 against 13.4) and
//    2-bit codes (which no MFMA kernel takes); the decode kernel keeps 4-bit
//    M >= 3 (K = 8192: 14.2 against 15.8; K = 6144 M = 3: 11.1 against 14.7)
//    and the LDS-ring kernel 8-bit M >= 3 (K = 8192 g128 bf16 M = 4: 20.3
//    against 24.2).
//  * f32 x: everywhere it applies.  The alternative for f32 x at M >= 2 is
//    one M = 1 launch per row (the row-run kernel it replaced was 5-6x slower:
//    M = 4, K = N = 4096, 4-bit: 33.0 us).
inline bool mx_wins(int bits, int M, int x_dtype, int K) {
    if (x_dtype == DT_F32 || K > 8192) return true;
    if (K > 4096) return M == 2 || bits == 2;
    return bits == 8 || (bits == 2 && M >= 3) || (bits == 4 && M == 2 && x_dtype == DT_F16);
}

// 2 <= M <= 4, 2/4/8-bit codes where it wins (mx_wins), K <= 16384
// with each wave's part of K a whole number of 16-code chunks; NotSupported
// otherwise
template <int BITS>
LuxStatus launch_mx_b(const QmmArgs& a, hipStream_t st) {
    if constexpr (!MxCfg<BITS>::kOk) {
        return LuxStatus::NotSupported;
    } else {
        // each wave's part of K a whole number of 16-code chunks
        const int kw = a.K > 8192 ? 16 : a.K > 4096 ? 8 : 4;
        if (a.M < 2 || a.M > 4 || a.K > 16384 || a.K % (16 * kw) != 0 ||
            !mx_wins(BITS, a.M, a.x_dtype, a.K))
            return LuxStatus::NotSupported;
        // offsets within the 32-bit buffer ranges
        if ((size_t)a.N * a.K * BITS / 8 >= (1ull << 31)) return LuxStatus::NotSupported;
        if (a.x_dtype == DT_F32) {
            switch (a.sb_dtype) {
            case DT_F32: return launch_mx_m<BITS, DT_F32, DT_F32>(a, st);
            case DT_F16: return launch_mx_m<BITS, DT_F32, DT_F16>(a, st);
            default: return launch_mx_m<BITS, DT_F32, DT_BF16>(a, st);
            }
        }
        if (a.x_dtype == DT_F16) {
            switch (a.sb_dtype) {
            case DT_F32: return launch_mx_m<BITS, DT_F16, DT_F32>(a, st);
            case DT_F16: return launch_mx_m<BITS, DT_F16, DT_F16>(a, st);
            default: return launch_mx_m<BITS, DT_F16, DT_BF16>(a, st);
            }
        }
        switch (a.sb_dtype) {
        case DT_F32: return launch_mx_m<BITS, DT_BF16, DT_F32>(a, st);
        case DT_F16: return launch_mx_m<BITS, DT_BF16, DT_F16>(a, st);
        default: return launch_mx_m<BITS, DT_BF16, DT_BF16>(a, st);
        }
    }
}

}  // namespace gemv
}  // namespace lxq
