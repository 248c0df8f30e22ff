// qgemm_sk.h -- split-K small-M GEMM for 8 < M <= 64 (gfx950, MFMA): the GEMM
// semantics (weights dequantized to the activation type T, RNE of
// fmaf(s, q, b), fp32 accumulation), with x read once per 128 columns.
//
// A block owns a 128-column tile of the output (128 rows of W), all M rows of
// x, and one of S parts of K (S = 1: all of K).  Its 4 waves share the x tile
// of each super-step (128 codes of K) through LDS; wave w owns columns
// 32w..32w+31 and dequantizes its own W rows in registers.  The S parts of a
// tile meet through a workspace: each block writes its partial sums, and the
// block that finishes a tile last (a per-tile counter) adds the S partials
// in part order -- the same order whichever block is last, so results are
// deterministic -- and stores y.  That block sets the counter back to zero,
// so it reads zero again at the next launch (the workspace's counters start
// zeroed).
//
// Against the W-streaming kernel of qgemm_small.h (32 columns per block, K
// split over its 4 waves, x streamed once per block) x is read once per 128
// columns instead of once per 32, at the cost, when split, of the partials.
//
// MFMA v_mfma_f32_32x32x16_{bf16,f16}: A = x (rows m = lane % 32 of an M
// tile), B = W (column n = lane % 32).  Lane half h = lane / 32 owns codes
// [64 h, 64 h + 64) of each super-step (8 BITS contiguous bytes of its W
// row); sub-step s (0..7) takes codes 64 h + 8 s .. +8 of both halves, and
// the matching x values (chunk 8 h + s of row m).
//
// Every load returns into registers, PD super-steps ahead (x, W codes,
// scales and biases): each thread loads its share of the x tile (16-byte
// chunks, 16 threads per 256-byte row) and writes it into the LDS buffer of
// the next super-step; one barrier per super-step.  x chunk c of row m sits
// at chunk position c ^ (m % 16): the 16 lanes of a fragment read (16
// consecutive rows, one chunk) and of a write (one row, 16 chunks) touch 16
// distinct 16-byte slots of a 256-byte bank window.
#pragma once
#include <type_traits>

#include "qgemm_small.h"
#include "qsplit.h"

namespace lxq {
namespace sk {

using small::mfma;
using small::w_operand;

typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWaves = 4;
constexpr int kCols = 128;   // output columns (W rows) per block
constexpr int kSS = 128;     // codes of K per super-step
constexpr int PD = 4;        // super-steps of loads in flight (<= 168 VGPRs: 2 waves per SIMD)

// workspace: [tile counters: kCounterBytes]..[partials from kPartBase: tiles x S parts x M
// tiles x 16 KiB].  The counter region has one fixed size for every launch:
// K is split only when there are fewer than 256 tiles, and a counter slot
// must never be written by another shape's partials (its count would then
// never reach S)
constexpr int kMaxSplitTiles = 256;
constexpr size_t kCounterBytes = kMaxSplitTiles * 4;
// one part's partial sums of one tile: 32 rows x 128 columns of fp32 per M tile
constexpr size_t kPartTileBytes = 32 * kCols * 4;
// partial sums start past every GEMM's counter words (qsplit.h)
constexpr size_t kPartBase = split::kPartOffset;
static_assert(kCounterBytes <= split::kSkCounterBytes, "split-K counters within their workspace words");
__host__ __device__ constexpr size_t ws_bytes(int S, int M, int N) {
    return S > 1 ? kPartBase + (size_t)S * ((N + kCols - 1) / kCols) * ((M + 31) / 32) * kPartTileBytes : 0;
}
// buffer cache policy of the partials: device scope (sc1)
constexpr int kCachePolicyDevice = 16;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}

// the lane's 64 codes of a super-step: 8 BITS bytes at byte offset voff of its row
template <int BITS>
__device__ __forceinline__ void load_codes(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t* c) {
    constexpr int W = 2 * BITS;  // words
#pragma unroll
    for (int i = 0; i + 4 <= W; i += 4) {
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 4 * i, 0, 0);
        c[i] = v.x; c[i + 1] = v.y; c[i + 2] = v.z; c[i + 3] = v.w;
    }
    if constexpr (W % 4 == 2) {
        const u2 v = __builtin_amdgcn_raw_buffer_load_b64(r, voff + 4 * (W - 2), 0, 0);
        c[W - 2] = v.x; c[W - 1] = v.y;
    }
}

// a scale or bias as loaded: 16-bit values stay 16-bit until they are
// converted where used (a widening right after the load makes the compiler
// wait for that load there, draining the loads in flight behind it)
template <int SB>
using SbRaw = typename std::conditional<SB == DT_F32, uint32_t, uint16_t>::type;
template <int SB>
__device__ __forceinline__ SbRaw<SB> load_sb(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (SB == DT_F32) return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    else return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
template <int SB>
__device__ __forceinline__ float sb_val(SbRaw<SB> raw) {
    if constexpr (SB == DT_F32) return __uint_as_float(raw);
    else if constexpr (SB == DT_F16) return f16_to_f32(raw);
    else return bf16_to_f32(raw);
}

// LDS: two x buffers of MT*32 rows x 256 bytes
template <int MT>
struct Lay {
    static constexpr int kXBuf = MT * 32 * 256;
    static constexpr int kBytes = 2 * kXBuf;
};

__device__ __forceinline__ void lds_fence_barrier() {
    // this wave's LDS writes and reads are done; then every wave's are
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// NG: scale groups a lane's codes of one super-step span (2 for group size
// 32: sub-steps 0..3 and 4..7; else 1)
template <int BITS, int TX, int SB, int MT, int GS, bool EPI>
__global__ __launch_bounds__(64 * kWaves, 2) void qgemm_sk_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, void* __restrict__ y, int M, int K, int N, int S, void* __restrict__ ws,
    Epilogue ep) {
    using L = Lay<MT>;
    constexpr int NG = GS == 32 ? 2 : 1;
    constexpr int XR = 2 * MT;     // 16-byte x chunks per thread per super-step
    constexpr int CW = 2 * BITS;   // code words per lane per super-step
    __shared__ __attribute__((aligned(16))) uint8_t lds[L::kBytes];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31, h = lane >> 5;
    const int tile = blockIdx.x / S, part = blockIdx.x % S;
    const int n0 = tile * kCols;
    const int Kp = K / S;                    // a multiple of kSS
    const int k0 = part * Kp;
    const int nss = Kp / kSS;
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    const int G = K / GS;
    constexpr int kSb = SB == DT_F32 ? 4 : 2;

    // ---- per-thread addressing ----
    // x: chunk id = i * 256 + tid -> row r = id / 16 (clamped to M-1), chunk c = id % 16
    const auto xr = rsrc(x, (uint32_t)M * K * 2);
    uint32_t xoff[XR];
    int xlds[XR];
#pragma unroll
    for (int i = 0; i < XR; i++) {
        const int id = i * 256 + tid, r = id >> 4, c = id & 15;
        const int m = r < M ? r : M - 1;
        xoff[i] = ((uint32_t)m * K + (uint32_t)k0 + 8u * c) * 2u;
        xlds[i] = r * 256 + ((c ^ (r & 15)) << 4);
    }
    // W: the lane's row (rows past N re-read row N-1, never stored)
    const int nrow = min(n0 + 32 * wave + j, N - 1);
    const auto wr = rsrc(wq, (uint32_t)((size_t)N * row_bytes));
    const uint32_t woff = (uint32_t)nrow * row_bytes + (uint32_t)(k0 + 64 * h) * BITS / 8;
    const auto sr = rsrc(scales, (uint32_t)((size_t)N * G * kSb));
    const auto br = rsrc(biases, (uint32_t)((size_t)N * G * kSb));
    // group of sub-step 0 of the lane's half in super-step 0, and of sub-step 4 (group size 32)
    const uint32_t soff = ((uint32_t)nrow * G + (uint32_t)((k0 + 64 * h) / GS)) * kSb;

    uint32_t xv[PD][XR][4];
    uint32_t cw[PD][CW];
    SbRaw<SB> sv[PD][NG], bv[PD][NG];

    // the same buffers with no records: every access is out of range and
    // reads zeros without a memory request
    const auto xr0 = rsrc(x, 0), wr0 = rsrc(wq, 0), sr0 = rsrc(scales, 0), br0 = rsrc(biases, 0);
    auto issue = [&](int slot, int u, bool past) {
        // x tile, codes, scales and biases of super-step u into register
        // slot `slot`, as one batch in this order: the waits are counted in
        // issue order, so the scheduler may not move loads across batches.
        // `past` (uniform): a refill past the part's last super-step, issued
        // all the same (see the prologue) but from the empty buffers
        __builtin_amdgcn_sched_barrier(0);
        const auto xd = past ? xr0 : xr, wd = past ? wr0 : wr, sd = past ? sr0 : sr, bd = past ? br0 : br;
#pragma unroll
        for (int i = 0; i < XR; i++) {
            const u4 v = __builtin_amdgcn_raw_buffer_load_b128(xd, xoff[i] + (uint32_t)u * kSS * 2, 0, 0);
            xv[slot][i][0] = v.x; xv[slot][i][1] = v.y; xv[slot][i][2] = v.z; xv[slot][i][3] = v.w;
        }
        load_codes<BITS>(wd, woff + (uint32_t)u * kSS * BITS / 8, cw[slot]);
#pragma unroll
        for (int g = 0; g < NG; g++) {
            // group size 32: the second group of the half starts 32 codes later
            const uint32_t o = soff + ((uint32_t)u * kSS / GS + g) * kSb;
            sv[slot][g] = load_sb<SB>(sd, o);
            bv[slot][g] = load_sb<SB>(bd, o);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    auto write_x = [&](int slot, int buf) {
        uint8_t* xb = lds + buf * L::kXBuf;
#pragma unroll
        for (int i = 0; i < XR; i++)
            *reinterpret_cast<u4*>(xb + xlds[i]) = u4{xv[slot][i][0], xv[slot][i][1], xv[slot][i][2], xv[slot][i][3]};
    };

    f32x16 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[t][v] = 0.f;

    // Loads are issued unconditionally, past the part's last super-step too
    // (from the empty buffers, into a slot nothing reads): a conditional
    // issue leaves the compiler unable to count the loads in flight, and it
    // then drains them all before every super-step.
    // ---- prologue: super-steps 0 .. PD-1 in flight, x(0) into buffer 0 ----
#pragma unroll
    for (int p = 0; p < PD; p++) issue(p, min(p, nss - 1), p >= nss);
    write_x(0, 0);
    lds_fence_barrier();

    // super-step u from register slot `slot` and x buffer u & 1.  All of
    // the super-step's x fragments are read first: read where each MFMA
    // needs it, every sub-step waits out the LDS latency (measured: the
    // wave then waited most of its time)
    auto compute = [&](int slot, int u) {
        const uint8_t* xb = lds + (u & 1) * L::kXBuf;
        u4 a[8][MT];
#pragma unroll
        for (int s = 0; s < 8; s++)
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const int r = 32 * t + j, c = 8 * h + s;
                a[s][t] = *reinterpret_cast<const u4*>(xb + r * 256 + ((c ^ (r & 15)) << 4));
            }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int g = NG == 2 ? (s >> 2) : 0;
            const u4 wop = w_operand<BITS, TX>(cw[slot], sb_val<SB>(sv[slot][g]), sb_val<SB>(bv[slot][g]), s);
#pragma unroll
            for (int t = 0; t < MT; t++) acc[t] = mfma<TX>(a[s][t], wop, acc[t]);
        }
    };

    // ---- main loop: whole groups of PD super-steps, slot jj for super-step
    // g PD + jj.  No exit inside a group: on an exit path the refill's
    // loads are dead, and the compiler then sinks them past the barrier,
    // out of issue order. ----
    const int groups = nss / PD, rem = nss % PD;
    for (int g = 0; g < groups; g++) {
#pragma unroll
        for (int jj = 0; jj < PD; jj++) {
            const int u = g * PD + jj;
            // x of the next super-step into the other buffer (its last reader
            // finished before the previous barrier)
            if (u + 1 < nss) write_x((jj + 1) % PD, (u + 1) & 1);
            compute(jj, u);
            // refill this register slot with super-step u + PD
            issue(jj, min(u + PD, nss - 1), u + PD >= nss);
            lds_fence_barrier();
        }
    }
    // ---- the last nss % PD super-steps: slots 0 .. rem-1, no loads ----
#pragma unroll
    for (int jj = 0; jj < PD - 1; jj++) {
        if (jj < rem) {
            const int u = groups * PD + jj;
            if (u + 1 < nss) write_x(jj + 1, (u + 1) & 1);
            compute(jj, u);
            lds_fence_barrier();
        }
    }

    // ---- the S parts of the tile meet ----
    // 32x32 accumulator layout: lane holds column j (lane % 32), VGPR v row 8 (v/4) + 4 h + v % 4
    const int n = n0 + 32 * wave + j;
    if (S == 1) {
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
                if (m < M && n < N) store_out<EPI>(y, (size_t)m * N + n, n, ep, acc[t][v]);
            }
        return;
    }
    // The partials and counters cross blocks on different XCDs, whose L2s
    // are not coherent with each other: they are written and read only with
    // the device-scope cache policy (sc1), the instructions of the
    // compiler's device-scope atomic accesses, which need none of the L2
    // writeback and invalidate that a device-scope fence costs (measured:
    // such fences made a launch 4-5x slower).  As plain buffer accesses
    // they stay in flight together, where atomic loads are waited for one
    // by one.  Order: each wave's partial stores complete (vmcnt(0)), the
    // block meets at the barrier, then one thread counts the part in; the
    // block that counts last loads the partials after it has seen the count.
    //
    // A part's partial sums keep the accumulator's register layout: per M
    // tile t, row group q (rows 8q .. 8q+7, skipped at or past M) and wave,
    // 64 lanes x 16 bytes, so each lane moves 16-byte vectors.
    const int tiles = (int)gridDim.x / S;
    uint32_t* counters = static_cast<uint32_t*>(ws);
    const auto pr = rsrc(static_cast<uint8_t*>(ws) + kPartBase, (uint32_t)((size_t)tiles * S * MT * kPartTileBytes));
    auto part_off = [&](int q_part, int t, int q) {
        return (uint32_t)(((size_t)(tile * S + q_part) * MT + t) * kPartTileBytes) + (uint32_t)((q * kWaves + wave) * 1024 + lane * 16);
    };
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (32 * t + 8 * q < M)
                __builtin_amdgcn_raw_buffer_store_b128(
                    u4{__float_as_uint(acc[t][4 * q]), __float_as_uint(acc[t][4 * q + 1]),
                       __float_as_uint(acc[t][4 * q + 2]), __float_as_uint(acc[t][4 * q + 3])},
                    pr, part_off(part, t, q), 0, kCachePolicyDevice);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ uint32_t last;
    if (tid == 0) {
        const uint32_t before =
            __hip_atomic_fetch_add(&counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = before == (uint32_t)(S - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (last == 0u) return;
    // the last part of this tile: add the S partials in part order, store y,
    // and zero the counter again for the next launch
    if (tid == 0) __hip_atomic_store(&counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // parts in order (the same order whichever block is last); up to kPB
    // parts' row groups are loaded together, one memory round trip per kPB
    // parts (one part per trip left S round trips at the kernel's tail:
    // 7 parts, K = 3584, took 21 µs)
    constexpr int kPB = 4;
    float sum[MT][4][4];
    for (int q0 = 0; q0 < S; q0 += kPB) {
        u4 v[kPB][MT][4];
        // loads on every path (parts past S re-read part S - 1, row groups
        // past M their never-written slots; neither is used): a load on only
        // some paths makes the compiler drain the ones before it
#pragma unroll
        for (int pp = 0; pp < kPB; pp++) {
            const int qp = q0 + pp < S ? q0 + pp : S - 1;
#pragma unroll
            for (int t = 0; t < MT; t++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    v[pp][t][q] = __builtin_amdgcn_raw_buffer_load_b128(pr, part_off(qp, t, q), 0, kCachePolicyDevice);
        }
#pragma unroll
        for (int pp = 0; pp < kPB; pp++)
            if (q0 + pp < S)
#pragma unroll
                for (int t = 0; t < MT; t++)
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        if (32 * t + 8 * q < M) {
                            const float f[4] = {__uint_as_float(v[pp][t][q].x), __uint_as_float(v[pp][t][q].y),
                                                __uint_as_float(v[pp][t][q].z), __uint_as_float(v[pp][t][q].w)};
#pragma unroll
                            for (int e = 0; e < 4; e++)
                                sum[t][q][e] = q0 + pp == 0 ? f[e] : sum[t][q][e] + f[e];
                        }
    }
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = 32 * t + 8 * q + 4 * h + e;
                if (m < M && n < N) store_out<EPI>(y, (size_t)m * N + n, n, ep, sum[t][q][e]);
            }
}

// ---- launch ----

template <int BITS, int TX, int SB, int MT, int GS, bool EPI>
LuxStatus launch_e(const QmmArgs& a, int S, hipStream_t st) {
    static_assert(Lay<MT>::kBytes <= 64 * 1024, "static LDS");
    const int tiles = (a.N + kCols - 1) / kCols;
    if (planned(a, "qgemm_sk_kernel")) return LuxStatus::Ok;
    hipLaunchKernelGGL((qgemm_sk_kernel<BITS, TX, SB, MT, GS, EPI>), dim3(tiles * S), dim3(64 * kWaves), 0, st, a.x,
                       a.wq, a.scales, a.biases, a.y, a.M, a.K, a.N, S, a.ws, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

template <int BITS, int TX, int SB, int MT, int GS>
LuxStatus launch_ep(const QmmArgs& a, int S, hipStream_t st) {
    return a.has_epilogue() ? launch_e<BITS, TX, SB, MT, GS, true>(a, S, st)
                            : launch_e<BITS, TX, SB, MT, GS, false>(a, S, st);
}

template <int BITS, int TX, int SB, int MT>
LuxStatus launch_gs(const QmmArgs& a, int S, hipStream_t st) {
    switch (a.group_size) {
    case 32: return launch_ep<BITS, TX, SB, MT, 32>(a, S, st);
    case 64: return launch_ep<BITS, TX, SB, MT, 64>(a, S, st);
    default: return launch_ep<BITS, TX, SB, MT, 128>(a, S, st);
    }
}

template <int BITS, int TX, int SB>
LuxStatus launch_mt(const QmmArgs& a, int S, hipStream_t st) {
    return a.M <= 32 ? launch_gs<BITS, TX, SB, 1>(a, S, st) : launch_gs<BITS, TX, SB, 2>(a, S, st);
}

template <int BITS, int TX>
LuxStatus launch_sb(const QmmArgs& a, int S, hipStream_t st) {
    switch (a.sb_dtype) {
    case DT_F32: return launch_mt<BITS, TX, DT_F32>(a, S, st);
    case DT_F16: return launch_mt<BITS, TX, DT_F16>(a, S, st);
    default: return launch_mt<BITS, TX, DT_BF16>(a, S, st);
    }
}

// one translation unit per code width (qgemm_sk_b{2,3,4,5,6,8}.hip)
template <int BITS>
LuxStatus launch_bits(const QmmArgs& a, int S, hipStream_t st) {
    return a.x_dtype == DT_F16 ? launch_sb<BITS, DT_F16>(a, S, st) : launch_sb<BITS, DT_BF16>(a, S, st);
}

}  // namespace sk

}  // namespace lxq
