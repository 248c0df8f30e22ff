// qgemm_small.hip -- launcher of the small-M MFMA GEMM (kernel in qgemm_small.h).
#include "qgemm_small.h"

namespace lxq {
namespace small {

template <int BITS, int TX, int SB, int MT, int GS, bool EPI>
LuxStatus launch_e(const QmmArgs& a, hipStream_t st) {
    using L = Lay<BITS, SB, MT, GS>;
    static_assert(L::kBytes <= 160 * 1024, "LDS");
    auto kern = qgemm_small_kernel<BITS, TX, SB, MT, GS, EPI>;
    // once per instantiation; a function-local static initializes exactly once
    // even when several threads make the first call together
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes);
    if (attr != hipSuccess) return LuxStatus::Internal;
    hipLaunchKernelGGL(kern, dim3((a.N + 31) / 32), dim3(64 * kWaves), L::kBytes, st, a.x, a.wq, a.scales, a.biases,
                       a.y, a.M, a.K, a.N, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

template <int BITS, int TX, int SB, int MT, int GS>
LuxStatus launch(const QmmArgs& a, hipStream_t st) {
    return a.has_epilogue() ? launch_e<BITS, TX, SB, MT, GS, true>(a, st)
                            : launch_e<BITS, TX, SB, MT, GS, false>(a, st);
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

template <int BITS>
LuxStatus launch_tx(const QmmArgs& a, hipStream_t st) {
    return a.x_dtype == DT_F16 ? launch_sb<BITS, DT_F16>(a, st) : launch_sb<BITS, DT_BF16>(a, st);
}

}  // namespace small

LuxStatus launch_qgemm_small(const QmmArgs& a, hipStream_t st) {
    using namespace small;
    if (a.M <= 8 || a.M > 64 || a.x_dtype == DT_F32 || a.K % 1024 != 0) return LuxStatus::NotSupported;
    // 32-bit DMA offsets
    if ((size_t)a.M * a.K * 2 >= (1ull << 31) || (size_t)a.N * a.K * a.bits / 8 >= (1ull << 31))
        return LuxStatus::NotSupported;
    switch (a.bits) {
    case 2: return launch_tx<2>(a, st);
    case 3: return launch_tx<3>(a, st);
    case 4: return launch_tx<4>(a, st);
    case 5: return launch_tx<5>(a, st);
    case 6: return launch_tx<6>(a, st);
    case 8: return launch_tx<8>(a, st);
    default: return LuxStatus::NotSupported;
    }
}

}  // namespace lxq
