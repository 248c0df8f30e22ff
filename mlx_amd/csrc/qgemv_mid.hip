// qgemv_mid.hip -- launcher of the exact-form mid-M MFMA kernel (qgemv_mid.h).
#include "qgemv_mid.h"

namespace lxq {
namespace mid {

template <int BITS, int TX, int SB, int GS, int XR, bool EPI>
LuxStatus launch_e(const QmmArgs& a, hipStream_t st) {
    using L = Lay<BITS, SB, GS, XR>;
    static_assert(L::kBytes <= 160 * 1024, "LDS");
    if (planned(a, "qgemv_mid_kernel")) return LuxStatus::Ok;
    auto kern = qgemv_mid_kernel<BITS, TX, SB, GS, XR, EPI>;
    // once per instantiation; a function-local static initializes exactly once
    // even when several threads make the first call together
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes);
    if (attr != hipSuccess) return LuxStatus::Internal;
    hipLaunchKernelGGL(kern, dim3((a.N + 31) / 32), dim3(64 * kWaves), L::kBytes, st, a.x, a.wq, a.scales, a.biases,
                       a.y, a.M, a.K, a.N, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

template <int BITS, int TX, int SB, int GS, int XR>
LuxStatus launch(const QmmArgs& a, hipStream_t st) {
    return a.has_epilogue() ? launch_e<BITS, TX, SB, GS, XR, true>(a, st)
                            : launch_e<BITS, TX, SB, GS, XR, false>(a, st);
}

// one x DMA (8 rows) per step for M <= 8, two for M <= 16
template <int BITS, int TX, int SB, int GS>
LuxStatus launch_xr(const QmmArgs& a, hipStream_t st) {
    return a.M <= 8 ? launch<BITS, TX, SB, GS, 1>(a, st) : launch<BITS, TX, SB, GS, 2>(a, st);
}

template <int BITS, int TX, int SB>
LuxStatus launch_gs(const QmmArgs& a, hipStream_t st) {
    switch (a.group_size) {
    case 32: return launch_xr<BITS, TX, SB, 32>(a, st);
    case 64: return launch_xr<BITS, TX, SB, 64>(a, st);
    case 128: return launch_xr<BITS, TX, SB, 128>(a, st);
    default: return LuxStatus::NotSupported;
    }
}

template <int BITS, int TX>
LuxStatus launch_sb(const QmmArgs& a, hipStream_t st) {
    switch (a.sb_dtype) {
    case DT_F32: return launch_gs<BITS, TX, DT_F32>(a, st);
    case DT_F16: return launch_gs<BITS, TX, DT_F16>(a, st);
    default: return launch_gs<BITS, TX, DT_BF16>(a, st);
    }
}

}  // namespace mid

LuxStatus launch_qgemv_mid(const QmmArgs& a, hipStream_t st) {
    using namespace mid;
    if (a.M < 2 || a.M > 16 || (a.bits != 4 && a.bits != 8) || a.x_dtype == DT_F32 || a.K % 1024 != 0)
        return LuxStatus::NotSupported;
    // 32-bit DMA offsets
    if ((size_t)a.M * a.K * 2 >= (1ull << 31) || (size_t)a.N * a.K * a.bits / 8 >= (1ull << 31))
        return LuxStatus::NotSupported;
    if (a.bits == 4) return a.x_dtype == DT_F16 ? launch_sb<4, DT_F16>(a, st) : launch_sb<4, DT_BF16>(a, st);
    return a.x_dtype == DT_F16 ? launch_sb<8, DT_F16>(a, st) : launch_sb<8, DT_BF16>(a, st);
}

}  // namespace lxq
