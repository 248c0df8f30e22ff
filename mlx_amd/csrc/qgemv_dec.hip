// qgemv_dec.hip -- launcher of the MFMA decode kernel (qgemv_dec.h).
#include "qgemv_dec.h"

namespace lxq {
namespace dec {

template <int TX, int SB, int GS, bool EPI>
LuxStatus launch_e(const QmmArgs& a, hipStream_t st) {
    const size_t lds = dec_lds_bytes(a.M, a.K);
    if (lds > 160 * 1024) return LuxStatus::NotSupported;
    auto kern = qgemv_dec_kernel<TX, SB, GS, EPI>;
    static bool attr_set = false;  // one per instantiation
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024) != hipSuccess)
            return LuxStatus::Internal;
        attr_set = true;
    }
    const int blocks = (a.N + 16 * kTiles - 1) / (16 * kTiles);
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * (a.K / kKW)), lds, st, a.x, a.wq, a.scales, a.biases, a.y, a.M,
                       a.K, a.N, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

template <int TX, int SB, int GS>
LuxStatus launch(const QmmArgs& a, hipStream_t st) {
    return a.has_epilogue() ? launch_e<TX, SB, GS, true>(a, st) : launch_e<TX, SB, GS, false>(a, st);
}

template <int TX, int SB>
LuxStatus launch_gs(const QmmArgs& a, hipStream_t st) {
    switch (a.group_size) {
    case 32:
        // a wave's f32 scale rows at group size 32 (128 B each) do not fit in registers
        if constexpr (SB == DT_F32) return LuxStatus::NotSupported;
        else return launch<TX, SB, 32>(a, st);
    case 64: return launch<TX, SB, 64>(a, st);
    case 128: return launch<TX, SB, 128>(a, st);
    default: return LuxStatus::NotSupported;
    }
}

template <int TX>
LuxStatus launch_sb(const QmmArgs& a, hipStream_t st) {
    switch (a.sb_dtype) {
    case DT_F32: return launch_gs<TX, DT_F32>(a, st);
    case DT_F16: return launch_gs<TX, DT_F16>(a, st);
    default: return launch_gs<TX, DT_BF16>(a, st);
    }
}

}  // namespace dec

LuxStatus launch_qgemv_dec(const QmmArgs& a, hipStream_t st) {
    using namespace dec;
    if (a.M < 2 || a.M > kMaxM || a.bits != 4 || a.x_dtype == DT_F32) return LuxStatus::NotSupported;
    if (a.K % kKW != 0 || a.K / kKW > 8) return LuxStatus::NotSupported;
    // 32-bit buffer offsets
    if ((size_t)a.M * a.K * 2 >= (1ull << 31) || (size_t)a.N * a.K / 2 >= (1ull << 31)) return LuxStatus::NotSupported;
    return a.x_dtype == DT_F16 ? launch_sb<DT_F16>(a, st) : launch_sb<DT_BF16>(a, st);
}

}  // namespace lxq
