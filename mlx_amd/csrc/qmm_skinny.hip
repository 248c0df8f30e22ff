// qmm_skinny.hip -- launcher of the small-M MFMA kernel.
#include "qmm_skinny.h"

namespace lxq {
namespace skinny {

template <int BITS, int TX, int SB, int GS, int GW, bool EPI>
LuxStatus launch_e(const QmmArgs& a, int KS, hipStream_t st) {
    constexpr int kSb = SB == DT_F32 ? 4 : 2;
    const int tiles = kWaves / KS;
    const size_t lds = skinny_lds_bytes(a.M, a.K, a.K / GS, kSb, tiles);
    if (lds > 160 * 1024) return LuxStatus::NotSupported;
    if (planned(a, "qmm_skinny_kernel")) return LuxStatus::Ok;
    auto kern = qmm_skinny_kernel<BITS, TX, SB, GS, GW, EPI>;
    // once per instantiation; a function-local static initializes exactly once
    // even when several threads make the first call together
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return LuxStatus::Internal;
    const int rows = 16 * tiles;
    const int blocks = (a.N + rows - 1) / rows;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * kWaves), lds, st, a.x, a.wq, a.scales, a.biases, a.y, a.M,
                       a.K, a.N, KS, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

template <int BITS, int TX, int SB, int GS, int GW>
LuxStatus launch(const QmmArgs& a, int KS, hipStream_t st) {
    return a.has_epilogue() ? launch_e<BITS, TX, SB, GS, GW, true>(a, KS, st)
                            : launch_e<BITS, TX, SB, GS, GW, false>(a, KS, st);
}

// groups per wave GW in {8, 16, 32}; the 8-bit, group-128 slice of 8 words
// allows at most 16 groups in flight (vmcnt)
template <int BITS, int TX, int SB, int GS>
LuxStatus launch_gw(const QmmArgs& a, hipStream_t st) {
    const int G = a.K / GS;
    for (int KS : {4, 2, 1}) {
        if (G % KS) continue;
        const int gw = G / KS;
        if (gw == 8) return launch<BITS, TX, SB, GS, 8>(a, KS, st);
        if (gw == 16) return launch<BITS, TX, SB, GS, 16>(a, KS, st);
        if constexpr (!(BITS == 8 && GS == 128))
            if (gw == 32) return launch<BITS, TX, SB, GS, 32>(a, KS, st);
    }
    return LuxStatus::NotSupported;
}

template <int BITS, int TX, int SB>
LuxStatus launch_gs(const QmmArgs& a, hipStream_t st) {
    switch (a.group_size) {
    case 32: return launch_gw<BITS, TX, SB, 32>(a, st);
    case 64: return launch_gw<BITS, TX, SB, 64>(a, st);
    case 128: return launch_gw<BITS, TX, SB, 128>(a, st);
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

}  // namespace skinny

LuxStatus launch_qmm_skinny(const QmmArgs& a, hipStream_t st) {
    using namespace skinny;
    if (a.M < 2 || a.M > 16 || (a.bits != 4 && a.bits != 8) || a.x_dtype == DT_F32) return LuxStatus::NotSupported;
    // 32-bit buffer offsets (the scale arrays are smaller than the codes)
    if ((size_t)a.M * a.K * 2 >= (1ull << 31) || (size_t)a.N * a.K * a.bits / 8 >= (1ull << 31))
        return LuxStatus::NotSupported;
    if (a.bits == 4) return a.x_dtype == DT_F16 ? launch_sb<4, DT_F16>(a, st) : launch_sb<4, DT_BF16>(a, st);
    return a.x_dtype == DT_F16 ? launch_sb<8, DT_F16>(a, st) : launch_sb<8, DT_BF16>(a, st);
}

}  // namespace lxq
