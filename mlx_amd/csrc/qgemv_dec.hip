// qgemv_dec.hip -- launcher of the MFMA decode kernel (qgemv_dec.h).
#include "qgemv_dec.h"

namespace lxq {
namespace dec {

// block shape: 16-row tiles per block, and codes of K per wave (kDecKW512:
// 512 where the wave count K/512 stays within 8 and the shape fits, else
// 1024).  Measured at c1 (K = 4096, N = 14336), M = 2 / 4 / 8: 2 tiles x
// 1024 codes 11.5-11.9 / 12.1-12.4 / 12.5 us; 2 x 512 12.0 / 12.5-12.8 /
// 13.2; 4 x 1024 14.9 / 15.3-15.4 / 15.6; 4 x 512 14.5 / 14.7 / 15.1.
constexpr int kDecTiles = 2;
constexpr bool kDecKW512 = false;

template <int TX, int SB, int GS, bool EPI, int TILES, int KW>
LuxStatus launch_e(const QmmArgs& a, hipStream_t st) {
    const size_t lds = dec_lds_bytes(a.M, a.K, TILES, KW);
    if (lds > 160 * 1024) return LuxStatus::NotSupported;
    auto kern = qgemv_dec_kernel<TX, SB, GS, EPI, TILES, KW>;
    // once per instantiation; a function-local static initializes exactly once
    // even when several threads make the first call together
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return LuxStatus::Internal;
    const int blocks = (a.N + 16 * TILES - 1) / (16 * TILES);
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * (a.K / KW)), lds, st, a.x, a.wq, a.scales, a.biases, a.y, a.M,
                       a.K, a.N, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

template <int TX, int SB, int GS, bool EPI>
LuxStatus launch_kw(const QmmArgs& a, hipStream_t st) {
    if constexpr (kDecKW512 && dec_ok<GS, SB, kDecTiles, 512>()) {
        if (a.K / 512 <= 8) return launch_e<TX, SB, GS, EPI, kDecTiles, 512>(a, st);
    }
    if constexpr (dec_ok<GS, SB, kDecTiles, 1024>()) return launch_e<TX, SB, GS, EPI, kDecTiles, 1024>(a, st);
    else return launch_e<TX, SB, GS, EPI, 2, 1024>(a, st);
}

template <int TX, int SB, int GS>
LuxStatus launch(const QmmArgs& a, hipStream_t st) {
    return a.has_epilogue() ? launch_kw<TX, SB, GS, true>(a, st) : launch_kw<TX, SB, GS, false>(a, st);
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
    if (a.K % 1024 != 0 || a.K / 1024 > 8) return LuxStatus::NotSupported;
    // 32-bit buffer offsets
    if ((size_t)a.M * a.K * 2 >= (1ull << 31) || (size_t)a.N * a.K / 2 >= (1ull << 31)) return LuxStatus::NotSupported;
    return a.x_dtype == DT_F16 ? launch_sb<DT_F16>(a, st) : launch_sb<DT_BF16>(a, st);
}

}  // namespace lxq
