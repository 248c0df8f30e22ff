// qgemv_dec.hip -- launcher of the MFMA decode kernel (qgemv_dec.h).
#include "qgemv_dec.h"

namespace lxq {
namespace dec {

// Block shape: 1024 codes of K per wave; 2 16-row tiles per block (their
// MFMAs share each x operand), or 1 where 2-tile blocks would leave CUs
// without a block and every 1-tile block is resident at once.  Measured
// (graph replays, us), M = 2 / 4 / 8:
//   K = 4096, N = 14336: 2 tiles 11.5 / 12.3 / 13.0, 1 tile 11.7 / 13.0 / 15.5;
//     2 x 512 codes 12.0 / 12.5-12.8 / 13.2; 4 tiles 14.9 / 15.3 / 15.6
//   K = 4096, N = 4096 (128 2-tile blocks): 2 tiles 7.4 / 7.8 / 8.0, 1 tile 5.9 / 6.2 / 6.4
//   K = 8192, N = 8192, M = 4 / 8: 2 tiles 16.3 / 16.9, 1 tile 14.8 / 19.0
//     (at M = 8 one 1-tile block fills a CU's LDS: the 512 blocks run in two rounds)
// x staging: shared by the block's waves (one barrier) up to K = 4096, per
// wave above (no barrier).  Measured, per wave against shared: K = 8192,
// M = 8, N = 8192 14.9 us against 17.0, N = 28672 47.2 against 54.5;
// K = 6144, N = 8192, M = 4 / 8 11.5-11.8 / 12.0 against 12.2-12.5 / 13.2;
// at K = 4096 per wave costs 0-5 % (c1 M = 4 12.3-12.6 against 12.0-12.6;
// N = 4096, M = 4 6.18 against 5.9).
constexpr int kDecSharedXMaxK = 4096;
constexpr int kCUs = 256;           // gfx950 (MI355X)
// 1-tile blocks with 512 codes per wave (K <= 4096), against 1024: K = 4096,
// N = 4096, M = 4 / 8 5.84 / 6.12 us against 6.13 / 6.41; N = 6144, M = 4
// 7.50 against 7.83; K = 2048, N = 8192, M = 8 5.64 against 7.12
constexpr bool kDec1KW512 = true;
constexpr int kWavesPerCU1 = 20;    // 1-tile kernel: <= 96 VGPRs, 5 waves per SIMD

template <int TX, int SB, int GS, bool EPI, int TILES, int KW = 1024>
LuxStatus launch_e(const QmmArgs& a, hipStream_t st) {
    const size_t lds = dec_lds_bytes(a.M, a.K, TILES, KW);
    if (lds > 160 * 1024) return LuxStatus::NotSupported;
    if (planned(a, "qgemv_dec_kernel")) return LuxStatus::Ok;
    auto kern = qgemv_dec_kernel<TX, SB, GS, EPI, TILES, KW>;
    // once per instantiation; a function-local static initializes exactly once
    // even when several threads make the first call together
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return LuxStatus::Internal;
    const int blocks = (a.N + 16 * TILES - 1) / (16 * TILES);
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * (a.K / KW)), lds, st, a.x, a.wq, a.scales, a.biases, a.y, a.M,
                       a.K, a.N, a.K > kDecSharedXMaxK ? 1 : 0, a.epi());
    return hipGetLastError() == hipSuccess ? LuxStatus::Ok : LuxStatus::Internal;
}

template <int TX, int SB, int GS, bool EPI>
LuxStatus launch_kw(const QmmArgs& a, hipStream_t st) {
    static_assert(dec_ok<GS, SB, 1, 1024>() && dec_ok<GS, SB, 2, 1024>(), "block shapes");
    // 1-tile blocks: 512 codes per wave where that keeps a block within 8 waves
    constexpr bool kw512_ok = kDec1KW512 && dec_ok<GS, SB, 1, 512>();
    const bool kw512 = kw512_ok && a.K / 512 <= 8;
    const int kw1 = kw512 ? 512 : 1024;
    const long b2 = (a.N + 31) / 32, b1 = (a.N + 15) / 16;
    const size_t lds1 = dec_lds_bytes(a.M, a.K, 1, kw1);
    const long lds_fit = lds1 <= 160 * 1024 ? (long)(160 * 1024 / lds1) : 0;
    const long wave_fit = kWavesPerCU1 / (a.K / kw1);
    const long per_cu = lds_fit < wave_fit ? lds_fit : wave_fit;
    if (b2 <= kCUs && b1 <= per_cu * kCUs) {
        if constexpr (kw512_ok) {
            if (kw512) return launch_e<TX, SB, GS, EPI, 1, 512>(a, st);
        }
        return launch_e<TX, SB, GS, EPI, 1>(a, st);
    }
    return launch_e<TX, SB, GS, EPI, 2>(a, st);
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
