// qgemv_q4.hip -- launcher of the 4x4x4-MFMA decode GEMV (qgemv_q4.h).
#include "qgemv_q4.h"

namespace lxq {
namespace q4 {

template <int TX, int SB, int XS, int RG, int KW>
LuxStatus launch_q(const QmmArgs& a, hipStream_t st) {
    switch (mx_sb_loads(4 * RG, a.K / a.group_size, SB, KW)) {
    case 1: return launch_k<TX, SB, XS, RG, 1, KW>(a, st);
    case 2: return launch_k<TX, SB, XS, RG, 2, KW>(a, st);
    default: return launch_k<TX, SB, XS, RG, 4, KW>(a, st);
    }
}

// waves per block: K / 512; 16-row blocks at 16 waves (4 waves per SIMD,
// 128 VGPRs), else 28 rows where that balances the grid better (mx_rows)
template <int TX, int SB, int XS>
LuxStatus launch_w(const QmmArgs& a, hipStream_t st) {
    const bool r28 = gemv::mx_rows(a.N) == 28;
    switch (a.K) {
    case 2048: return r28 ? launch_q<TX, SB, XS, 7, 4>(a, st) : launch_q<TX, SB, XS, 4, 4>(a, st);
    case 4096: return r28 ? launch_q<TX, SB, XS, 7, 8>(a, st) : launch_q<TX, SB, XS, 4, 8>(a, st);
    default: return launch_q<TX, SB, XS, 4, 16>(a, st);
    }
}

template <int TX, int SB>
LuxStatus launch_x(const QmmArgs& a, hipStream_t st) {
    return a.M <= 4 ? launch_w<TX, SB, 1>(a, st) : launch_w<TX, SB, 2>(a, st);
}

template <int TX>
LuxStatus launch_sb(const QmmArgs& a, hipStream_t st) {
    switch (a.sb_dtype) {
    case DT_F32: return launch_x<TX, DT_F32>(a, st);
    case DT_F16: return launch_x<TX, DT_F16>(a, st);
    default: return launch_x<TX, DT_BF16>(a, st);
    }
}

}  // namespace q4

LuxStatus launch_qgemv_q4(const QmmArgs& a, hipStream_t st) {
    using namespace q4;
    if (a.M < 2 || a.M > 8 || a.bits != 4 || a.x_dtype == DT_F32) return LuxStatus::NotSupported;
    if (a.K != 2048 && a.K != 4096 && a.K != 8192) return LuxStatus::NotSupported;
    if (a.group_size != 32 && a.group_size != 64 && a.group_size != 128) return LuxStatus::NotSupported;
    // offsets within the 32-bit buffer ranges
    if ((size_t)a.N * a.K / 2 >= (1ull << 31)) return LuxStatus::NotSupported;
    return a.x_dtype == DT_F16 ? launch_sb<DT_F16>(a, st) : launch_sb<DT_BF16>(a, st);
}

}  // namespace lxq
