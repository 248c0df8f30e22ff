// qgemv_q4.hip -- launcher of the 4x4x4-MFMA decode GEMV (qgemv_q4.h).
#include "qgemv_q4.h"

namespace lxq {
namespace q4 {

template <int TX, int SB, int XS, int RG, int KW, int CH = 1>
LuxStatus launch_q(const QmmArgs& a, hipStream_t st) {
    switch (mx_sb_loads(4 * RG, a.K / a.group_size, SB, KW)) {
    case 1: return launch_k<TX, SB, XS, RG, 1, KW, CH>(a, st);
    case 2: return launch_k<TX, SB, XS, RG, 2, KW, CH>(a, st);
    default: return launch_k<TX, SB, XS, RG, 4, KW, CH>(a, st);
    }
}

// waves per block: K / 512; 16-row blocks at 16 waves (4 waves per SIMD,
// 128 VGPRs), else 28 rows where that balances the grid better (mx_rows).
// 8192 < K <= 16384 with one set of x rows (M <= 4): two chunks per lane on
// 12, 14 or 16 waves (the fewest that reach K; lanes past K idle) and
// 16-row blocks.  Against the K-split whole-line kernel that took these
// shapes (same box, 4-bit g64 f16, µs): K = 14336, N = 4096, M = 2 / 3 / 4:
// 11.93 / 16.10 / 16.16 -> 9.90 / 10.51 / 11.23; N = 8192 22.05 / 30.65 /
// 30.76 -> 18.66 / 19.86 / 21.45; K = 12288, N = 4096 11.36 / 15.54 / 15.59
// -> 8.54 / 9.18 / 9.65; K = 16384, N = 8192 23.68 / 32.31 / 32.45 ->
// 21.55 / 22.85 / 24.82.  K short of the waves' reach (another box): K =
// 11008, N = 4096 11.23 / 15.55 / 15.58 -> 8.56 / 8.98 / 9.54; N = 5120
// 19.86 / 28.54 / 28.57 -> 14.39 / 15.38 / 16.57; K = 9216, N = 4096 10.97
// / 15.19 / 15.25 -> 8.22 / 8.68 / 9.07; K = 13824, N = 5120 20.51 / 29.08
// / 29.13 -> 17.91 / 19.30 / 20.64.  Two sets (M = 5 .. 8) hold twice the
// x and spill at these wave counts (31-37 µs against 25.4 for the mid-M
// kernel that keeps them).
template <int TX, int SB, int XS>
LuxStatus launch_w(const QmmArgs& a, hipStream_t st) {
    const bool r28 = gemv::mx_rows(a.N) == 28;
    switch (a.K) {
    case 2048: return r28 ? launch_q<TX, SB, XS, 7, 4>(a, st) : launch_q<TX, SB, XS, 4, 4>(a, st);
    case 4096: return r28 ? launch_q<TX, SB, XS, 7, 8>(a, st) : launch_q<TX, SB, XS, 4, 8>(a, st);
    case 8192: return launch_q<TX, SB, XS, 4, 16>(a, st);
    default: break;
    }
    if constexpr (XS == 1) {
        // any other K up to 16384 (K % 32 = 0): the next of these, lanes
        // past K idle (they add nothing)
        if (a.K % 32 == 0 && a.K > 8192 && a.K <= 16384) {
            if (a.K <= 12288) return launch_q<TX, SB, 1, 4, 12, 2>(a, st);
            if (a.K <= 14336) return launch_q<TX, SB, 1, 4, 14, 2>(a, st);
            return launch_q<TX, SB, 1, 4, 16, 2>(a, st);
        }
    }
    return LuxStatus::NotSupported;
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
    // one chunk per lane up to K = 8192; two for the long K at M <= 4
    const bool one = a.K == 2048 || a.K == 4096 || a.K == 8192;
    const bool two = a.M <= 4 && a.K % 32 == 0 && a.K > 8192 && a.K <= 16384;
    if (!one && !two) return LuxStatus::NotSupported;
    if (a.group_size != 32 && a.group_size != 64 && a.group_size != 128) return LuxStatus::NotSupported;
    // offsets within the 32-bit buffer ranges
    if ((size_t)a.N * a.K / 2 >= (1ull << 31)) return LuxStatus::NotSupported;
    return a.x_dtype == DT_F16 ? launch_sb<DT_F16>(a, st) : launch_sb<DT_BF16>(a, st);
}

}  // namespace lxq
