// qgemm_small.hip -- dispatch of the small-M MFMA GEMM (kernel in qgemm_small.h,
// one translation unit per code width: qgemm_small_b{2,3,4,5,6,8}.hip).
#include "qgemm_small.h"

namespace lxq {
namespace small {
extern template LuxStatus launch_tx<2>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_tx<3>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_tx<4>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_tx<5>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_tx<6>(const QmmArgs&, hipStream_t);
extern template LuxStatus launch_tx<8>(const QmmArgs&, hipStream_t);
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
