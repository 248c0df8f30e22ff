// qgemm_small_b4.hip -- 4-bit instantiations of the small-M MFMA GEMM.
#include "qgemm_small.h"

namespace lxq {
namespace small {
template LuxStatus launch_tx<4>(const QmmArgs&, hipStream_t);
}  // namespace small
}  // namespace lxq
