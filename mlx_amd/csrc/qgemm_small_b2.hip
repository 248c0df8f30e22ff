// qgemm_small_b2.hip -- 2-bit instantiations of the small-M MFMA GEMM.
#include "qgemm_small.h"

namespace lxq {
namespace small {
template LuxStatus launch_tx<2>(const QmmArgs&, hipStream_t);
}  // namespace small
}  // namespace lxq
