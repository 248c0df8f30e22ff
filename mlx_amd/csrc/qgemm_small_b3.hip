// qgemm_small_b3.hip -- 3-bit instantiations of the small-M MFMA GEMM.
#include "qgemm_small.h"

namespace lxq {
namespace small {
template LuxStatus launch_tx<3>(const QmmArgs&, hipStream_t);
}  // namespace small
}  // namespace lxq
