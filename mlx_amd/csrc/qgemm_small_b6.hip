// qgemm_small_b6.hip -- 6-bit instantiations of the small-M MFMA GEMM.
#include "qgemm_small.h"

namespace lxq {
namespace small {
template LuxStatus launch_tx<6>(const QmmArgs&, hipStream_t);
}  // namespace small
}  // namespace lxq
