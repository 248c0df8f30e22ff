// qgemm_small_b5.hip -- 5-bit instantiations of the small-M MFMA GEMM.
#include "qgemm_small.h"

namespace lxq {
namespace small {
template LuxStatus launch_tx<5>(const QmmArgs&, hipStream_t);
}  // namespace small
}  // namespace lxq
