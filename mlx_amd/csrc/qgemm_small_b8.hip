// qgemm_small_b8.hip -- 8-bit instantiations of the small-M MFMA GEMM.
#include "qgemm_small.h"

namespace lxq {
namespace small {
template LuxStatus launch_tx<8>(const QmmArgs&, hipStream_t);
}  // namespace small
}  // namespace lxq
