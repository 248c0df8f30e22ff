// qgemm_sk_b6.hip -- 6-bit instantiations of the split-K small-M GEMM.
#include "qgemm_sk.h"

namespace lxq {
namespace sk {
template LuxStatus launch_bits<6>(const QmmArgs&, int, hipStream_t);
}  // namespace sk
}  // namespace lxq
