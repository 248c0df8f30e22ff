// qgemm_sk_b2.hip -- 2-bit instantiations of the split-K small-M GEMM.
#include "qgemm_sk.h"

namespace lxq {
namespace sk {
template LuxStatus launch_bits<2>(const QmmArgs&, int, hipStream_t);
}  // namespace sk
}  // namespace lxq
