// qgemm_sk_b8.hip -- 8-bit instantiations of the split-K small-M GEMM.
#include "qgemm_sk.h"

namespace lxq {
namespace sk {
template LuxStatus launch_bits<8>(const QmmArgs&, int, hipStream_t);
}  // namespace sk
}  // namespace lxq
