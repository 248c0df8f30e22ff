// qgemv_b5.hip -- 5-bit instantiations of the GEMV kernels.
#include "qgemv_impl.h"
#include "qgemv_line.h"
#include "qgemv_mx.h"

namespace lxq {
namespace gemv {
template LuxStatus launch_b<5>(const QmmArgs&, hipStream_t);
template LuxStatus launch_mx_b<5>(const QmmArgs&, hipStream_t);
}  // namespace gemv
}  // namespace lxq
