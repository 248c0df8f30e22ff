// explicit instantiation: register-W large GEMM, f16 activations, group size 128
#include "qgemm_rw.h"
namespace lxq {
namespace rw {
template LuxStatus launch_tg<DT_F16, 128>(const QmmArgs&, hipStream_t);
}  // namespace rw
}  // namespace lxq
