// explicit instantiation: register-W large GEMM, bf16 activations, group size 64
#include "qgemm_rw.h"
namespace lxq {
namespace rw {
template LuxStatus launch_tg<DT_BF16, 64>(const QmmArgs&, hipStream_t);
}  // namespace rw
}  // namespace lxq
