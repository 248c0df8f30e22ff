// explicit instantiation: MFMA dequant GEMM, group size 64
#include "qgemm_impl.h"
namespace lxq {
namespace gemm {
template LuxStatus launch_g<64>(const QmmArgs&, hipStream_t);
}  // namespace gemm
}  // namespace lxq
