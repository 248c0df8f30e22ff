// explicit instantiation: MFMA dequant GEMM, group size 32
#include "qgemm_impl.h"
namespace lxq {
namespace gemm {
template LuxStatus launch_g<32>(const QmmArgs&, hipStream_t);
}  // namespace gemm
}  // namespace lxq
