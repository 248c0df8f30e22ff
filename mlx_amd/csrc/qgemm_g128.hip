// explicit instantiation: MFMA dequant GEMM, group size 128
#include "qgemm_impl.h"
namespace lxq {
namespace gemm {
template LuxStatus launch_g<128>(const QmmArgs&, hipStream_t);
}  // namespace gemm
}  // namespace lxq
