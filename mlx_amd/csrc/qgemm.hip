// qgemm.hip -- MFMA GEMM for large M (gfx950).  Placeholder until the tiled
// kernel lands: reports NotSupported so the dispatcher uses the GEMV.
#include "kernels.h"

namespace lxq {

LuxStatus launch_qgemm(const QmmArgs&, hipStream_t) { return LuxStatus::NotSupported; }

}  // namespace lxq
