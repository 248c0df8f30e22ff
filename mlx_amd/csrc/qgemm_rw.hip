// qgemm_rw.hip -- dispatch of the register-W large GEMM (kernels in
// qgemm_rw.h, one translation unit per activation type and group size:
// qgemm_rw_{bf16,f16}_g{32,64,128}.hip).
#include "qgemm_rw.h"

namespace lxq {

LuxStatus launch_qgemm_rw(const QmmArgs& a, hipStream_t st) {
    if (!rw::applies(a.M, a.K, a.N, a.bits, a.x_dtype)) return LuxStatus::NotSupported;
    const bool bf = a.x_dtype == DT_BF16;
    switch (a.group_size) {
    case 32: return bf ? rw::launch_tg<DT_BF16, 32>(a, st) : rw::launch_tg<DT_F16, 32>(a, st);
    case 64: return bf ? rw::launch_tg<DT_BF16, 64>(a, st) : rw::launch_tg<DT_F16, 64>(a, st);
    case 128: return bf ? rw::launch_tg<DT_BF16, 128>(a, st) : rw::launch_tg<DT_F16, 128>(a, st);
    default: return LuxStatus::NotSupported;
    }
}

}  // namespace lxq
