// qgemm.hip -- dispatch of the MFMA dequant GEMM (kernels in qgemm_impl.h,
// one translation unit per group size: qgemm_g{32,64,128}.hip).
#include <cstdlib>

#include "qgemm_impl.h"

namespace lxq {

LuxStatus launch_qgemm(const QmmArgs& a, hipStream_t st) {
    // M > 64 with 4/8-bit codes and K % 1024 == 0: the register-W kernel
    // (unless LUX_HIP_GEMM_RW=0 asks for the kernels below)
    static const bool rw_on = [] {
        const char* e = std::getenv("LUX_HIP_GEMM_RW");
        return !(e && e[0] == '0');
    }();
    if (rw_on) {
        const LuxStatus s = launch_qgemm_rw(a, st);
        if (s != LuxStatus::NotSupported) return s;
    }
    // 8 < M <= 64: the split-K small-M kernel, else the W-streaming one
    if (a.M <= 64) {
        LuxStatus s = launch_qgemm_sk(a, st);
        if (s != LuxStatus::NotSupported) return s;
        s = launch_qgemm_small(a, st);
        if (s != LuxStatus::NotSupported) return s;
    }
    // the scale windows cover 4 K steps of 64 codes
    if (a.K % 256 != 0) return LuxStatus::NotSupported;
    // x and W offsets are 32-bit: each must stay below 4 GiB
    if ((size_t)a.M * a.K * 2 >= (1ull << 32) || (size_t)a.N * a.K * a.bits / 8 >= (1ull << 32))
        return LuxStatus::NotSupported;
    switch (a.group_size) {
    case 32: return gemm::launch_g<32>(a, st);
    case 64: return gemm::launch_g<64>(a, st);
    case 128: return gemm::launch_g<128>(a, st);
    default: return LuxStatus::NotSupported;
    }
}

}  // namespace lxq
