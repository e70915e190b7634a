// fwd_d96.hip — the fp16/bf16 forward kernels of width 96 (head dims 72..96 in steps of 8, the
// columns past the head dim zero; workgroup shapes C, CF, CN, CS, CL, CR of launch_fwd in fwd_kernel.hpp).
#include "fwd_kernel.hpp"

namespace fa {

int launch_fwd_d96(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws) {
  if (dtype == FA_F16) return launch_fwd<_Float16, FwdCfg<96, 64, 8, 2>, FwdCfg<96, 32, 4, 2>, FwdCfg<96, 32, 2, 2>, FwdCfg<96, 64, 4, 2>, FwdCfg<96, 64, 8, 2>, FwdCfg<96, 32, 2, 2>>(p, st, ws);
  return launch_fwd<__bf16, FwdCfg<96, 64, 8, 2>, FwdCfg<96, 32, 4, 2>, FwdCfg<96, 32, 2, 2>, FwdCfg<96, 64, 4, 2>, FwdCfg<96, 64, 8, 2>, FwdCfg<96, 32, 2, 2>>(p, st, ws);
}

}  // namespace fa
