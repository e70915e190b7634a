// fwd_d224.hip — the fp16/bf16 forward kernels of width 224 (head dims 200..224 in steps of 8, the
// columns past the head dim zero; workgroup shapes C, CF, CN of launch_fwd in fwd_kernel.hpp).
#include "fwd_kernel.hpp"

namespace fa {

int launch_fwd_d224(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws) {
  if (dtype == FA_F16) return launch_fwd<_Float16, FwdCfg<224, 32, 4, 1>, FwdCfg<224, 32, 4, 1>, FwdCfg<224, 32, 2, 1>>(p, st, ws);
  return launch_fwd<__bf16, FwdCfg<224, 32, 4, 1>, FwdCfg<224, 32, 4, 1>, FwdCfg<224, 32, 2, 1>>(p, st, ws);
}

}  // namespace fa
