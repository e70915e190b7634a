// fwd_d64.hip — the fp16/bf16 forward kernels of width 64 (head dims 40..64 in steps of 8, the
// columns past the head dim zero; workgroup shapes C, CF, CN, CS, CL, CR of launch_fwd in fwd_kernel.hpp).
#include "fwd_kernel.hpp"

namespace fa {

int launch_fwd_d64(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws) {
  if (dtype == FA_F16) return launch_fwd<_Float16, FwdCfg<64, 64, 8, 2>, FwdCfg<64, 64, 8, 2>, FwdCfg<64, 64, 4, 2>, FwdCfg<64, 64, 4, 2>,
                                          FwdCfg<64, 64, 4, 3>, FwdCfg<64, 64, 2, 2>>(p, st, ws);
  return launch_fwd<__bf16, FwdCfg<64, 64, 8, 2>, FwdCfg<64, 64, 8, 2>, FwdCfg<64, 64, 4, 2>, FwdCfg<64, 64, 4, 2>,
                                          FwdCfg<64, 64, 4, 3>, FwdCfg<64, 64, 2, 2>>(p, st, ws);
}

}  // namespace fa
