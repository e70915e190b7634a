// fwd_d256.hip — the fp16/bf16 forward kernels of width 256 (head dims 232..256 in steps of 8, the
// columns past the head dim zero; workgroup shapes C, CF, CN of launch_fwd in fwd_kernel.hpp).
#include "fwd_kernel.hpp"

namespace fa {

int launch_fwd_d256(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws) {
  // 64-key tiles for the softcap / dropout kernels (dense causal softcap +4%, packed causal
  // softcap +3.5%); the plain kernels are 20% slower with them, and the narrow-window ones 8%
  using C = FwdCfg<256, 32, 4, 1>;
  using CF = FwdCfg<256, 64, 4, 1>;
  using CN = FwdCfg<256, 32, 2, 1>;
  if (dtype == FA_F16) return launch_fwd<_Float16, C, CF, CN>(p, st, ws);
  return launch_fwd<__bf16, C, CF, CN>(p, st, ws);
}

}  // namespace fa
