// fwd_d128.hip — the fp16/bf16 forward kernels for head_dim 128 (workgroup shapes C, CF, CN of
// launch_fwd in fwd_kernel.hpp).
#include "fwd_kernel.hpp"

namespace fa {

int launch_fwd_d128(const FwdParams& p, int dtype, hipStream_t st) {
  if (dtype == FA_F16) return launch_fwd<_Float16, FwdCfg<128, 64, 8, 2>, FwdCfg<128, 32, 4, 2>, FwdCfg<128, 32, 2, 2>>(p, st);
  return launch_fwd<__bf16, FwdCfg<128, 64, 8, 2>, FwdCfg<128, 32, 4, 2>, FwdCfg<128, 32, 2, 2>>(p, st);
}

}  // namespace fa
