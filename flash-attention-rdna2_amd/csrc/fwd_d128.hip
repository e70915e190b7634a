// fwd_d128.hip — the fp16/bf16 forward kernels of width 128 (head dims 104..128 in steps of 8, the
// columns past the head dim zero; workgroup shapes C, CF, CN, CR of launch_fwd in fwd_kernel.hpp).
#include "fwd_kernel.hpp"

namespace fa {

int launch_fwd_d128(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws) {
  // no separate small-grid shape: with the heaviest-first work order the 8-wave shape is as
  // fast on short grids (causal S=4096 H=32: 1.00-1.03x the 4-wave one, which spilled 24 bytes)
  using C = FwdCfg<128, 64, 8, 2>;
  using CF = FwdCfg<128, 32, 4, 2>;
  using CN = FwdCfg<128, 32, 2, 2>;
  // short causal rows: the narrow-mask shape (64 rows per workgroup)
  if (dtype == FA_F16) return launch_fwd<_Float16, C, CF, CN, C, C, CN>(p, st, ws);
  return launch_fwd<__bf16, C, CF, CN, C, C, CN>(p, st, ws);
}

}  // namespace fa
