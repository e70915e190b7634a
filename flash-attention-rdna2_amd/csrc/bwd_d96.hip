// bwd_d96.hip — the fp16/bf16 backward kernels of width 96 (head dims 72..96 in steps of 8, the columns
// past the head dim zero): dQ kernel BwdQCfg<96, 32, 4, 2>, wave-pair dK/dV kernel (with the dS-workspace path) BwdKVPCfg<96, 2, 2>.
#include "bwd_kernel.hpp"

namespace fa {

int launch_bwd_d96(const FableBwdParams& p, int dtype, hipStream_t st) {
  using CQ = BwdQCfg<96, 32, 4, 2>;
  using CKV = BwdKVPCfg<96, 2, 2>;
  if (dtype == FA_F16) return launch_bwd<_Float16, CQ, CKV>(p, st);
  return launch_bwd<__bf16, CQ, CKV>(p, st);
}

}  // namespace fa
