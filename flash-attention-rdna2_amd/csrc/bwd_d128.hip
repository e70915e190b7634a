// bwd_d128.hip — the fp16/bf16 backward kernels of width 128 (head dims 104..128 in steps of 8, the columns
// past the head dim zero): dQ kernel BwdQCfg<128, 32, 4, 2>, wave-pair dK/dV kernel (with the dS-workspace path) BwdKVPCfg<128, 4, 2>.
#include "bwd_kernel.hpp"

namespace fa {

int launch_bwd_d128(const FableBwdParams& p, int dtype, hipStream_t st) {
  using CQ = BwdQCfg<128, 32, 4, 2>;
  using CKV = BwdKVPCfg<128, 4, 2>;
  if (dtype == FA_F16) return launch_bwd<_Float16, CQ, CKV>(p, st);
  return launch_bwd<__bf16, CQ, CKV>(p, st);
}

}  // namespace fa
