// bwd_d64.hip — the fp16/bf16 backward kernels of width 64 (head dims 40..64 in steps of 8, the columns
// past the head dim zero): dQ kernel BwdQCfg<64, 64, 4, 2>, wave-pair dK/dV kernel (with the dS-workspace path) BwdKVPCfg<64, 2, 3, 3>
// at three waves per SIMD (168 registers; at two, 170 and one workgroup fewer per CU: 1.06-1.13x).
#include "bwd_kernel.hpp"

namespace fa {

int launch_bwd_d64(const FableBwdParams& p, int dtype, hipStream_t st) {
  using CQ = BwdQCfg<64, 64, 4, 2>;
  using CKV = BwdKVPCfg<64, 2, 3, 3>;
  if (dtype == FA_F16) return launch_bwd<_Float16, CQ, CKV>(p, st);
  return launch_bwd<__bf16, CQ, CKV>(p, st);
}

}  // namespace fa
