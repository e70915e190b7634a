// bwd_d192.hip — the fp16/bf16 backward kernels of width 192 (head dims 168..192 in steps of 8, the columns
// past the head dim zero): dQ kernel BwdQCfg<192, 32, 4, 1> and dK/dV kernel BwdKVCfg<192, 4, 1>, both
// one wave per SIMD and without a head-dim split (each wave holds its 192-wide accumulators).
#include "bwd_kernel.hpp"

namespace fa {

int launch_bwd_d192(const FableBwdParams& p, int dtype, hipStream_t st) {
  using CQ = BwdQCfg<192, 32, 4, 1>;
  using CKV = BwdKVCfg<192, 4, 1>;
  if (dtype == FA_F16) return launch_bwd<_Float16, CQ, CKV>(p, st);
  return launch_bwd<__bf16, CQ, CKV>(p, st);
}

}  // namespace fa
