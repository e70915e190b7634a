// bwd_d160.hip — the fp16/bf16 backward kernels of width 160 (head dims 136..160 in steps of 8, the columns
// past the head dim zero): dQ kernel BwdQCfg<160, 32, 4, 1>, dK/dV kernel with one wave per SIMD BwdKVCfg<160, 2, 1>.
#include "bwd_kernel.hpp"

namespace fa {

int launch_bwd_d160(const FableBwdParams& p, int dtype, hipStream_t st) {
  using CQ = BwdQCfg<160, 32, 4, 1>;
  using CKV = BwdKVCfg<160, 2, 1>;
  if (dtype == FA_F16) return launch_bwd<_Float16, CQ, CKV>(p, st);
  return launch_bwd<__bf16, CQ, CKV>(p, st);
}

}  // namespace fa
