// bwd_d224.hip — the fp16/bf16 backward kernels for head dims 200..224 (in steps of 8, the
// columns past the head dim zero): dQ kernel BwdQCfg<224, 32, 4, 1> of width 224; dK/dV in the
// 256-wide kernel BwdKVCfg<256, 4, 1, 2>, which splits the head dim in two passes of 128 columns
// (1.14x the work of width 224): a 224-wide dK/dV kernel without a head-dim split holds 224
// accumulator and 112 operand registers per lane, 134 more than one wave per SIMD has, and 7
// columns of 32 split only into 7 passes of S and dP.
#include "bwd_kernel.hpp"

namespace fa {

int launch_bwd_d224(const FableBwdParams& p, int dtype, hipStream_t st) {
  using CQ = BwdQCfg<224, 32, 4, 1>;
  using CKV = BwdKVCfg<256, 4, 1, 2>;
  if (dtype == FA_F16) return launch_bwd<_Float16, CQ, CKV>(p, st);
  return launch_bwd<__bf16, CQ, CKV>(p, st);
}

}  // namespace fa
