// bwd_d256.hip — the fp16/bf16 backward kernels of width 256 (head dims 232..256 in steps of 8, the columns
// past the head dim zero): dQ kernel BwdQCfg<256, 32, 4, 1> (no head-dim split) and dK/dV kernel
// BwdKVCfg<256, 4, 1, 2> (the head dim in two passes of 128 columns), both one wave per SIMD.
#include "bwd_kernel.hpp"

namespace fa {

int launch_bwd_d256(const FableBwdParams& p, int dtype, hipStream_t st) {
  using CQ = BwdQCfg<256, 32, 4, 1>;
  using CKV = BwdKVCfg<256, 4, 1, 2>;
  if (dtype == FA_F16) return launch_bwd<_Float16, CQ, CKV>(p, st);
  return launch_bwd<__bf16, CQ, CKV>(p, st);
}

}  // namespace fa
