// bwd_d32.hip — the fp16/bf16 backward kernels of width 32 (head dims 8..32 in steps of 8, the columns
// past the head dim zero): dQ kernel BwdQCfg<32, 64, 4, 2>, wave-pair dK/dV kernel (with the dS-workspace path) BwdKVPCfg<32, 2, 3, 3>
// at three waves per SIMD (129-137 registers; 1.14-1.16x over two).
#include "bwd_kernel.hpp"

namespace fa {

int launch_bwd_d32(const FableBwdParams& p, int dtype, hipStream_t st) {
  using CQ = BwdQCfg<32, 64, 4, 2>;
  using CKV = BwdKVPCfg<32, 2, 3, 3>;
  if (dtype == FA_F16) return launch_bwd<_Float16, CQ, CKV>(p, st);
  return launch_bwd<__bf16, CQ, CKV>(p, st);
}

}  // namespace fa
