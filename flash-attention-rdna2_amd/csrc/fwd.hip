// fwd.hip — fa_forward_launch, the forward's C-ABI entry point: argument checks and dispatch to
// the per-head-dim fp16/bf16 kernels (fwd_d64/128/256.hip, kernel in fwd_kernel.hpp) and the
// fp32 kernels (fwd_f32.hip). Reference launcher: kernels/fa_forward.hip:424-451.
#include "attn_device.hpp"
#include "fwd_common.hpp"
#include "status.hpp"

namespace fa {

static int dispatch_hd(const FwdParams& p, int dtype, hipStream_t st) {
  switch (p.HD) {
    case 64: return launch_fwd_d64(p, dtype, st);
    case 128: return launch_fwd_d128(p, dtype, st);
    case 256: return launch_fwd_d256(p, dtype, st);
    default: return fail(FA_ERR_HEADDIM, "fa_forward_launch: head_dim=%d has no kernel (64, 128, 256)", p.HD);
  }
}

}  // namespace fa

extern "C" int fa_forward_launch(FwdParams p, int dtype, void* stream) {
  using namespace fa;
  if (!p.Q || !p.K || !p.V || !p.O) return fail(FA_ERR_ARG, "fa_forward_launch: null tensor pointer");
  if (p.NH <= 0 || p.gqa <= 0 || p.NH % p.gqa) return fail(FA_ERR_ARG, "fa_forward_launch: NH=%d gqa=%d", p.NH, p.gqa);
  if (!(p.dropout_p >= 0.0f && p.dropout_p < 1.0f)) return fail(FA_ERR_ARG, "fa_forward_launch: dropout_p=%g", p.dropout_p);
  if ((p.cu_q == nullptr) != (p.cu_k == nullptr)) return fail(FA_ERR_ARG, "fa_forward_launch: cu_q and cu_k go together");
  if (!p.cu_q && p.batch <= 0) return FA_OK;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case FA_F16:
    case FA_BF16: return dispatch_hd(p, dtype, st);
    case FA_F32: return launch_fwd_f32(p, st);
    default: return fail(FA_ERR_DTYPE, "fa_forward_launch: dtype %d not implemented (fp16/bf16/fp32)", dtype);
  }
}
