// bwd.hip — fable_attn_bwd and fable_attn_bwd_ds_bytes, the backward's C-ABI entry points:
// argument checks and dispatch to the per-width fp16/bf16 kernels (bwd_dNN.hip, kernels in
// bwd_kernel.hpp) and the fp32 kernels (bwd_f32.hip). Reference launcher:
// kernels/backward.hip:508-521.
#include "bwd_kernel.hpp"

namespace fa {

// fp16/bf16: every head dim that is a multiple of 8 up to 256 runs in the kernel of the next
// multiple of 32 (bwd_dNN.hip; the columns between are zero)
static int bwd_dispatch(const FableBwdParams& p, int dtype, hipStream_t st) {
  if (p.D <= 0 || p.D > 256 || p.D % 8)
    return fail(FA_ERR_HEADDIM, "fable_attn_bwd: head_dim=%d has no kernel (multiples of 8 up to 256)", p.D);
  switch (bwd_width(p.D)) {
    case 32: return launch_bwd_d32(p, dtype, st);
    case 64: return launch_bwd_d64(p, dtype, st);
    case 96: return launch_bwd_d96(p, dtype, st);
    case 128: return launch_bwd_d128(p, dtype, st);
    case 160: return launch_bwd_d160(p, dtype, st);
    case 192: return launch_bwd_d192(p, dtype, st);
    case 224: return launch_bwd_d224(p, dtype, st);
    default: return launch_bwd_d256(p, dtype, st);
  }
}

}  // namespace fa

namespace fa {
// A window at least as long as the sequences bounds nothing: dropping it keeps every mask bound
// in 32 bits (and the dS workspace layout the same for the size query and the launch).
static void normalize_windows(FableBwdParams& p) {
  if (p.win_left >= p.SK) p.win_left = -1;
  if (p.win_right >= p.SQ) p.win_right = -1;
}
}  // namespace fa

extern "C" int64_t fable_attn_bwd_ds_bytes(FableBwdParams p, int dtype) {
  if ((dtype != FA_F16 && dtype != FA_BF16) || p.D <= 0 || p.D % 8 || fa::bwd_width(p.D) > 256 || p.B <= 0 ||
      p.Hq <= 0)
    return 0;
  fa::normalize_windows(p);
  return fa::ds_bytes(p);
}

extern "C" int fable_attn_bwd(FableBwdParams p, int dtype, void* stream) {
  using namespace fa;
  if (!p.Q || !p.K || !p.V || !p.O || !p.dO || !p.dQ || !p.dK || !p.dV || !p.lse || !p.dsum)
    return fail(FA_ERR_ARG, "fable_attn_bwd: null pointer");
  if (p.Hq <= 0 || p.Hk <= 0 || p.Hq % p.Hk || p.gqa != p.Hq / p.Hk)
    return fail(FA_ERR_ARG, "fable_attn_bwd: Hq=%d Hk=%d gqa=%d", p.Hq, p.Hk, p.gqa);
  if (p.dropout && !(p.dropout_p >= 0.0f && p.dropout_p < 1.0f))
    return fail(FA_ERR_ARG, "fable_attn_bwd: dropout_p=%g", p.dropout_p);
  if ((p.cu_q == nullptr) != (p.cu_k == nullptr))
    return fail(FA_ERR_ARG, "fable_attn_bwd: cu_q and cu_k go together");
  if (p.B <= 0 || p.SQ < 0 || p.SK < 0) return FA_OK;  // empty ranges write zero gradients
  normalize_windows(p);
  if (!p.cu_q && p.lse_sb == 0 && p.lse_sh == 0) {  // dense [B,Hq,SQ] LSE / dsum
    p.lse_sh = p.SQ;
    p.lse_sb = (int64_t)p.Hq * p.SQ;
  }
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case FA_F16:
    case FA_BF16: return bwd_dispatch(p, dtype, st);
    case FA_F32: return launch_bwd_f32(p, st);
    default: return fail(FA_ERR_DTYPE, "fable_attn_bwd: dtype %d not implemented (fp16/bf16/fp32)", dtype);
  }
}
