// fwd.hip — fable_attn_fwd, the forward's C-ABI entry point: argument checks and dispatch to
// the per-width fp16/bf16 kernels (fwd_d32.hip .. fwd_d256.hip, kernel in fwd_kernel.hpp) and the
// fp32 kernels (fwd_f32.hip). Reference launcher: kernels/fa_forward.hip:424-451.
#include "attn_device.hpp"
#include "fwd_common.hpp"
#include "status.hpp"

namespace fa {

// fp16/bf16: every head dim that is a multiple of 8 up to 256 runs in the kernel of the next
// multiple of 32 (the columns between are zero: at most 24 of them, <= 1.75x the MFMA work at
// head dim 8, <= 1.1x from 80 up)
static int dispatch_hd(const FableFwdParams& p, int dtype, hipStream_t st) {
  if (p.HD <= 0 || p.HD > 256 || p.HD % 8)
    return fail(FA_ERR_HEADDIM, "fable_attn_fwd: head_dim=%d has no kernel (multiples of 8 up to 256)", p.HD);
  switch ((p.HD + 31) / 32) {
    case 1: return launch_fwd_d32(p, dtype, st);
    case 2: return launch_fwd_d64(p, dtype, st);
    case 3: return launch_fwd_d96(p, dtype, st);
    case 4: return launch_fwd_d128(p, dtype, st);
    case 5: return launch_fwd_d160(p, dtype, st);
    case 6: return launch_fwd_d192(p, dtype, st);
    case 7: return launch_fwd_d224(p, dtype, st);
    default: return launch_fwd_d256(p, dtype, st);
  }
}

}  // namespace fa

extern "C" int fable_attn_fwd(FableFwdParams p, int dtype, void* stream) {
  using namespace fa;
  if (!p.Q || !p.K || !p.V || !p.O) return fail(FA_ERR_ARG, "fable_attn_fwd: null tensor pointer");
  if (p.NH <= 0 || p.gqa <= 0 || p.NH % p.gqa) return fail(FA_ERR_ARG, "fable_attn_fwd: NH=%d gqa=%d", p.NH, p.gqa);
  if (!(p.dropout_p >= 0.0f && p.dropout_p < 1.0f)) return fail(FA_ERR_ARG, "fable_attn_fwd: dropout_p=%g", p.dropout_p);
  if ((p.cu_q == nullptr) != (p.cu_k == nullptr)) return fail(FA_ERR_ARG, "fable_attn_fwd: cu_q and cu_k go together");
  if (!p.cu_q && p.batch <= 0) return FA_OK;
  if (p.SQ < 0 || p.SK < 0) return fail(FA_ERR_ARG, "fable_attn_fwd: SQ=%d SK=%d", p.SQ, p.SK);
  // A window or chunk at least as long as the sequences bounds nothing; dropping it keeps every
  // mask bound the kernels form (row + delta + window) inside 32-bit range.
  if (p.win_left >= p.SK) p.win_left = -1;
  if (p.win_right >= p.SQ) p.win_right = -1;
  if (p.attn_chunk >= p.SK) p.attn_chunk = 0;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case FA_F16:
    case FA_BF16: return dispatch_hd(p, dtype, st);
    case FA_F32: return launch_fwd_f32(p, st);
    default: return fail(FA_ERR_DTYPE, "fable_attn_fwd: dtype %d not implemented (fp16/bf16/fp32)", dtype);
  }
}
