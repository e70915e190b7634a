// ref_abi.hip — the reference's three launchers with the reference's struct layouts
// (package/csrc/fa_iface.h:9-68), so the reference's own glue (package/csrc/dispatch.cpp) binds
// to this library unchanged. Each one maps its struct onto the extended parameter struct and
// runs the same entry point the Python binding uses (fable_attn_fwd / _bwd / _dec); nothing
// else differs. Fields that only the reference's gfx1030 kernels needed (the bf16
// power-of-two shifts) and fields its launcher overwrote (page_shift, page_mask, append) are
// ignored. The reference's launchers return void and printf+abort on a bad argument; these
// return the status and print the message to stderr on failure (a caller that declares them
// void never reads the status).
#include <stdio.h>

#include "attn_device.hpp"
#include "status.hpp"

namespace {

fa_strides st3(const Strides& s) { return fa_strides{s.b, s.h, s.s}; }
fa_strides st3(const Str& s) { return fa_strides{s.b, s.h, s.s}; }

int report(int rc, const char* what) {
  if (rc != FA_OK) fprintf(stderr, "%s: %s\n", what, fable_attn_last_error());
  return rc;
}

}  // namespace

// fa_iface.h:65; reference launcher kernels/fa_forward.hip:424-451
extern "C" int fa_forward_launch(FwdParams r, int dtype, void* stream) {
  // The reference writes LSE[h*SQ + q] with no batch or sequence offset (fa_forward.hip:305-306):
  // only a dense single-batch call has a defined LSE there.
  if (r.LSE && (r.cu_q || r.batch != 1))
    return report(fa::fail(FA_ERR_ARG, "fa_forward_launch: LSE in the reference layout needs a dense call "
                                       "with batch == 1 (it has no batch stride); use fable_attn_fwd"),
                  "fa_forward_launch");
  FableFwdParams p{};
  p.Q = r.Q; p.K = r.K; p.V = r.V; p.O = r.O; p.LSE = r.LSE;
  p.sQ = st3(r.sQ); p.sK = st3(r.sK); p.sV = st3(r.sV); p.sO = st3(r.sO);
  p.SQ = r.SQ; p.SK = r.SK; p.HD = r.HD; p.NH = r.NH; p.gqa = r.gqa;
  p.scale = r.scale; p.softcap = r.softcap;
  p.win_left = r.win_left; p.win_right = r.win_right;
  p.alibi_slopes = r.alibi_slopes;
  p.causal = r.causal;
  p.dropout_p = r.dropout_p; p.philox_seed = r.philox_seed;
  p.cu_q = r.cu_q; p.cu_k = r.cu_k;
  p.batch = r.batch;
  p.attn_chunk = r.attn_chunk;
  p.seqused_q = r.seqused_q; p.seqused_k = r.seqused_k;
  p.lse_sb = 0;
  p.lse_sh = r.SQ;
  return report(fable_attn_fwd(p, dtype, stream), "fa_forward_launch");
}

// fa_iface.h:66; reference launcher kernels/backward.hip:508-521
extern "C" int fable_attn_backward_launch(BwdParams r, int MODE, void* stream) {
  FableBwdParams p{};
  p.Q = r.Q; p.K = r.K; p.V = r.V; p.O = r.O; p.dO = r.dO;
  p.dQ = r.dQ; p.dK = r.dK; p.dV = r.dV;
  p.lse = r.lse; p.dsum = r.dsum;
  p.qs = st3(r.qs); p.ks = st3(r.ks); p.vs = st3(r.vs); p.os = st3(r.os); p.dos = st3(r.dos);
  p.dqs = st3(r.dqs); p.dks = st3(r.dks); p.dvs = st3(r.dvs);
  p.B = r.B; p.Hq = r.Hq; p.Hk = r.Hk; p.SQ = r.SQ; p.SK = r.SK; p.D = r.D; p.gqa = r.gqa;
  p.scale = r.scale; p.softcap = r.softcap;
  p.alibi = r.alibi;
  p.causal = r.causal; p.win_left = r.win_left; p.win_right = r.win_right;
  p.dropout = r.dropout; p.drop_seed = r.drop_seed; p.dropout_p = r.dropout_p; p.keep_scale = r.keep_scale;
  // dense [B][Hq][SQ] lse/dsum (backward.hip:95): zero strides select that layout
  p.lse_sb = 0;
  p.lse_sh = 0;
  return report(fable_attn_bwd(p, MODE, stream), "fable_attn_backward_launch");
}

// fa_iface.h:67-68; reference launcher kernels/fa_decode.hip:343-362
extern "C" int fa_decode_launch(DecParams r, int dtype, void* stream, const void* new_k, const void* new_v) {
  FableDecParams p{};
  p.q = r.q; p.Kc = r.Kc; p.Vc = r.Vc;
  p.block_table = r.block_table;
  p.o = r.o;
  p.scratch = r.scratch;
  p.ctx_len = r.ctx_len;
  p.cos = r.cos; p.sin = r.sin;
  p.batch = r.batch; p.NH = r.NH; p.gqa = r.gqa; p.HD = r.HD; p.page = r.page;
  p.max_blocks = r.max_blocks; p.nsplit = r.nsplit; p.window = r.window;
  p.rotary = r.rotary;
  p.scale = r.scale;
  p.leftpad = r.leftpad;
  p.lse_out = r.lse_out;
  p.softcap = r.softcap;
  p.alibi = r.alibi;
  p.nq = r.nq;
  p.rotary_dim = r.rotary_dim;
  p.rotary_pos = r.rotary_pos;
  return report(fable_attn_dec(p, dtype, stream, new_k, new_v), "fa_decode_launch");
}
