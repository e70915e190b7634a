// fwd_common.hpp — the forward's sequence views and mask ranges, shared by the fp16/bf16
// kernels (fwd_kernel.hpp) and the fp32 kernels (fwd_f32.hip). Mask contract of the reference
// (kernels/fa_forward.hip:224-233, FableFwdParams in include/fable_attn_abi.h).
#pragma once
#include "attn_device.hpp"

namespace fa {

// the running max (log2 units) moves only when a tile exceeds it by more than this
constexpr float kLazyMax = 8.0f;

struct SeqView {
  int SQ, SK;
  long long q0, k0, v0, o0;  // element offsets of row 0 of this sequence (batch folded in)
  long long lse0;            // element offset of row 0 in LSE
};

// lengths and row-0 offsets of sequence z, head h (dense: batch element z; varlen: packed rows
// cu_q[z].. / cu_k[z].., cut by seqused)
__device__ __forceinline__ SeqView seq_view(const FableFwdParams& p, int z, int h) {
  SeqView sv;
  if (p.cu_q) {
    const int qs = p.cu_q[z], ks = p.cu_k[z];
    sv.SQ = p.cu_q[z + 1] - qs;
    sv.SK = p.cu_k[z + 1] - ks;
    if (p.seqused_q) sv.SQ = min(sv.SQ, p.seqused_q[z]);
    if (p.seqused_k) sv.SK = min(sv.SK, p.seqused_k[z]);
    sv.q0 = (long long)qs * p.sQ.s;
    sv.k0 = (long long)ks * p.sK.s;
    sv.v0 = (long long)ks * p.sV.s;
    sv.o0 = (long long)qs * p.sO.s;
    sv.lse0 = (long long)h * p.lse_sh + qs;
  } else {
    sv.SQ = p.SQ;
    sv.SK = p.SK;
    sv.q0 = (long long)z * p.sQ.b;
    sv.k0 = (long long)z * p.sK.b;
    sv.v0 = (long long)z * p.sV.b;
    sv.o0 = (long long)z * p.sO.b;
    sv.lse0 = (long long)z * p.lse_sb + (long long)h * p.lse_sh;
  }
  return sv;
}

// visible key range [k0, k1) for query rows [r0, r1] (reference mask contract)
template <bool CAUSAL, bool FEAT>
__device__ __forceinline__ void key_range(const FableFwdParams& p, int r0, int r1, int delta, int SK,
                                          int& k0, int& k1) {
  k0 = 0;
  k1 = SK;
  if (CAUSAL) k1 = min(k1, r1 + delta + 1);
  if (FEAT) {
    if (p.win_left >= 0) k0 = max(k0, r0 + delta - p.win_left);
    if (p.win_right >= 0) k1 = min(k1, r1 + delta + p.win_right + 1);
    if (p.attn_chunk > 0) {
      const int a = max(r0 + delta, 0), b = max(r1 + delta, 0);
      k0 = max(k0, (a / p.attn_chunk) * p.attn_chunk);
      k1 = min(k1, (b / p.attn_chunk + 1) * p.attn_chunk);
    }
  }
}

// key j visible to query i (delta = SK - SQ, bottom-right alignment)
template <bool CAUSAL, bool FEAT>
__device__ __forceinline__ bool fwd_visible(const FableFwdParams& p, int i, int j, int delta, int SK) {
  bool ok = j < SK;
  if (CAUSAL) ok = ok && j <= i + delta;
  if (FEAT) {
    if (p.win_left >= 0) ok = ok && j >= i + delta - p.win_left;
    if (p.win_right >= 0) ok = ok && j <= i + delta + p.win_right;
    if (p.attn_chunk > 0) {
      const int cs = (max(i + delta, 0) / p.attn_chunk) * p.attn_chunk;
      ok = ok && j >= cs && j < cs + p.attn_chunk;
    }
  }
  return ok;
}

// Key split of a small forward grid (fp16/bf16, dense or packed varlen batches, no left
// window, chunk or dropout): when the query tiles of a call fill few of the CUs, `n`
// workgroups per query tile each take a contiguous share of its key tiles and write an fp32
// partial O (row-major, head dim p.HD) and its LSE for every row of the tile, at row
// r = item * br + (row within the tile), split after split (item: the query tile's work item,
// sequence-head-major as the grid); a second kernel (fwd_split_combine_kernel, fwd.hip) merges
// them into O and LSE, through the same sequence view as the forward.
struct FwdSplit {
  int n;           // workgroups per query tile; 1: no split, the kernel writes O and LSE itself
  int nqt, br;     // query tiles per (sequence, head) and rows per tile of the launch
  long long rows;  // work items * br
  float* o;        // [n][rows][p.HD]
  float* lse;      // [n][rows], natural log; -inf where a split saw no key of the row
};

// A launch request: the caller's workspace for a key split (null / too small: no split), or a
// query for the bytes a split of this call would use (nothing is launched).
struct FwdWs {
  void* ptr;
  long long bytes;
  bool query;
  long long need;  // out: workspace bytes of the split this call takes (0: none)
};

// the fp16/bf16 forward per kernel width (fwd_d32 ... fwd_d256.hip: head dims up to the width,
// in steps of 8) and the fp32 forward (fwd_f32.hip), dispatched from fable_attn_fwd
int launch_fwd_d32(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws);
int launch_fwd_d64(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws);
int launch_fwd_d96(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws);
int launch_fwd_d128(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws);
int launch_fwd_d160(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws);
int launch_fwd_d192(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws);
int launch_fwd_d224(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws);
int launch_fwd_d256(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws);
int launch_fwd_f32(const FableFwdParams& p, hipStream_t st);
// merge of the key-split partials (fwd.hip)
int launch_fwd_split_combine(const FableFwdParams& p, int dtype, const FwdSplit& sp, hipStream_t st);

}  // namespace fa
