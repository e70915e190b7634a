// bwd_common.hpp — the backward's mask ranges, logit transform and sequence views, shared by
// the fp16/bf16 kernels (bwd.hip) and the fp32 kernels (bwd_f32.hip). Mask contract and math of
// the reference backward (kernels/backward.hip:109-202, FableBwdParams in include/fable_attn_abi.h).
#pragma once
#include "attn_device.hpp"

namespace fa {

// Written with bitwise ands, not early returns: per score the compiler then emits compares and
// one select instead of a divergent branch (with its exec-mask bookkeeping) per score.
template <bool CAUSAL, bool FEAT>
__device__ __forceinline__ bool visible_b(const FableBwdParams& p, int q, int key, int delta, int SQ, int SK) {
  bool ok = (key < SK) & (q < SQ);
  if (CAUSAL) ok &= key <= q + delta;
  if (FEAT) {
    ok &= (p.win_left < 0) | (key >= q + delta - p.win_left);
    ok &= (p.win_right < 0) | (key <= q + delta + p.win_right);
  }
  return ok;
}

// keys visible to query rows [r0, r1]: [k0, k1)
template <bool CAUSAL, bool FEAT>
__device__ __forceinline__ void key_range_b(const FableBwdParams& p, int r0, int r1, int delta, int SK, int& k0, int& k1) {
  k0 = 0;
  k1 = SK;
  if (CAUSAL) k1 = min(k1, r1 + delta + 1);
  if (FEAT) {
    if (p.win_left >= 0) k0 = max(k0, r0 + delta - p.win_left);
    if (p.win_right >= 0) k1 = min(k1, r1 + delta + p.win_right + 1);
  }
}

// queries that see some key in [k0, k1]: [q0, q1)
template <bool CAUSAL, bool FEAT>
__device__ __forceinline__ void query_range_b(const FableBwdParams& p, int k0, int k1, int delta, int SQ, int& q0, int& q1) {
  q0 = 0;
  q1 = SQ;
  if (CAUSAL) q0 = max(q0, k0 - delta);
  if (FEAT) {
    if (p.win_right >= 0) q0 = max(q0, k0 - delta - p.win_right);
    if (p.win_left >= 0) q1 = min(q1, k1 - delta + p.win_left + 1);
  }
}

// logit transform of one score: returns log2-domain logit, and d(logit)/d(scale*q.k)
template <bool FEAT>
__device__ __forceinline__ float bwd_logit2(const FableBwdParams& p, float s, float c_log2, float slope, int q,
                                            int key, float& deriv) {
  if (!FEAT) {
    deriv = 1.0f;
    return s * c_log2;
  }
  float x = s * p.scale;
  deriv = 1.0f;
  if (p.softcap > 0.0f) {
    // (the reciprocal is uniform: one division per call site after hoisting, not per score)
    const float t = tanh_exp(x * (1.0f / p.softcap));
    x = p.softcap * t;
    deriv = 1.0f - t * t;
  }
  x += slope * (float)(key - q);
  return x * kLog2e;
}

// Lengths and first packed rows of sequence b (dense: the whole [SQ, SK] and row 0; varlen:
// from cu_q/cu_k, cut by seqused). Pointer bases are base + b*str.b + row*str.s + h*str.h, so
// varlen callers pass b strides of 0; lse/dsum (b, h, q) is at b*lse_sb + h*lse_sh + qo + q.
struct BwdSeq {
  int SQ, SK;
  long long qo, ko;
};
__device__ __forceinline__ BwdSeq bwd_seq(const FableBwdParams& p, int b) {
  BwdSeq s;
  if (p.cu_q) {
    s.qo = p.cu_q[b];
    s.ko = p.cu_k[b];
    s.SQ = p.cu_q[b + 1] - p.cu_q[b];
    s.SK = p.cu_k[b + 1] - p.cu_k[b];
    if (p.seqused_q) s.SQ = min(s.SQ, p.seqused_q[b]);
    if (p.seqused_k) s.SK = min(s.SK, p.seqused_k[b]);
  } else {
    s.qo = s.ko = 0;
    s.SQ = p.SQ;
    s.SK = p.SK;
  }
  return s;
}

// With a dS workspace the pair kernel stores each dS tile it computes (32 queries x 32 keys,
// 2 KiB) and dQ = dS.K is one product per tile, instead of recomputing S, P and dP.
// Workspace layout: tile (b, h, kb32, qb32) at ((b*Hq + h)*nkb + kb32)*nqb + qb32 (in 1024-element
// tiles; nkb = ceil(SK/32), nqb = ceil(SQ/32) of the longest sequence). A tile is the pair
// kernel's register layout, written with two 16-byte stores per lane: half sh (512 elements)
// holds, for key k, the 16 query slots 16*k .. 16*k+15, and slot 8*hh + e is query
// 16*sh + 8*(e/4) + 4*hh + e%4 (the MFMA C-row order of the S = Q.K^T product). Slot n of the
// 32 in a tile (n = 16*sh + 8*hh + e) is therefore query ds_slot_query(n).
__host__ __device__ inline long long ds_tiles_per_head(int SQ, int SK) {
  return (long long)((SK + 31) >> 5) * ((SQ + 31) >> 5);
}
template <typename T>
__device__ __forceinline__ T* ds_tile(const FableBwdParams& p, int b, int h, int kb32, int qb32) {
  const long long nqb = (p.SQ + 31) >> 5, nkb = (p.SK + 31) >> 5;
  return (T*)p.ds_ws + ((((long long)b * p.Hq + h) * nkb + kb32) * nqb + qb32) * 1024;
}
__device__ __forceinline__ int ds_slot_query(int n) {
  return 16 * (n >> 4) + 8 * ((n >> 2) & 1) + 4 * ((n >> 3) & 1) + (n & 3);
}

// the fp32 backward (bwd_f32.hip), dispatched from fable_attn_bwd
int launch_bwd_f32(const FableBwdParams& p, hipStream_t st);

}  // namespace fa
