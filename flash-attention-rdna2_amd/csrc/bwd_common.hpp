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
// Workspace layout: only the tiles some query of the 32-row block sees some key of the 32-key
// block of are stored (about half the rectangle under a causal mask, a band under a window).
// Key block kb keeps the query blocks [qb0(kb), qb1(kb)) (ds_span, the query_range_b of the
// block). The workspace starts with a table of nkb + 1 ints, padded to 256 bytes:
// tbl[kb] = (tiles of key blocks before kb) - qb0(kb), tbl[nkb] = T, the tiles per (b, h); tile
// (b, h, kb, qb) follows at ((b*Hq + h)*T + tbl[kb] + qb) tiles of 1024 elements. The dsum kernel
// writes the table (workgroup 0), before the pair kernel runs. Packed variable-length batches
// keep every query block of the longest sequence (qb0 = 0, qb1 = ceil(SQ/32)). A tile is the
// pair kernel's register layout, written with two 16-byte stores per lane: half sh (512
// elements) holds, for key k, the 16 query slots 16*k .. 16*k+15, and slot 8*hh + e is query
// 16*sh + 8*(e/4) + 4*hh + e%4 (the MFMA C-row order of the S = Q.K^T product). Slot n of the
// 32 in a tile (n = 16*sh + 8*hh + e) is therefore query ds_slot_query(n).
// (The windows are those fable_attn_bwd normalised: a bound at least as long as the sequences
// is -1, so every term below stays in 32-bit range.)
__host__ __device__ inline void ds_span(const FableBwdParams& p, int kb, int& qb0, int& qb1) {
  const int nqb = (p.SQ + 31) >> 5;
  if (p.cu_q) {
    qb0 = 0;
    qb1 = nqb;
    return;
  }
  const int k0 = 32 * kb, k1 = (k0 + 31 < p.SK - 1 ? k0 + 31 : p.SK - 1), delta = p.SK - p.SQ;
  int q0 = 0, q1 = p.SQ;
  if (p.causal && k0 - delta > q0) q0 = k0 - delta;
  if (p.win_right >= 0 && k0 - delta - p.win_right > q0) q0 = k0 - delta - p.win_right;
  if (p.win_left >= 0 && k1 - delta + p.win_left + 1 < q1) q1 = k1 - delta + p.win_left + 1;
  if (q1 <= q0) {
    qb0 = qb1 = 0;
  } else {
    qb0 = q0 >> 5;
    qb1 = (q1 + 31) >> 5;
  }
}
// ds_span inside a kernel instance: CAUSAL is p.causal, and the window terms exist only under
// FEAT (fable_attn_bwd picks a FEAT instance for every window but the causal right bound 0,
// which the causal term already covers), so the runtime flag tests drop out
template <bool CAUSAL, bool FEAT>
__device__ __forceinline__ void ds_span_k(const FableBwdParams& p, int kb, int& qb0, int& qb1) {
  const int nqb = (p.SQ + 31) >> 5;
  if (p.cu_q) {
    qb0 = 0;
    qb1 = nqb;
    return;
  }
  const int k0 = 32 * kb, delta = p.SK - p.SQ;
  int q0 = 0, q1 = p.SQ;
  if (CAUSAL) q0 = max(q0, k0 - delta);
  if (FEAT) {
    if (p.win_right >= 0) q0 = max(q0, k0 - delta - p.win_right);
    if (p.win_left >= 0) q1 = min(q1, min(k0 + 31, p.SK - 1) - delta + p.win_left + 1);
  }
  if (q1 <= q0) {
    qb0 = qb1 = 0;
  } else {
    qb0 = q0 >> 5;
    qb1 = (q1 + 31) >> 5;
  }
}
__host__ __device__ inline long long ds_header_bytes(int nkb) {
  return ((long long)(nkb + 1) * 4 + 255) / 256 * 256;
}
// tiles per (b, h) of the layout above (host side, for the workspace size)
inline long long ds_tiles_per_head(const FableBwdParams& p) {
  const int nkb = (p.SK + 31) >> 5;
  long long t = 0;
  for (int kb = 0; kb < nkb; kb++) {
    int a, z;
    ds_span(p, kb, a, z);
    t += z - a;
  }
  return t;
}
// the table of the layout above, built by one workgroup of 256 threads (all of them call it)
__device__ inline void ds_build_table(const FableBwdParams& p) {
  __shared__ int part[256];
  const int nkb = (p.SK + 31) >> 5, t = threadIdx.x;
  const int per = (nkb + 255) / 256, kb0 = t * per, kb1 = min(kb0 + per, nkb);
  int sum = 0;
  for (int kb = kb0; kb < kb1; kb++) {
    int a, z;
    ds_span(p, kb, a, z);
    sum += z - a;
  }
  part[t] = sum;
  __syncthreads();
  if (t == 0) {
    int run = 0;
    for (int i = 0; i < 256; i++) {
      const int x = part[i];
      part[i] = run;
      run += x;
    }
  }
  __syncthreads();
  int* tbl = (int*)p.ds_ws;
  int run = part[t];
  for (int kb = kb0; kb < kb1; kb++) {
    int a, z;
    ds_span(p, kb, a, z);
    tbl[kb] = run - a;
    run += z - a;
  }
  if (t == 255) tbl[nkb] = run;
}
// tile (b, h) base and the table of the layout above
template <typename T>
__device__ __forceinline__ T* ds_head_tiles(const FableBwdParams& p, int b, int h, int tiles_per_head) {
  const int nkb = (p.SK + 31) >> 5;
  return (T*)((char*)p.ds_ws + ds_header_bytes(nkb)) + ((long long)b * p.Hq + h) * tiles_per_head * 1024;
}
__device__ __forceinline__ int ds_slot_query(int n) {
  return 16 * (n >> 4) + 8 * ((n >> 2) & 1) + 4 * ((n >> 3) & 1) + (n & 3);
}

// the fp32 backward (bwd_f32.hip), dispatched from fable_attn_bwd
int launch_bwd_f32(const FableBwdParams& p, hipStream_t st);

// kernel width for head dim D (a multiple of 8 up to 256): the next multiple of 32
inline int bwd_width(int D) { return (D + 31) / 32 * 32; }
// the fp16/bf16 kernels of each width (bwd_dNN.hip), dispatched from fable_attn_bwd
int launch_bwd_d32(const FableBwdParams& p, int dtype, hipStream_t st);
int launch_bwd_d64(const FableBwdParams& p, int dtype, hipStream_t st);
int launch_bwd_d96(const FableBwdParams& p, int dtype, hipStream_t st);
int launch_bwd_d128(const FableBwdParams& p, int dtype, hipStream_t st);
int launch_bwd_d160(const FableBwdParams& p, int dtype, hipStream_t st);
int launch_bwd_d192(const FableBwdParams& p, int dtype, hipStream_t st);
int launch_bwd_d224(const FableBwdParams& p, int dtype, hipStream_t st);
int launch_bwd_d256(const FableBwdParams& p, int dtype, hipStream_t st);

}  // namespace fa
