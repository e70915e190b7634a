/*
 * fable_attn_abi.h — the C-ABI boundary of the MI355X (gfx950) exact-attention library
 * `libfable_attn_hip.so`.
 *
 * One header, included verbatim by the HIP translation units that implement the entry points
 * and by every host caller. Parameter structs are passed BY VALUE, as the reference passes
 * them, and are plain C: device pointers as `const void*` / `void*`, strides in ELEMENTS, the
 * innermost (head_dim) stride is always 1. Every row of every tensor (its base pointer plus any
 * combination of its strides) must be 16-byte aligned: the kernels move rows in 16-byte loads
 * and stores (for 16-bit types, pointers and strides multiples of 8 elements). No torch or HIP
 * types appear in any signature; a stream is `void*` (a `hipStream_t`, NULL = the legacy
 * default stream). Nothing allocates: every output, workspace and scratch buffer belongs to the
 * caller. Work is enqueued asynchronously on the stream; no entry point synchronises.
 *
 * Two sets of entry points (paths relative to the reference repository root):
 *
 * 1. The reference's own launchers, bit for bit: the structs Strides/FwdParams, Str/BwdParams
 *    and DecParams have exactly the layout of package/csrc/fa_iface.h:9-63 and the three
 *    launchers its :65-68 declares, so the reference's compiled glue
 *    (package/csrc/dispatch.cpp) links against this library unchanged. The fields the
 *    reference needed only for gfx1030 (bf16 power-of-two shifts sc_q/sc_k/sc_v and
 *    shQ/shK/shV/shdO; page_shift/page_mask/append, which its launcher overwrote) are accepted
 *    and ignored: gfx950 MFMA takes bf16 natively and the decode launcher derives the rest.
 *    The reference's launchers return void; these return an int status (FA_OK == 0) in the
 *    return register, which a caller declaring them void ignores. On failure they also print
 *    the message to stderr, since such a caller never reads the status (the reference printed
 *    and aborted).
 *
 * 2. This library's extended entry points (fable_attn_fwd/bwd/dec with FableFwdParams,
 *    FableBwdParams, FableDecParams), used by the Python binding: the forward writes LSE for
 *    every batch element and for packed variable-length batches (lse_sb/lse_sh), the backward
 *    takes packed variable-length batches natively (cu_q/cu_k) and an optional dS workspace
 *    that removes the dQ kernel's recomputation, plus the combine kernel, the decode split
 *    planner and introspection.
 */
#ifndef FABLE_ATTN_ABI_H
#define FABLE_ATTN_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FABLE_ATTN_ABI_VERSION 5

/* dtype codes, same values as the reference (fa_forward.hip:403, backward.hip:25) */
enum { FA_F16 = 0, FA_BF16 = 1, FA_F32 = 2 };

/* status codes returned by every launcher */
enum {
  FA_OK = 0,
  FA_ERR_DTYPE = 1,        /* dtype not implemented by this entry point */
  FA_ERR_HEADDIM = 2,      /* head_dim has no instantiated kernel */
  FA_ERR_ARG = 3,          /* inconsistent argument (shape, alignment, null pointer) */
  FA_ERR_UNSUPPORTED = 4,  /* feature combination not implemented */
  FA_ERR_LAUNCH = 5        /* the HIP runtime rejected the launch */
};

/* ========================================================================================
 * 1. The reference's launchers with the reference's struct layouts (fa_iface.h:9-68).
 * ======================================================================================== */

/* Element strides {batch, head, seq} of a [B, H, S, D] view (fa_iface.h:9, :27). */
typedef struct Strides { long long b, h, s; } Strides;
typedef struct Str { long long b, h, s; } Str;

/* fa_iface.h:10-24. Semantics as FableFwdParams below, with these limits of the reference
 * layout: LSE (optional) is [NH][SQ] of ONE batch element — there is no batch stride, so a call
 * with LSE != NULL must be dense with batch == 1 (the reference's glue calls once per batch
 * element, dispatch.cpp:61-78); sc_q/sc_k/sc_v are ignored. */
typedef struct FwdParams {
  const void* Q; const void* K; const void* V; void* O; float* LSE;
  Strides sQ, sK, sV, sO;
  int SQ, SK, HD, NH, gqa;
  float scale, softcap;
  int win_left, win_right;
  const float* alibi_slopes;
  int causal;
  float dropout_p; unsigned long long philox_seed;
  const int* cu_q; const int* cu_k;
  int batch;
  float sc_q, sc_k, sc_v;
  int attn_chunk;
  const int* seqused_q; const int* seqused_k;
} FwdParams;

/* fa_iface.h:28-38. Dense [B,H,S,D] views only; lse and dsum are [B][Hq][SQ] fp32 (dsum is a
 * caller-allocated workspace, overwritten); shQ/shK/shV/shdO are ignored. The dQ kernel
 * recomputes S and dP (this struct has no field for a dS workspace; fable_attn_bwd takes one). */
typedef struct BwdParams {
  const void *Q, *K, *V, *O, *dO; void *dQ, *dK, *dV;
  const float *lse; float *dsum;
  Str qs, ks, vs, os, dos, dqs, dks, dvs;
  int B, Hq, Hk, SQ, SK, D, gqa;
  float scale, softcap;
  const float *alibi;
  int causal, win_left, win_right;
  int dropout; unsigned long long drop_seed; float dropout_p, keep_scale;
  int shQ, shK, shV, shdO;
} BwdParams;

/* fa_iface.h:42-63. Semantics as FableDecParams below; page_shift/page_mask/append are derived
 * by the launcher (as the reference's launcher overwrote them) and sc_q/sc_k/sc_v are ignored.
 * scratch holds batch*nq*NH*nsplit*(HD+2) floats. */
typedef struct DecParams {
  const void* q;
  const void* Kc; const void* Vc;
  const int* block_table;
  void* o;
  float* scratch;
  const int* ctx_len;
  const float* cos; const float* sin;
  int batch, NH, gqa, HD, page, max_blocks, nsplit, window;
  int page_shift, page_mask;
  int rotary;
  float scale;
  float sc_q, sc_k, sc_v;
  const int* leftpad;
  float* lse_out;
  float softcap;
  const float* alibi;
  int nq;
  int append;
  int rotary_dim;
  const int* rotary_pos;
} DecParams;

/* fa_iface.h:65  extern "C" void fa_forward_launch(FwdParams p, int dtype, void* stream) */
int fa_forward_launch(FwdParams p, int dtype, void* stream);

/* fa_iface.h:66  extern "C" void fable_attn_backward_launch(BwdParams pr, int MODE, void* stream) */
int fable_attn_backward_launch(BwdParams pr, int MODE, void* stream);

/* fa_iface.h:67-68  extern "C" void fa_decode_launch(DecParams p, int dtype, void* stream,
 *                                                    const void* new_k, const void* new_v) */
int fa_decode_launch(DecParams p, int dtype, void* stream, const void* new_k, const void* new_v);

/* ========================================================================================
 * 2. This library's extended entry points (used by the Python binding).
 * ======================================================================================== */

/* Element strides of a [batch, head, seq, head_dim] view; head_dim stride is 1. */
typedef struct fa_strides {
  int64_t b, h, s;
} fa_strides;

/* Forward parameters: the reference's FwdParams (fa_iface.h:10-24, fa_forward.hip:23-49)
 * without the bf16 shift fields, plus LSE strides.
 * Dense: Q [B,NH,SQ,HD], K/V [B,NH/gqa,SK,HD] as strided views, batch = B.
 * Varlen: cu_q/cu_k non-null (int32, batch+1 entries), SQ/SK = max_seqlen_q/k (grid size),
 *         sequence z occupies rows cu_q[z]..cu_q[z+1] (seq stride sQ.s), sQ.b/sK.b are ignored;
 *         seqused_q/seqused_k (optional) shorten sequence z to seqused[z] rows.
 * Visibility of key j to query i (delta = SK_z - SQ_z, bottom-right alignment):
 *         causal: j <= i+delta;  win_left >= 0: j >= i+delta-win_left;
 *         win_right >= 0: j <= i+delta+win_right;  attn_chunk > 0: j in the chunk of
 *         max(i+delta,0). Logit = scale*q.k, then softcap*tanh(logit/softcap) if softcap > 0,
 *         then + alibi_slopes[h]*(j-i). A row with no visible key gets O = 0 and LSE = -inf.
 * LSE (natural log, fp32, optional): dense LSE[b*lse_sb + h*lse_sh + i];
 *         varlen LSE[h*lse_sh + cu_q[z] + i] (lse_sb ignored). */
typedef struct FableFwdParams {
  const void* Q;
  const void* K;
  const void* V;
  void* O;
  float* LSE;
  fa_strides sQ, sK, sV, sO;
  int32_t SQ, SK, HD, NH, gqa;
  float scale, softcap;
  int32_t win_left, win_right;
  const float* alibi_slopes;
  int32_t causal;
  /* dropout: Philox4x32-10 word 0 on (idx, 0, 0) under key philox_seed, idx = (h*SQ + q)*SK + key
   * (per-sequence SQ/SK for varlen); kept iff (word0 >> 8) * 2^-24 >= dropout_p, scaled by
   * 1/(1-dropout_p) after the row sum (fa_common.hpp:71-88, fa_forward.hip:255-259) */
  float dropout_p;
  uint64_t philox_seed;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int32_t batch;
  int32_t attn_chunk;
  const int32_t* seqused_q;
  const int32_t* seqused_k;
  int64_t lse_sb, lse_sh;
} FableFwdParams;

/* Backward parameters: the reference's BwdParams (fa_iface.h:28-38, backward.hip:59-73) without
 * the bf16 shift fields, plus packed variable-length batches and the dS workspace.
 * Q,O,dO,dQ [B,Hq,SQ,D]; K,V,dK,dV [B,Hk,SK,D] (strided, D contiguous);
 * lse [B,Hq,SQ] fp32 contiguous (from the forward); dsum: fp32 workspace [B,Hq,SQ]
 * (caller-allocated, overwritten). Masking/softcap/alibi exactly as FableFwdParams. */
typedef struct FableBwdParams {
  const void* Q;
  const void* K;
  const void* V;
  const void* O;
  const void* dO;
  void* dQ;
  void* dK;
  void* dV;
  const float* lse;
  float* dsum;
  fa_strides qs, ks, vs, os, dos, dqs, dks, dvs;
  int32_t B, Hq, Hk, SQ, SK, D, gqa;
  float scale, softcap;
  const float* alibi;
  int32_t causal, win_left, win_right;
  int32_t dropout; /* the forward's stream: drop_seed = its philox_seed, keep_scale = 1/(1-p) */
  uint64_t drop_seed;
  float dropout_p, keep_scale;
  /* Packed variable-length sequences (cu_q != NULL; the reference has no native varlen
   * backward and loops over sequences in Python, flash_attn_interface.py:523-540). Rows of
   * sequence b start at row cu_q[b] of the packed [total_q, H, D] Q, O, dO, dQ and at row
   * cu_k[b] of K, V, dK, dV (set the b strides to 0); B is the number of sequences, SQ/SK the
   * longest lengths (they size the grid); seqused_q/k, when set, cut a sequence short.
   * lse/dsum element (b, h, q) sits at b*lse_sb + h*lse_sh + (cu_q ? cu_q[b] : 0) + q; with
   * cu_q == NULL and both strides 0 the dense [B,Hq,SQ] layout is assumed. */
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* seqused_q;
  const int32_t* seqused_k;
  int64_t lse_sb, lse_sh;
  /* dS workspace (no reference counterpart; ABI version 3). When ds_ws is set and ds_ws_bytes
   * >= fable_attn_bwd_ds_bytes(p, dtype) > 0, the dK/dV kernel writes every dS tile it computes
   * once, and dQ = dS.K becomes one product per tile; otherwise a dQ kernel recomputes S and
   * dP. Device memory, 16-byte aligned (an unaligned buffer is not used), any contents on
   * entry, scratch on exit. */
  void* ds_ws;
  int64_t ds_ws_bytes;
} FableBwdParams;

/* Paged-KV decode parameters: the reference's DecParams (fa_iface.h:42-63, fa_decode.hip:13-35)
 * without the fields its launcher derived or that only gfx1030 needed.
 * q [batch, nq, NH, HD] contiguous; Kc/Vc [num_blocks, page, NH/gqa, HD] contiguous;
 * block_table [batch, max_blocks] int32; ctx_len [batch] int32 = cache length BEFORE the
 * append (flash_attn cache_seqlens); o [batch, nq, NH, HD]; scratch fp32
 * [batch*nq*NH*nsplit*(HD+2)] (caller-allocated; may be NULL when nsplit == 1 with fp16/bf16,
 * where the partial kernel writes o and lse_out itself); lse_out [batch*nq*NH] or NULL.
 * New token tk of sequence b sits at position ctx_len[b]+tk and sees keys
 * [max(leftpad[b], pos-window+1 if window>=0), ctx_len[b] + (append ? tk+1 : 0)).
 * page must be a power of two. rotary: 0 none, 1 neox (half split), 2 interleaved (pairs);
 * cos/sin tables [seqlen_ro, rotary_dim/2] fp32, row chosen by (rotary_pos ? rotary_pos[b] :
 * ctx_len[b]) + tk; rotary_dim 0 means HD. */
typedef struct FableDecParams {
  const void* q;
  const void* Kc;
  const void* Vc;
  const int32_t* block_table;
  void* o;
  float* scratch;
  const int32_t* ctx_len;
  const float* cos;
  const float* sin;
  int32_t batch, NH, gqa, HD, page, max_blocks, nsplit, window;
  int32_t rotary;
  float scale;
  const int32_t* leftpad;
  float* lse_out;
  float softcap;
  const float* alibi;
  int32_t nq;
  int32_t rotary_dim;
  const int32_t* rotary_pos;
} FableDecParams;

/* LSE-weighted merge of split partial results (flash_attn_combine).
 * Reference: package/fable_attn/flash_attn_interface.py:567-580 (pure torch there).
 * out_partial [nsplit, B, S, H, D] (dtype of in_dtype) with element strides
 * op_s (split), op_b, op_s_seq, op_h (D contiguous); lse_partial [nsplit, B, H, S] fp32 with
 * strides lp_s, lp_b, lp_h, lp_seq; out [B, S, H, D] dense in out_dtype. */
typedef struct CombineParams {
  const void* out_partial;
  const float* lse_partial;
  void* out;
  int32_t nsplit, B, S, H, D;
  int64_t op_split, op_b, op_seq, op_h;
  int64_t lp_split, lp_b, lp_h, lp_seq;
  int32_t in_dtype, out_dtype;
} CombineParams;

/* Entry points. Each returns FA_OK or an FA_ERR_* code; work is enqueued asynchronously on
 * `stream`; nothing is allocated or freed; every pointer is device memory. */

/* the forward (reference launcher kernels/fa_forward.hip:424-451); dense or packed varlen */
int fable_attn_fwd(FableFwdParams p, int dtype, void* stream);

/* The forward with a caller-owned workspace for a key split: when the query tiles of a call fill
 * few of the CUs (fp16/bf16, dense or packed varlen batches, no left window, chunk or dropout),
 * several workgroups per query tile each take a share of its keys, write fp32 partials to `ws`,
 * and a second kernel merges them into O and LSE. fable_attn_fwd_ws_bytes gives the bytes this call would use (0: no
 * split for this call; -1: the call is invalid, see fable_attn_last_error); a `ws` that is NULL,
 * smaller, or not 256-byte aligned runs the call unsplit. Same results as fable_attn_fwd up to
 * fp32 summation order. No reference counterpart (the reference launches one workgroup per query
 * tile, kernels/fa_forward.hip:424-451); added for short sequences with few heads. */
int64_t fable_attn_fwd_ws_bytes(FableFwdParams p, int dtype);
int fable_attn_fwd_ws(FableFwdParams p, int dtype, void* ws, int64_t ws_bytes, void* stream);

/* the backward (reference launcher kernels/backward.hip:508-521); dense or packed varlen */
int fable_attn_bwd(FableBwdParams p, int dtype, void* stream);

/* Bytes of FableBwdParams.ds_ws the backward can use for these shapes (fp16/bf16 at every head
 * dim; 0 for fp32, which recomputes, or when no query sees a key). No reference counterpart: the
 * reference backward recomputes dS in its dQ kernel (backward.hip:298-387). A table of
 * ceil(SK/32)+1 ints padded to a multiple of 256 bytes, then 2 KiB per 32x32 (query, key) tile
 * holding a visible pair, for every (batch, q head). */
int64_t fable_attn_bwd_ds_bytes(FableBwdParams p, int dtype);

/* paged-KV decode (reference launcher kernels/fa_decode.hip:343-362).
 * new_k/new_v [batch, nq, NH/gqa, HD] (NULL = no append) are written into the paged cache
 * (with rotary on k) before attention, in stream order: no device-wide synchronisation. */
int fable_attn_dec(FableDecParams p, int dtype, void* stream, const void* new_k, const void* new_v);

/* fable_attn_dec without allocation. No counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). p.scratch is ignored: the split partials go to a fixed device array owned
 * by the library, one per GPU, kept until the process ends, of
 * fable_attn_dec_noalloc_max_floats() floats (16 MiB); a call needing more
 * (batch*nq*NH*nsplit*(HD+2) floats) fails with FA_ERR_ARG, except with nsplit == 1 in
 * fp16/bf16, which never touches the array and has no size limit. Nothing is allocated or freed.
 * The stream's device must be the current device. Calls that overlap on one GPU share the
 * array and race: the caller serialises them. Otherwise exactly fable_attn_dec (same kernels,
 * same results). */
int fable_attn_dec_noalloc(FableDecParams p, int dtype, void* stream, const void* new_k,
                           const void* new_v);
int64_t fable_attn_dec_noalloc_max_floats(void);

/* split count chosen for a decode call (reference heuristic: dispatch.cpp:182-200, retuned for
 * 256 CUs); num_splits_hint > 0 is honoured (clamped to [1, 512]). */
int fa_decode_num_splits(int batch, int nq, int NH, int gqa, int64_t ctx_bound, int num_splits_hint);

/* flash_attn_combine as a kernel (the reference computes it with torch ops). */
int fa_combine_launch(CombineParams p, void* stream);

/* introspection for bindings and tests */
int fable_attn_abi_version(void);
/* sizeof of a struct: 0 FableFwdParams, 1 FableBwdParams, 2 FableDecParams, 3 CombineParams,
 * 4 fa_strides, 5 FwdParams, 6 BwdParams, 7 DecParams (0 for any other value) */
size_t fable_attn_struct_size(int which);
const char* fable_attn_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* FABLE_ATTN_ABI_H */
