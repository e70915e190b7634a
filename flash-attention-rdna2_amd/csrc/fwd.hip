// fwd.hip — the forward's C-ABI entry points (fable_attn_fwd, fable_attn_fwd_ws and the
// workspace query): argument checks and dispatch to the per-width fp16/bf16 kernels
// (fwd_d32.hip .. fwd_d256.hip, kernel in fwd_kernel.hpp) and the fp32 kernels (fwd_f32.hip);
// the merge of a key-split forward's partials. Reference launcher: kernels/fa_forward.hip:424-451.
#include "attn_device.hpp"
#include "fwd_common.hpp"
#include "status.hpp"

namespace fa {

// fp16/bf16: every head dim that is a multiple of 8 up to 256 runs in the kernel of the next
// multiple of 32 (the columns between are zero: at most 24 of them, <= 1.75x the MFMA work at
// head dim 8, <= 1.1x from 80 up)
static int dispatch_hd(const FableFwdParams& p, int dtype, hipStream_t st, FwdWs& ws) {
  if (p.HD <= 0 || p.HD > 256 || p.HD % 8)
    return fail(FA_ERR_HEADDIM, "fable_attn_fwd: head_dim=%d has no kernel (multiples of 8 up to 256)", p.HD);
  switch ((p.HD + 31) / 32) {
    case 1: return launch_fwd_d32(p, dtype, st, ws);
    case 2: return launch_fwd_d64(p, dtype, st, ws);
    case 3: return launch_fwd_d96(p, dtype, st, ws);
    case 4: return launch_fwd_d128(p, dtype, st, ws);
    case 5: return launch_fwd_d160(p, dtype, st, ws);
    case 6: return launch_fwd_d192(p, dtype, st, ws);
    case 7: return launch_fwd_d224(p, dtype, st, ws);
    default: return launch_fwd_d256(p, dtype, st, ws);
  }
}

// Merge of the key-split partials: one thread per (row, 4 head dims). Row r belongs to work
// item w = r / br (query tile, head, sequence, decoded as the forward does) and is query
// qt*br + r % br of that sequence; rows past the sequence's end are left alone.
// LSE = m + log(sum_s exp(lse_s - m)), O = sum_s exp(lse_s - LSE) O_s; a row no split saw gets
// O = 0 and LSE = -inf, as in the unsplit kernel. Every share writes every row of its work
// item (a share without keys writes O = 0, LSE = -inf). All NMAX >= n shares' values are loaded
// before any is used (indices past n - 1 repeat the last share and are not summed), so the
// thread waits out one memory latency instead of one per share; the sum runs in share order.
template <typename T, int NMAX>
__global__ __launch_bounds__(256) void fwd_split_combine_kernel(FableFwdParams p, FwdSplit sp) {
  const int ch = p.HD / 4;
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= sp.rows * ch) return;
  const long long r = gid / ch;
  const int c = (int)(gid - r * ch);
  const int w = (int)(r / sp.br), qti = w % sp.nqt, zh = w / sp.nqt;
  const int h = zh % p.NH, z = zh / p.NH;
  const int qt = p.causal ? sp.nqt - 1 - qti : qti;
  const SeqView sv = seq_view(p, z, h);
  const int q = qt * sp.br + (int)(r - (long long)w * sp.br);
  if (q >= sv.SQ) return;
  float ls[NMAX];
  f32x4 ov[NMAX];
#pragma unroll
  for (int k = 0; k < NMAX; k++) {
    const long long rk = (long long)min(k, sp.n - 1) * sp.rows + r;
    ls[k] = sp.lse[rk];
    ov[k] = *(const f32x4*)(sp.o + rk * p.HD + 4 * c);
  }
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < NMAX; k++)
    if (k < sp.n) m = fmaxf(m, ls[k]);
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  float wsum = 0.0f;
  if (m != -INFINITY) {
#pragma unroll
    for (int k = 0; k < NMAX; k++) {
      if (k < sp.n) {
        const float wk = __expf(ls[k] - m);
        wsum += wk;
        acc += wk * ov[k];
      }
    }
  }
  const float inv = m != -INFINITY ? 1.0f / wsum : 0.0f;
  typename Dt<T>::V4 o;
#pragma unroll
  for (int e = 0; e < 4; e++) o[e] = (T)(acc[e] * inv);
  T* dst = (T*)p.O + sv.o0 + (long long)h * p.sO.h + (long long)q * p.sO.s + 4 * c;
  *(u32x2*)dst = __builtin_bit_cast(u32x2, o);
  if (c == 0 && p.LSE) p.LSE[sv.lse0 + q] = m != -INFINITY ? m + __logf(wsum) : -INFINITY;
}

template <typename T>
static void launch_combine(const FableFwdParams& p, const FwdSplit& sp, dim3 grid, hipStream_t st) {
  if (sp.n <= 2)
    hipLaunchKernelGGL((fwd_split_combine_kernel<T, 2>), grid, dim3(256), 0, st, p, sp);
  else if (sp.n <= 4)
    hipLaunchKernelGGL((fwd_split_combine_kernel<T, 4>), grid, dim3(256), 0, st, p, sp);
  else if (sp.n <= 8)
    hipLaunchKernelGGL((fwd_split_combine_kernel<T, 8>), grid, dim3(256), 0, st, p, sp);
  else
    hipLaunchKernelGGL((fwd_split_combine_kernel<T, 16>), grid, dim3(256), 0, st, p, sp);
}

int launch_fwd_split_combine(const FableFwdParams& p, int dtype, const FwdSplit& sp, hipStream_t st) {
  if (sp.n < 2 || sp.n > 16) return fail(FA_ERR_ARG, "fable_attn_fwd: %d key splits (2..16)", sp.n);
  const long long items = sp.rows * (p.HD / 4);
  const dim3 grid((unsigned)((items + 255) / 256));
  if (dtype == FA_F16)
    launch_combine<_Float16>(p, sp, grid, st);
  else
    launch_combine<__bf16>(p, sp, grid, st);
  return launch_status("fable_attn_fwd (split merge)");
}

// checks shared by the entry points (a workspace query needs no tensor pointers); 1 when the
// call has nothing to do
static int fwd_check(FableFwdParams& p, int dtype, bool query, int& rc) {
  rc = FA_OK;
  if (!query && (!p.Q || !p.K || !p.V || !p.O))
    return rc = fail(FA_ERR_ARG, "fable_attn_fwd: null tensor pointer"), 1;
  if (p.NH <= 0 || p.gqa <= 0 || p.NH % p.gqa) return rc = fail(FA_ERR_ARG, "fable_attn_fwd: NH=%d gqa=%d", p.NH, p.gqa), 1;
  if (!(p.dropout_p >= 0.0f && p.dropout_p < 1.0f)) return rc = fail(FA_ERR_ARG, "fable_attn_fwd: dropout_p=%g", p.dropout_p), 1;
  if ((p.cu_q == nullptr) != (p.cu_k == nullptr)) return rc = fail(FA_ERR_ARG, "fable_attn_fwd: cu_q and cu_k go together"), 1;
  if (!p.cu_q && p.batch <= 0) return 1;
  if (p.SQ < 0 || p.SK < 0) return rc = fail(FA_ERR_ARG, "fable_attn_fwd: SQ=%d SK=%d", p.SQ, p.SK), 1;
  // A window or chunk at least as long as the sequences bounds nothing; dropping it keeps every
  // mask bound the kernels form (row + delta + window) inside 32-bit range.
  if (p.win_left >= p.SK) p.win_left = -1;
  if (p.win_right >= p.SQ) p.win_right = -1;
  if (p.attn_chunk >= p.SK) p.attn_chunk = 0;
  if (dtype != FA_F16 && dtype != FA_BF16 && dtype != FA_F32)
    return rc = fail(FA_ERR_DTYPE, "fable_attn_fwd: dtype %d not implemented (fp16/bf16/fp32)", dtype), 1;
  return 0;
}

static int fwd_run(FableFwdParams p, int dtype, FwdWs& ws, hipStream_t st) {
  int rc;
  if (fwd_check(p, dtype, ws.query, rc)) return rc;
  if (dtype == FA_F32) return ws.query ? FA_OK : launch_fwd_f32(p, st);
  return dispatch_hd(p, dtype, st, ws);
}

}  // namespace fa

extern "C" int fable_attn_fwd(FableFwdParams p, int dtype, void* stream) {
  fa::FwdWs ws{nullptr, 0, false, 0};
  return fa::fwd_run(p, dtype, ws, (hipStream_t)stream);
}

extern "C" int64_t fable_attn_fwd_ws_bytes(FableFwdParams p, int dtype) {
  fa::FwdWs ws{nullptr, 0, true, 0};
  if (fa::fwd_run(p, dtype, ws, nullptr) != FA_OK) return -1;
  return ws.need;
}

extern "C" int fable_attn_fwd_ws(FableFwdParams p, int dtype, void* ws_ptr, int64_t ws_bytes, void* stream) {
  fa::FwdWs ws{ws_ptr, ws_bytes, false, 0};
  return fa::fwd_run(p, dtype, ws, (hipStream_t)stream);
}
