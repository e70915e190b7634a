// combine.hip — flash_attn_combine as one kernel: LSE-weighted merge of split partials.
//
// Reference math (pure torch there): package/fable_attn/flash_attn_interface.py:567-580:
//   m = max_s lse_s;  w_s = exp(lse_s - m);  out = sum_s w_s * out_s / max(sum_s w_s, 1e-30).
// One thread per (row, head-dim element); a row is (b, seq, h). Rows whose partials are all
// empty (every lse = -inf) produce 0 instead of the NaN the torch expression yields.
#include "attn_device.hpp"
#include "status.hpp"

namespace fa {

template <typename TI>
__device__ __forceinline__ float ld_as_f32(const void* p, long long i) {
  return (float)((const TI*)p)[i];
}

template <typename TI, typename TO, int NC>
__global__ __launch_bounds__(256) void combine_kernel(CombineParams c) {
  const long long rows = (long long)c.B * c.S * c.H;
  const int dgrp = (c.D + 63) / 64;
  const long long gid = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (gid >= rows * dgrp) return;
  const long long row = gid / dgrp;
  const int d = (int)(gid % dgrp) * 64 + (threadIdx.x & 63);
  const int h = (int)(row % c.H);
  const long long bs = row / c.H;
  const int s = (int)(bs % c.S), b = (int)(bs / c.S);
  const long long lbase = (long long)b * c.lp_b + (long long)h * c.lp_h + (long long)s * c.lp_seq;
  // splits in chunks of NC (2, 4 or 8, at least the split count up to 8) whose loads are all
  // issued before any is used (indices past the last split repeat it and are not used): a few
  // memory latencies instead of one per split; sums in split order
  constexpr int kC = NC;
  const int ns = c.nsplit;
  float m = -INFINITY;
  for (int k0 = 0; k0 < ns; k0 += kC) {
    float l[kC];
#pragma unroll
    for (int u = 0; u < kC; u++) l[u] = c.lse_partial[lbase + (long long)min(k0 + u, ns - 1) * c.lp_split];
#pragma unroll
    for (int u = 0; u < kC; u++)
      if (k0 + u < ns) m = fmaxf(m, l[u]);
  }
  if (d >= c.D) return;
  const long long obase = (long long)b * c.op_b + (long long)s * c.op_seq + (long long)h * c.op_h + d;
  float acc = 0.0f, ws = 0.0f;
  if (m != -INFINITY) {
    for (int k0 = 0; k0 < ns; k0 += kC) {
      float l[kC], o[kC];
#pragma unroll
      for (int u = 0; u < kC; u++) {
        const long long k = min(k0 + u, ns - 1);
        l[u] = c.lse_partial[lbase + k * c.lp_split];
        o[u] = ld_as_f32<TI>(c.out_partial, obase + k * c.op_split);
      }
#pragma unroll
      for (int u = 0; u < kC; u++) {
        if (k0 + u < ns) {
          const float w = __expf(l[u] - m);
          ws += w;
          acc += w * o[u];
        }
      }
    }
  }
  const float r = m != -INFINITY ? acc / fmaxf(ws, 1e-30f) : 0.0f;
  ((TO*)c.out)[row * c.D + d] = (TO)r;
}

template <typename TI, typename TO>
static void launch_nc(const CombineParams& c, dim3 grid, dim3 block, hipStream_t st) {
  if (c.nsplit <= 2)
    hipLaunchKernelGGL((combine_kernel<TI, TO, 2>), grid, block, 0, st, c);
  else if (c.nsplit <= 4)
    hipLaunchKernelGGL((combine_kernel<TI, TO, 4>), grid, block, 0, st, c);
  else
    hipLaunchKernelGGL((combine_kernel<TI, TO, 8>), grid, block, 0, st, c);
}

template <typename TI>
static int launch_in(const CombineParams& c, hipStream_t st) {
  const long long items = (long long)c.B * c.S * c.H * ((c.D + 63) / 64);
  dim3 grid((unsigned)((items + 3) / 4)), block(256);
  switch (c.out_dtype) {
    case FA_F16: launch_nc<TI, _Float16>(c, grid, block, st); break;
    case FA_BF16: launch_nc<TI, __bf16>(c, grid, block, st); break;
    case FA_F32: launch_nc<TI, float>(c, grid, block, st); break;
    default: return fail(FA_ERR_DTYPE, "fa_combine_launch: out dtype %d", c.out_dtype);
  }
  return launch_status("fa_combine_launch");
}

}  // namespace fa

extern "C" int fa_combine_launch(CombineParams c, void* stream) {
  using namespace fa;
  if (!c.out_partial || !c.lse_partial || !c.out) return fail(FA_ERR_ARG, "fa_combine_launch: null pointer");
  if (c.nsplit <= 0 || c.B < 0 || c.S < 0 || c.H < 0 || c.D <= 0) return fail(FA_ERR_ARG, "fa_combine_launch: bad shape");
  if ((long long)c.B * c.S * c.H == 0) return FA_OK;
  if ((long long)c.B * c.S * c.H * ((c.D + 63) / 64) / 4 >= 0x7FFFFFFFLL) return fail(FA_ERR_ARG, "fa_combine_launch: too many rows");
  hipStream_t st = (hipStream_t)stream;
  switch (c.in_dtype) {
    case FA_F16: return launch_in<_Float16>(c, st);
    case FA_BF16: return launch_in<__bf16>(c, st);
    case FA_F32: return launch_in<float>(c, st);
    default: return fail(FA_ERR_DTYPE, "fa_combine_launch: in dtype %d", c.in_dtype);
  }
}
