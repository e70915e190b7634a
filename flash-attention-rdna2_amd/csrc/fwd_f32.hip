// fwd_f32.hip — exact attention forward for gfx950 in fp32 (inputs, outputs and arithmetic).
//
// The reference runs fp32 through a separate small-tile kernel (kernels/fa_forward.hip:317-400,
// dispatched at :440-447); same FableFwdParams contract and masking as the fp16/bf16 path. Here the
// products run on v_mfma_f32_16x16x4_f32 (fp32 operands, fp32 accumulate; the matrix cores'
// fp32 rate equals the VALU's, so fp32 stays on the MFMA pipe and leaves the VALU to softmax):
//
//  * a wave owns 16 queries (lane l: query l % 16, group g = l / 16); a workgroup of NW waves
//    covers 16*NW rows of one (sequence, head). Q lives in registers as the B operand of
//    S^T = K . Q^T: lane (q, g) holds Q[q][g*HD/4 + t], t = 0..HD/4-1, and the A operand reads
//    K[key][g*HD/4 + t] from LDS with the same contraction mapping.
//  * the S^T accumulator puts keys 4g..4g+3 of each 16-key block in lane (q, g): the lane's
//    probabilities are already the B operand of O^T = V^T . P^T over the key pairs (4g + j),
//    whose A operand is one float per lane, V[4g + j][16db + q], read conflict-free.
//  * online softmax in the log2 domain with the fp16 kernels' lazy rescale; the row max and
//    row sum reduce over the four lane groups. Softcap uses tanhf (fp32 needs its accuracy).
//  * K and V tiles are double-buffered in LDS with rows padded by 16 bytes; one barrier per
//    tile; tiles outside the mask are never loaded.
//  * kernel widths 64, 128 and 256: a head dim p.HD below the width (any multiple of 8) runs
//    with the columns past it zero. Each 16-byte chunk of a row lies wholly inside or outside
//    the head dim; outside ones are not loaded (zeros in registers and LDS, so they add nothing
//    to q.k, and the O columns they produce are not stored).
#include "attn_device.hpp"
#include "fwd_common.hpp"
#include "status.hpp"

namespace fa {

__device__ __forceinline__ f32x4 mma16f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// the other three lane groups of a 16-lane column
__device__ __forceinline__ float quad_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float quad_sum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

template <int HD_, int BC_, int NW_, int WPE_>
struct F32Cfg {
  static constexpr int HD = HD_, BC = BC_, NW = NW_, WPE = WPE_;
  static constexpr int NT = NW * 64;
  static constexpr int BR = NW * 16;     // query rows per workgroup
  static constexpr int NKB = BC / 16;    // 16-key blocks per tile
  static constexpr int NQ = HD / 4;      // contraction steps of S (and Q floats per lane)
  static constexpr int NDB = HD / 16;    // 16-dim blocks of O^T
  static constexpr int STR = HD + 4;     // LDS row stride (floats)
  static constexpr int TILE = BC * STR;
  static constexpr int CH = HD / 4;      // float4 chunks per row
  static constexpr int KJ = BC * CH / NT;  // chunks each thread loads per K (or V) tile
  static constexpr int RSTEP = NT / CH;
  static_assert(HD % 64 == 0 && BC % 16 == 0 && (BC * CH) % NT == 0 && NT % CH == 0, "shape");
};

template <class C, bool CAUSAL, bool FEAT, bool DROP>
__global__ __attribute__((amdgpu_flat_work_group_size(C::NT, C::NT),
                          amdgpu_waves_per_eu(C::WPE, C::WPE))) void
fwd_f32_kernel(FableFwdParams p, int nqt) {
  __shared__ __attribute__((aligned(16))) float kl[2 * C::TILE];
  __shared__ __attribute__((aligned(16))) float vl[2 * C::TILE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, g = lane >> 4;

  const int w = xcd_group_remap(blockIdx.x, gridDim.x, nqt, p.gqa, kFwdUMajor);
  const int qti = w % nqt, zh = w / nqt;
  const int h = zh % p.NH, z = zh / p.NH;
  const int qt = CAUSAL ? (nqt - 1 - qti) : qti;
  const int kvh = h / p.gqa;
  const SeqView sv = seq_view(p, z, h);
  const int SQ = sv.SQ, SK = sv.SK, HDr = p.HD;
  const int qb = qt * C::BR;
  if (qb >= SQ) return;
  const int delta = SK - SQ;

  const float* Qg = (const float*)p.Q + sv.q0 + (long long)h * p.sQ.h;
  const float* Kg = (const float*)p.K + sv.k0 + (long long)kvh * p.sK.h;
  const float* Vg = (const float*)p.V + sv.v0 + (long long)kvh * p.sV.h;
  float* Og = (float*)p.O + sv.o0 + (long long)h * p.sO.h;

  int bk0, bk1;
  key_range<CAUSAL, FEAT>(p, qb, min(qb + C::BR, SQ) - 1, delta, SK, bk0, bk1);
  const int qw = qb + wave * 16;
  const bool wave_rows = qw < SQ;
  int wk0 = 0, wk1 = 0;
  if (wave_rows) key_range<CAUSAL, FEAT>(p, qw, min(qw + 16, SQ) - 1, delta, SK, wk0, wk1);
  const int kstart = (bk0 / C::BC) * C::BC;
  const int ntiles = bk1 > bk0 ? (bk1 - kstart + C::BC - 1) / C::BC : 0;

  // Q: lane (q, g) holds Q[qw + q][g*HD/4 + t]
  const int qi = qw + c16;
  float qreg[C::NQ];
#pragma unroll
  for (int u = 0; u < C::NQ / 4; u++) {
    f32x4 v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (qi < SQ && g * C::NQ + 4 * u < HDr) v = *(const f32x4*)(Qg + (long long)qi * p.sQ.s + g * C::NQ + 4 * u);
#pragma unroll
    for (int e = 0; e < 4; e++) qreg[4 * u + e] = v[e];
  }

  f32x4 oacc[C::NDB];
#pragma unroll
  for (int db = 0; db < C::NDB; db++) oacc[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -INFINITY, l_run = 0.0f;
  const float c_log2 = p.scale * kLog2e;
  const float aslope2 = (FEAT && p.alibi_slopes) ? p.alibi_slopes[h] * kLog2e : 0.0f;
  const float inv_cap = p.softcap > 0.0f ? 1.0f / p.softcap : 0.0f;
  const float keep_scale = DROP ? 1.0f / (1.0f - p.dropout_p) : 1.0f;

  // tile loads: thread chunk j is row RSTEP*j + tid/CH, float4 column tid%CH
  const int lrow = tid / C::CH, lcol = 4 * (tid % C::CH);
  f32x4 ldk[C::KJ], ldv[C::KJ];
  auto gload = [&](int kb) {
#pragma unroll
    for (int j = 0; j < C::KJ; j++) {
      const int r = kb + lrow + j * C::RSTEP;
      ldk[j] = ldv[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (r < SK && lcol < HDr) {
        ldk[j] = *(const f32x4*)(Kg + (long long)r * p.sK.s + lcol);
        ldv[j] = *(const f32x4*)(Vg + (long long)r * p.sV.s + lcol);
      }
    }
  };
  auto lstore = [&](int st) {
#pragma unroll
    for (int j = 0; j < C::KJ; j++) {
      const int o = st * C::TILE + (lrow + j * C::RSTEP) * C::STR + lcol;
      *(f32x4*)(kl + o) = ldk[j];
      *(f32x4*)(vl + o) = ldv[j];
    }
  };

  if (ntiles > 0) {
    gload(kstart);
    lstore(0);
  }
  __syncthreads();
  for (int t = 0; t < ntiles; t++) {
    const int kb = kstart + t * C::BC, st = t & 1;
    if (t + 1 < ntiles) gload(kb + C::BC);
    if (wave_rows && kb < wk1 && kb + C::BC > wk0) {
      // S^T = K . Q^T: s[b] lane (q, g) holds key kb + 16b + 4g + j, query qi
      f32x4 s[C::NKB];
#pragma unroll
      for (int b = 0; b < C::NKB; b++) s[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      const float* kp = kl + st * C::TILE + c16 * C::STR + g * C::NQ;
#pragma unroll
      for (int u = 0; u < C::NQ / 4; u++)
#pragma unroll
        for (int b = 0; b < C::NKB; b++) {
          const f32x4 a = *(const f32x4*)(kp + b * 16 * C::STR + 4 * u);
#pragma unroll
          for (int e = 0; e < 4; e++) s[b] = mma16f32(a[e], qreg[4 * u + e], s[b]);
        }
      // softmax (log2 domain)
      const bool masked = FEAT || kb + C::BC > SK || (CAUSAL && kb + C::BC - 1 > qw + delta) || qw + 16 > SQ;
      float mx = -INFINITY;
#pragma unroll
      for (int b = 0; b < C::NKB; b++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int key = kb + 16 * b + 4 * g + j;
          float x;
          if (FEAT) {
            x = s[b][j] * p.scale;
            if (p.softcap > 0.0f) x = p.softcap * tanhf(x * inv_cap);
            x = x * kLog2e + aslope2 * (float)(key - qi);
          } else {
            x = s[b][j] * c_log2;
          }
          if (masked && !(qi < SQ && fwd_visible<CAUSAL, FEAT>(p, qi, key, delta, SK))) x = -INFINITY;
          s[b][j] = x;
          mx = fmaxf(mx, x);
        }
      mx = quad_max(mx);
      const float m_cand = fmaxf(m_run, mx);
      if (m_cand > m_run + kLazyMax) {  // uniform across the lane groups of a query
        const float corr = exp2_fast(m_run - m_cand);
#pragma unroll
        for (int db = 0; db < C::NDB; db++) oacc[db] *= corr;
        l_run *= corr;
        m_run = m_cand;
      }
      const float m_use = m_run == -INFINITY ? 0.0f : m_run;
#pragma unroll
      for (int b = 0; b < C::NKB; b++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float pe = exp2_fast(s[b][j] - m_use);
          l_run += pe;
          float pz = pe;
          if constexpr (DROP) {
            const int key = kb + 16 * b + 4 * g + j;
            pz *= dropout_z(p.philox_seed, ((uint64_t)h * SQ + qi) * SK + key, p.dropout_p, keep_scale);
          }
          s[b][j] = pz;
        }
      // O^T += V^T . P^T over key pairs 16b + 4g + j
      const float* vp = vl + st * C::TILE + 4 * g * C::STR + c16;
#pragma unroll
      for (int b = 0; b < C::NKB; b++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float* row = vp + (16 * b + j) * C::STR;
#pragma unroll
          for (int db = 0; db < C::NDB; db++) oacc[db] = mma16f32(row[16 * db], s[b][j], oacc[db]);
        }
    }
    if (t + 1 < ntiles) lstore((t + 1) & 1);
    __syncthreads();
  }

  // epilogue: lane (q, g) holds O^T[16db + 4g + j][q]
  const float l_tot = quad_sum(l_run);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (qi < SQ) {
    float* orow = Og + (long long)qi * p.sO.s + 4 * g;
#pragma unroll
    for (int db = 0; db < C::NDB; db++)
      if (16 * db + 4 * g < HDr) *(f32x4*)(orow + 16 * db) = oacc[db] * inv;
    if (p.LSE && g == 0) p.LSE[sv.lse0 + qi] = l_tot > 0.0f ? m_run * kLn2 + logf(l_tot) : -INFINITY;
  }
}

template <class C>
static int launch_f32(const FableFwdParams& p, hipStream_t st) {
  const bool drop = p.dropout_p > 0.0f;
  const bool feat = drop || p.softcap > 0.0f || p.alibi_slopes != nullptr || p.attn_chunk > 0 ||
                    p.win_left >= 0 || (p.win_right >= 0 && !(p.win_right == 0 && p.causal));
  const int nqt = (p.SQ + C::BR - 1) / C::BR;
  const long long nblk = (long long)nqt * p.NH * p.batch;
  if (nblk <= 0) return FA_OK;
  if (nblk > 0x7FFFFFFF) return fail(FA_ERR_ARG, "fable_attn_fwd: grid too large");
  const dim3 grid((unsigned)nblk), block(C::NT);
  if (p.causal) {
    if (drop) hipLaunchKernelGGL((fwd_f32_kernel<C, true, true, true>), grid, block, 0, st, p, nqt);
    else if (feat) hipLaunchKernelGGL((fwd_f32_kernel<C, true, true, false>), grid, block, 0, st, p, nqt);
    else hipLaunchKernelGGL((fwd_f32_kernel<C, true, false, false>), grid, block, 0, st, p, nqt);
  } else {
    if (drop) hipLaunchKernelGGL((fwd_f32_kernel<C, false, true, true>), grid, block, 0, st, p, nqt);
    else if (feat) hipLaunchKernelGGL((fwd_f32_kernel<C, false, true, false>), grid, block, 0, st, p, nqt);
    else hipLaunchKernelGGL((fwd_f32_kernel<C, false, false, false>), grid, block, 0, st, p, nqt);
  }
  return launch_status("fable_attn_fwd");
}

// every head dim that is a multiple of 8 up to 256, in the kernel of width 64, 128 or 256
int launch_fwd_f32(const FableFwdParams& p, hipStream_t st) {
  if (p.HD <= 0 || p.HD > 256 || p.HD % 8)
    return fail(FA_ERR_HEADDIM, "fable_attn_fwd: head_dim=%d has no fp32 kernel (multiples of 8 up to 256)", p.HD);
  if (p.HD <= 64) return launch_f32<F32Cfg<64, 64, 8, 2>>(p, st);
  if (p.HD <= 128) return launch_f32<F32Cfg<128, 64, 8, 2>>(p, st);
  return launch_f32<F32Cfg<256, 32, 8, 2>>(p, st);
}

}  // namespace fa
