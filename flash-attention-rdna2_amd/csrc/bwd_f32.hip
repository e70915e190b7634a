// bwd_f32.hip — exact attention backward for gfx950 in fp32, atomic-free and deterministic.
//
// The reference runs fp32 through its backward's plain-output mode (kernels/backward.hip:126,
// 257, 344: MODE == BW_F32, fmaf products, D <= 224). Same FableBwdParams contract and math as the
// fp16/bf16 kernels of bwd.hip (P recomputed from the forward LSE; dS = P*(z*dP - D)*softcap'),
// the same two-kernel split in stream order, on v_mfma_f32_16x16x4_f32:
//
//  1. dQ kernel: a wave owns 16 queries; Q and dO live in registers as B operands (lane
//     (q, g) holds dims g*HD/4 + t). It writes D = rowsum(O*dO) for kernel 2, then streams K/V
//     tiles through LDS: S^T = K.Q^T and dP^T = V.dO^T put keys 4g..4g+3 of each 16-key block
//     in lane (q, g), so dS^T is already the B operand of dQ^T = K^T.dS^T, whose A operand is
//     one float per lane (K[4g + j][16db + q]).
//  2. dK/dV kernel: a wave owns 16 keys; K and V live in registers (at D = 256 two workgroups
//     split the dK/dV columns of a key block, each computing S and dP). It streams the Q/dO tiles
//     (with their LSE/D rows) of every q head sharing the kv head, in a fixed order:
//     S = Q.K^T and dP = dO.V^T put queries 4g..4g+3 of each 16-query block in lane (key, g),
//     the B operands of dV^T += dO^T.(z*P) and dK^T += Q^T.dS.
// Softcap uses tanhf (fp32 needs its accuracy). Kernel widths 64, 128 and 256 serve every head
// dim p.D that is a multiple of 8: 16-byte chunks past it are not loaded (zeros) and gradient
// columns past it are not stored.
#include "attn_device.hpp"
#include "bwd_common.hpp"
#include "status.hpp"

namespace fa {

__device__ __forceinline__ f32x4 mma16f32_b(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float quad_sum_b(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// log2-domain logit of one score and d(logit)/d(scale*q.k)
template <bool FEAT>
__device__ __forceinline__ float logit2_f32(const FableBwdParams& p, float s, float c_log2, float slope, float inv_cap,
                                            int q, int key, float& deriv) {
  deriv = 1.0f;
  if (!FEAT) return s * c_log2;
  float x = s * p.scale;
  if (p.softcap > 0.0f) {
    const float t = tanhf(x * inv_cap);
    x = p.softcap * t;
    deriv = 1.0f - t * t;
  }
  x += slope * (float)(key - q);
  return x * kLog2e;
}

template <int HD_, int BC_, int NW_, int WPE_>
struct F32BwdQCfg {
  static constexpr int HD = HD_, BC = BC_, NW = NW_, WPE = WPE_;
  static constexpr int NT = NW * 64;
  static constexpr int BQ = NW * 16;
  static constexpr int NKB = BC / 16;
  static constexpr int NQ = HD / 4;
  static constexpr int NDB = HD / 16;
  static constexpr int STR = HD + 4;
  static constexpr int TILE = BC * STR;
  static constexpr int CH = HD / 4;
  static constexpr int KJ = BC * CH / NT;
  static constexpr int RSTEP = NT / CH;
  static_assert(HD % 64 == 0 && BC % 16 == 0 && (BC * CH) % NT == 0 && NT % CH == 0, "shape");
};

template <class C, bool CAUSAL, bool FEAT, bool DROP>
__global__ __attribute__((amdgpu_flat_work_group_size(C::NT, C::NT),
                          amdgpu_waves_per_eu(C::WPE, C::WPE))) void
bwd_dq_f32_kernel(FableBwdParams p, int nqt) {
  __shared__ __attribute__((aligned(16))) float kl[2 * C::TILE];
  __shared__ __attribute__((aligned(16))) float vl[2 * C::TILE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, g = lane >> 4;

  const int w = xcd_group_remap(blockIdx.x, gridDim.x, nqt, p.gqa, kBwdUMajor);
  const int qti = w % nqt, zh = w / nqt;
  const int h = zh % p.Hq, b = zh / p.Hq;
  const int qt = CAUSAL ? (nqt - 1 - qti) : qti;
  const int kvh = h / p.gqa;
  const BwdSeq sq = bwd_seq(p, b);
  const int SQ = sq.SQ, SK = sq.SK, delta = SK - SQ, HDr = p.D;
  const int qb = qt * C::BQ;
  if (qb >= SQ) return;

  const float* Qg = (const float*)p.Q + (long long)b * p.qs.b + sq.qo * p.qs.s + (long long)h * p.qs.h;
  const float* dOg = (const float*)p.dO + (long long)b * p.dos.b + sq.qo * p.dos.s + (long long)h * p.dos.h;
  const float* Og = (const float*)p.O + (long long)b * p.os.b + sq.qo * p.os.s + (long long)h * p.os.h;
  const float* Kg = (const float*)p.K + (long long)b * p.ks.b + sq.ko * p.ks.s + (long long)kvh * p.ks.h;
  const float* Vg = (const float*)p.V + (long long)b * p.vs.b + sq.ko * p.vs.s + (long long)kvh * p.vs.h;
  float* dQg = (float*)p.dQ + (long long)b * p.dqs.b + sq.qo * p.dqs.s + (long long)h * p.dqs.h;
  const long long row0 = (long long)b * p.lse_sb + (long long)h * p.lse_sh + sq.qo;

  const int qw = qb + 16 * wave, qi = qw + c16;
  const bool wave_rows = qw < SQ;
  int bk0, bk1, wk0 = 0, wk1 = 0;
  key_range_b<CAUSAL, FEAT>(p, qb, min(qb + C::BQ, SQ) - 1, delta, SK, bk0, bk1);
  if (wave_rows) key_range_b<CAUSAL, FEAT>(p, qw, min(qw + 16, SQ) - 1, delta, SK, wk0, wk1);
  const int kstart = (bk0 / C::BC) * C::BC;
  const int ntiles = bk1 > bk0 ? (bk1 - kstart + C::BC - 1) / C::BC : 0;

  // Q, dO rows as B operands; D = rowsum(O*dO)
  float qreg[C::NQ], doreg[C::NQ];
  float dpart = 0.0f;
#pragma unroll
  for (int u = 0; u < C::NQ / 4; u++) {
    f32x4 a = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, d = a;
    const int c = g * C::NQ + 4 * u;
    if (qi < SQ && c < HDr) {
      a = *(const f32x4*)(Qg + (long long)qi * p.qs.s + c);
      d = *(const f32x4*)(dOg + (long long)qi * p.dos.s + c);
      const f32x4 o = *(const f32x4*)(Og + (long long)qi * p.os.s + c);
#pragma unroll
      for (int e = 0; e < 4; e++) dpart = fmaf(o[e], d[e], dpart);
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
      qreg[4 * u + e] = a[e];
      doreg[4 * u + e] = d[e];
    }
  }
  const float Di = quad_sum_b(dpart);
  float lse2 = INFINITY;  // rows past SQ and rows without visible keys contribute nothing
  if (qi < SQ) {
    const float l = p.lse[row0 + qi];
    lse2 = l == -INFINITY ? INFINITY : l * kLog2e;
    if (g == 0) p.dsum[row0 + qi] = Di;
  }
  const float c_log2 = p.scale * kLog2e;
  const float slope = (FEAT && p.alibi) ? p.alibi[h] : 0.0f;
  const float inv_cap = p.softcap > 0.0f ? 1.0f / p.softcap : 0.0f;

  f32x4 dqacc[C::NDB];
#pragma unroll
  for (int db = 0; db < C::NDB; db++) dqacc[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int lrow = tid / C::CH, lcol = 4 * (tid % C::CH);
  f32x4 ldk[C::KJ], ldv[C::KJ];
  auto gload = [&](int kb) {
#pragma unroll
    for (int j = 0; j < C::KJ; j++) {
      const int r = kb + lrow + j * C::RSTEP;
      ldk[j] = ldv[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (r < SK && lcol < HDr) {
        ldk[j] = *(const f32x4*)(Kg + (long long)r * p.ks.s + lcol);
        ldv[j] = *(const f32x4*)(Vg + (long long)r * p.vs.s + lcol);
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
      f32x4 s[C::NKB], dp[C::NKB];
#pragma unroll
      for (int bb = 0; bb < C::NKB; bb++) s[bb] = dp[bb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      const int ao = st * C::TILE + c16 * C::STR + g * C::NQ;
#pragma unroll
      for (int u = 0; u < C::NQ / 4; u++)
#pragma unroll
        for (int bb = 0; bb < C::NKB; bb++) {
          const f32x4 a = *(const f32x4*)(kl + ao + bb * 16 * C::STR + 4 * u);
          const f32x4 v = *(const f32x4*)(vl + ao + bb * 16 * C::STR + 4 * u);
#pragma unroll
          for (int e = 0; e < 4; e++) {
            s[bb] = mma16f32_b(a[e], qreg[4 * u + e], s[bb]);
            dp[bb] = mma16f32_b(v[e], doreg[4 * u + e], dp[bb]);
          }
        }
      // s[bb][j]: key kb + 16bb + 4g + j, query qi
      const bool edge = FEAT || (CAUSAL && kb + C::BC - 1 > qw + delta) || kb + C::BC > SK;
#pragma unroll
      for (int bb = 0; bb < C::NKB; bb++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int key = kb + 16 * bb + 4 * g + j;
          float deriv;
          const float x = logit2_f32<FEAT>(p, s[bb][j], c_log2, slope, inv_cap, qi, key, deriv);
          float pr = exp2_fast(x - lse2);
          if (edge && !visible_b<CAUSAL, FEAT>(p, qi, key, delta, SQ, SK)) pr = 0.0f;
          const float z = DROP ? dropout_z(p.drop_seed, ((uint64_t)h * SQ + qi) * SK + key, p.dropout_p, p.keep_scale)
                               : 1.0f;
          s[bb][j] = pr * (z * dp[bb][j] - Di) * deriv;  // dS^T (backward.hip:170-176)
        }
      // dQ^T += K^T . dS^T over key pairs 16bb + 4g + j
      const float* kp = kl + st * C::TILE + 4 * g * C::STR + c16;
#pragma unroll
      for (int bb = 0; bb < C::NKB; bb++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float* row = kp + (16 * bb + j) * C::STR;
#pragma unroll
          for (int db = 0; db < C::NDB; db++) dqacc[db] = mma16f32_b(row[16 * db], s[bb][j], dqacc[db]);
        }
    }
    if (t + 1 < ntiles) lstore((t + 1) & 1);
    __syncthreads();
  }
  if (qi < SQ) {
    float* row = dQg + (long long)qi * p.dqs.s + 4 * g;
#pragma unroll
    for (int db = 0; db < C::NDB; db++)
      if (16 * db + 4 * g < HDr) *(f32x4*)(row + 16 * db) = dqacc[db] * p.scale;
  }
}

template <int HD_, int BQ_, int NW_, int WPE_, int DSPLIT_ = 1>
struct F32BwdKVCfg {
  static constexpr int HD = HD_, BQ = BQ_, NW = NW_, WPE = WPE_;
  static constexpr int DSPLIT = DSPLIT_;  // workgroups splitting the dK/dV columns of a key block
  static constexpr int NT = NW * 64;
  static constexpr int BK = NW * 16;   // keys per workgroup
  static constexpr int NQB = BQ / 16;  // 16-query blocks per tile
  static constexpr int NQ = HD / 4;
  static constexpr int NDB = HD / 16 / DSPLIT;  // 16-dim blocks of dK^T/dV^T owned here
  static constexpr int STR = HD + 4;
  static constexpr int TT = BQ * STR;  // floats per Q (or dO) tile
  static constexpr int STAGE = 2 * TT;
  static constexpr int CH = HD / 4;
  static constexpr int QJ = BQ * CH / NT;  // chunks each thread loads per Q (or dO) tile
  static constexpr int RSTEP = NT / CH;
  static_assert(HD % 64 == 0 && BQ % 16 == 0 && (BQ * CH) % NT == 0 && NT % CH == 0 && NT >= 2 * BQ, "shape");
};

template <class C, bool CAUSAL, bool FEAT, bool DROP>
__global__ __attribute__((amdgpu_flat_work_group_size(C::NT, C::NT),
                          amdgpu_waves_per_eu(C::WPE, C::WPE))) void
bwd_dkdv_f32_kernel(FableBwdParams p, int nkt) {
  __shared__ __attribute__((aligned(16))) float lds[2 * C::STAGE];
  __shared__ __attribute__((aligned(16))) float rowv[2][2][C::BQ];  // [stage][lse2 | D][q]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, g = lane >> 4;

  const int w = xcd_group_remap(blockIdx.x, gridDim.x, C::DSPLIT * nkt, 1, kBwdUMajor);
  const int dpass = w % C::DSPLIT, w2 = w / C::DSPLIT;
  const int dbase = dpass * C::NDB * 16;  // first dK/dV column owned here
  const int kt = w2 % nkt, zh = w2 / nkt;
  const int kvh = zh % p.Hk, b = zh / p.Hk;
  const BwdSeq sq = bwd_seq(p, b);
  const int SQ = sq.SQ, SK = sq.SK, delta = SK - SQ, HDr = p.D;
  const int kb0 = kt * C::BK;
  if (kb0 >= SK) return;

  const float* Kg = (const float*)p.K + (long long)b * p.ks.b + sq.ko * p.ks.s + (long long)kvh * p.ks.h;
  const float* Vg = (const float*)p.V + (long long)b * p.vs.b + sq.ko * p.vs.s + (long long)kvh * p.vs.h;
  const int kw = kb0 + 16 * wave, key = kw + c16;
  const bool wave_keys = kw < SK;

  float kreg[C::NQ], vreg[C::NQ];
#pragma unroll
  for (int u = 0; u < C::NQ / 4; u++) {
    f32x4 a = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, v = a;
    if (key < SK && g * C::NQ + 4 * u < HDr) {
      a = *(const f32x4*)(Kg + (long long)key * p.ks.s + g * C::NQ + 4 * u);
      v = *(const f32x4*)(Vg + (long long)key * p.vs.s + g * C::NQ + 4 * u);
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
      kreg[4 * u + e] = a[e];
      vreg[4 * u + e] = v[e];
    }
  }
  f32x4 dkacc[C::NDB], dvacc[C::NDB];
#pragma unroll
  for (int db = 0; db < C::NDB; db++) dkacc[db] = dvacc[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  int bq0, bq1, wq0 = 0, wq1 = 0;
  query_range_b<CAUSAL, FEAT>(p, kb0, min(kb0 + C::BK, SK) - 1, delta, SQ, bq0, bq1);
  if (wave_keys) query_range_b<CAUSAL, FEAT>(p, kw, min(kw + 16, SK) - 1, delta, SQ, wq0, wq1);
  const int qstart = (max(bq0, 0) / C::BQ) * C::BQ;
  const int ntq = bq1 > bq0 ? (bq1 - qstart + C::BQ - 1) / C::BQ : 0;
  const int total = ntq * p.gqa;
  const float c_log2 = p.scale * kLog2e;
  const float inv_cap = p.softcap > 0.0f ? 1.0f / p.softcap : 0.0f;

  const int lrow = tid / C::CH, lcol = 4 * (tid % C::CH);
  f32x4 ldq[C::QJ], ldd[C::QJ];
  float lraw = 0.0f;
  bool lok = false;
  auto gload = [&](int it) {
    const int hg = it / ntq, qt0 = qstart + (it % ntq) * C::BQ;
    const int h = kvh * p.gqa + hg;
    const float* Qh = (const float*)p.Q + (long long)b * p.qs.b + sq.qo * p.qs.s + (long long)h * p.qs.h;
    const float* dOh = (const float*)p.dO + (long long)b * p.dos.b + sq.qo * p.dos.s + (long long)h * p.dos.h;
#pragma unroll
    for (int j = 0; j < C::QJ; j++) {
      const int q = qt0 + lrow + j * C::RSTEP;
      ldq[j] = ldd[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (q < SQ && lcol < HDr) {
        ldq[j] = *(const f32x4*)(Qh + (long long)q * p.qs.s + lcol);
        ldd[j] = *(const f32x4*)(dOh + (long long)q * p.dos.s + lcol);
      }
    }
    if (tid < 2 * C::BQ) {
      const int q = qt0 + tid % C::BQ;
      lok = q < SQ;
      if (lok) {
        const long long ri = (long long)b * p.lse_sb + (long long)h * p.lse_sh + sq.qo + q;
        lraw = tid < C::BQ ? p.lse[ri] : p.dsum[ri];
      }
    }
  };
  auto lstore = [&](int stage) {
    float* base = lds + stage * C::STAGE;
#pragma unroll
    for (int j = 0; j < C::QJ; j++) {
      const int o = (lrow + j * C::RSTEP) * C::STR + lcol;
      *(f32x4*)(base + o) = ldq[j];
      *(f32x4*)(base + C::TT + o) = ldd[j];
    }
    if (tid < 2 * C::BQ) {
      // rows past SQ and rows without visible keys (LSE = -inf) get P = 0 through LSE = +inf
      const float lv = tid < C::BQ ? ((lok && lraw != -INFINITY) ? lraw * kLog2e : INFINITY)
                                   : (lok ? lraw : 0.0f);
      rowv[stage][tid / C::BQ][tid % C::BQ] = lv;
    }
  };

  if (total > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();
  for (int it = 0; it < total; it++) {
    const int stage = it & 1;
    const int hg = it / ntq, qt0 = qstart + (it % ntq) * C::BQ;
    if (it + 1 < total) gload(it + 1);
    if (wave_keys && qt0 < wq1 && qt0 + C::BQ > wq0) {
      const int h = kvh * p.gqa + hg;
      const float slope = (FEAT && p.alibi) ? p.alibi[h] : 0.0f;
      const float* qs = lds + stage * C::STAGE;
      const float* dos = qs + C::TT;
      // S = Q.K^T, dP = dO.V^T: s[qb][j] is query qt0 + 16qb + 4g + j, key `key`
      f32x4 s[C::NQB], dp[C::NQB];
#pragma unroll
      for (int qb = 0; qb < C::NQB; qb++) s[qb] = dp[qb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      const int ao = c16 * C::STR + g * C::NQ;
#pragma unroll
      for (int u = 0; u < C::NQ / 4; u++)
#pragma unroll
        for (int qb = 0; qb < C::NQB; qb++) {
          const f32x4 a = *(const f32x4*)(qs + ao + qb * 16 * C::STR + 4 * u);
          const f32x4 d = *(const f32x4*)(dos + ao + qb * 16 * C::STR + 4 * u);
#pragma unroll
          for (int e = 0; e < 4; e++) {
            s[qb] = mma16f32_b(a[e], kreg[4 * u + e], s[qb]);
            dp[qb] = mma16f32_b(d[e], vreg[4 * u + e], dp[qb]);
          }
          // keep the scheduler from hoisting every LDS read of the loop (register pressure)
          if ((u & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
      const bool edge = FEAT || (CAUSAL && kw + 15 > qt0 + delta) || qt0 + C::BQ > SQ || kw + 16 > SK;
#pragma unroll
      for (int qb = 0; qb < C::NQB; qb++) {
        const f32x4 l4 = *(const f32x4*)&rowv[stage][0][16 * qb + 4 * g];
        const f32x4 d4 = *(const f32x4*)&rowv[stage][1][16 * qb + 4 * g];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int q = qt0 + 16 * qb + 4 * g + j;
          float deriv;
          const float x = logit2_f32<FEAT>(p, s[qb][j], c_log2, slope, inv_cap, q, key, deriv);
          float pr = exp2_fast(x - l4[j]);
          if (edge && !visible_b<CAUSAL, FEAT>(p, q, key, delta, SQ, SK)) pr = 0.0f;
          const float z = DROP ? dropout_z(p.drop_seed, ((uint64_t)h * SQ + q) * SK + key, p.dropout_p, p.keep_scale)
                               : 1.0f;
          s[qb][j] = z * pr;                               // P (dropped)
          dp[qb][j] = pr * (z * dp[qb][j] - d4[j]) * deriv;  // dS
        }
      }
      // dV^T += dO^T . P, dK^T += Q^T . dS over query pairs 16qb + 4g + j
#pragma unroll
      for (int qb = 0; qb < C::NQB; qb++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int o = (16 * qb + 4 * g + j) * C::STR + dbase + c16;
#pragma unroll
          for (int db = 0; db < C::NDB; db++) {
            dvacc[db] = mma16f32_b(dos[o + 16 * db], s[qb][j], dvacc[db]);
            dkacc[db] = mma16f32_b(qs[o + 16 * db], dp[qb][j], dkacc[db]);
          }
        }
    }
    if (it + 1 < total) lstore((it + 1) & 1);
    __syncthreads();
  }
  if (key < SK) {
    float* dkrow = (float*)p.dK + (long long)b * p.dks.b + (sq.ko + key) * p.dks.s + (long long)kvh * p.dks.h + dbase + 4 * g;
    float* dvrow = (float*)p.dV + (long long)b * p.dvs.b + (sq.ko + key) * p.dvs.s + (long long)kvh * p.dvs.h + dbase + 4 * g;
#pragma unroll
    for (int db = 0; db < C::NDB; db++)
      if (dbase + 16 * db + 4 * g < HDr) {
        *(f32x4*)(dkrow + 16 * db) = dkacc[db] * p.scale;
        *(f32x4*)(dvrow + 16 * db) = dvacc[db];
      }
  }
}

template <class CQ, class CKV, bool CAUSAL, bool FEAT, bool DROP>
static int launch_bwd_f32_2(const FableBwdParams& p, hipStream_t st) {
  const int nqt = (p.SQ + CQ::BQ - 1) / CQ::BQ;
  const int nkt = (p.SK + CKV::BK - 1) / CKV::BK;
  const long long gq = (long long)nqt * p.Hq * p.B;
  const long long gkv = (long long)nkt * p.Hk * p.B * CKV::DSPLIT;
  if (gq > 0x7FFFFFFF || gkv > 0x7FFFFFFF) return fail(FA_ERR_ARG, "fable_attn_bwd: grid too large");
  if (gq > 0) {
    hipLaunchKernelGGL((bwd_dq_f32_kernel<CQ, CAUSAL, FEAT, DROP>), dim3((unsigned)gq), dim3(CQ::NT), 0, st, p, nqt);
    if (int rc = launch_status("fable_attn_bwd (dq, fp32)")) return rc;
  }
  if (gkv > 0) {
    hipLaunchKernelGGL((bwd_dkdv_f32_kernel<CKV, CAUSAL, FEAT, DROP>), dim3((unsigned)gkv), dim3(CKV::NT), 0, st, p, nkt);
    if (int rc = launch_status("fable_attn_bwd (dkdv, fp32)")) return rc;
  }
  return FA_OK;
}

template <class CQ, class CKV>
static int launch_bwd_f32_1(const FableBwdParams& p, hipStream_t st) {
  const bool feat = p.dropout || p.softcap > 0.0f || p.alibi != nullptr || p.win_left >= 0 ||
                    (p.win_right >= 0 && !(p.win_right == 0 && p.causal));
  if (p.dropout)
    return p.causal ? launch_bwd_f32_2<CQ, CKV, true, true, true>(p, st) : launch_bwd_f32_2<CQ, CKV, false, true, true>(p, st);
  if (p.causal)
    return feat ? launch_bwd_f32_2<CQ, CKV, true, true, false>(p, st) : launch_bwd_f32_2<CQ, CKV, true, false, false>(p, st);
  return feat ? launch_bwd_f32_2<CQ, CKV, false, true, false>(p, st) : launch_bwd_f32_2<CQ, CKV, false, false, false>(p, st);
}

// every head dim that is a multiple of 8 up to 256, in the kernels of width 64, 128 or 256
int launch_bwd_f32(const FableBwdParams& p, hipStream_t st) {
  if (p.D <= 0 || p.D > 256 || p.D % 8)
    return fail(FA_ERR_HEADDIM, "fable_attn_bwd: head_dim=%d has no fp32 kernel (multiples of 8 up to 256)", p.D);
  if (p.D <= 64) return launch_bwd_f32_1<F32BwdQCfg<64, 64, 8, 2>, F32BwdKVCfg<64, 64, 8, 2>>(p, st);
  if (p.D <= 128) return launch_bwd_f32_1<F32BwdQCfg<128, 64, 8, 2>, F32BwdKVCfg<128, 32, 8, 2>>(p, st);
  return launch_bwd_f32_1<F32BwdQCfg<256, 32, 4, 1>, F32BwdKVCfg<256, 32, 4, 1, 2>>(p, st);
}

}  // namespace fa
