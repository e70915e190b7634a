// bwd_kernel.hpp — the fp16/bf16 backward kernels and their launchers, templated on the
// kernel width; each bwd_dNN.hip instantiates one width, bwd.hip holds the entry points.
//
// Replaces the reference backward (kernels/backward.hip: fa_bwd_preprocess :86-96, fill_pd
// :109-202, fa_bwd_dkdv :205-295, fa_bwd_dq :298-387, launcher :508-521); same FableBwdParams
// contract and math (P recomputed from the forward LSE; dS = P*(dP - D)*softcap'), two kernels
// in stream order, no atomics, fixed reduction order => bitwise reproducible:
//
//  1. dQ kernel: a wave owns 32 queries, Q and dO live in registers as MFMA B operands. It first
//     computes D = rowsum(O*dO) for its rows (and writes it for kernel 2; no separate
//     preprocess launch), then streams K/V tiles through LDS: S^T = K.Q^T and dP^T = V.dO^T on
//     v_mfma_f32_32x32x16; dS^T stays in registers as the B operand of dQ^T = K^T.dS^T, with
//     K^T read from the row-major K tile by ds_read_b64_tr_b16.
//  2. dK/dV kernel: a wave owns 32 keys, K and V live in registers as B operands. It streams
//     Q/dO tiles (and their LSE/D rows) of every q head sharing the kv head, in a fixed order:
//     S = Q.K^T and dP = dO.V^T; P and dS stay in registers as B operands of
//     dV^T += dO^T.P and dK^T += Q^T.dS (dO^T/Q^T by transposing LDS reads).
// On that recomputing path S and dP are computed in both kernels (the price of no atomics, as in
// the reference). With a dS workspace (FableBwdParams.ds_ws, fp16/bf16, every kernel width) the order
// is instead: a rowsum kernel for D, the dK/dV kernel, which also stores each dS tile once, and
// a dQ kernel that forms dQ = dS.K from the stored tiles; every product is computed once, still
// without atomics and in a fixed order.
// Probabilities are evaluated as exp2(s*scale*log2e - LSE*log2e).
#pragma once

#include <utility>
#include "attn_device.hpp"
#include "bwd_common.hpp"
#include "status.hpp"

namespace fa {

// ------------------------------------------------------------------------------------ dQ
// Offset (elements) of row r, 16-byte chunk c of a row-major LDS tile read two ways: by rows
// (16 consecutive rows at one chunk) and transposed (ds_read_b64_tr_b16: 4 consecutive rows x
// 4 aligned chunks per half-wave). With 16 chunks per row the chunk is XORed with the row's two
// low bit-pairs swapped, a bijection over 16 consecutive rows that also sends the 4 rows of a
// transposed read to 4 different 64-byte bank groups; other widths XOR the chunk with the row
// modulo the largest power of two (up to 16) that divides the chunks per row, so the chunk stays
// in its aligned group and inside the row (a width of 96 has 12 chunks: groups of 4).
template <int HD>
__device__ __forceinline__ int bofs(int r, int c) {
  constexpr int DCH = HD / 8;
  constexpr int SW = (DCH & -DCH) < 16 ? (DCH & -DCH) : 16;
  if constexpr (DCH == 16)
    return r * HD + 8 * (c ^ (((r & 3) << 2) | ((r >> 2) & 3)));
  else
    return kofs(r, c, HD, SW);
}

template <int HD_, int BC_, int NW_, int WPE_, int DSPLIT_ = 1>
struct BwdQCfg {
  static constexpr int HD = HD_, BC = BC_, NW = NW_, WPE = WPE_, DSPLIT = DSPLIT_;
  static constexpr int NT = NW * 64;
  static constexpr int BQ = NW * 32;
  static constexpr int NB = BC / 32;
  static constexpr int NG = BC / 16;
  static constexpr int NDS = HD / 16;
  static constexpr int NDB = HD / 32 / DSPLIT;  // 32-row blocks of dQ^T owned by one pass
  static constexpr int DCH = HD / 8;
  static constexpr int KCH = BC * DCH;  // 16-byte chunks per K (or V) tile
  static constexpr int HALF = NT / 2;
  static constexpr int PER = KCH / HALF;
  static constexpr int KT = BC * HD;
  static constexpr int STAGE = 2 * KT;
  static_assert(KCH % HALF == 0, "loader split");
};

template <typename T, class C, bool CAUSAL, bool FEAT, bool DROP = false>
__global__ __attribute__((amdgpu_flat_work_group_size(C::NT, C::NT),
                          amdgpu_waves_per_eu(C::WPE, C::WPE))) void
bwd_dq_kernel(FableBwdParams p, int nqt) {
  using V8 = typename Dt<T>::V8;
  using V4 = typename Dt<T>::V4;
  __shared__ __attribute__((aligned(16))) T lds[2 * C::STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5, j16 = lane & 15, mh = (lane >> 4) & 1;

  const int w = xcd_group_remap(blockIdx.x, gridDim.x, C::DSPLIT * nqt, p.gqa, kBwdUMajor);
  const int dpass = w % C::DSPLIT, w2 = w / C::DSPLIT;  // head-dim slice of dQ owned here
  const int qti = w2 % nqt, zh = w2 / nqt;
  const int h = zh % p.Hq, b = zh / p.Hq;
  const int qt = CAUSAL ? (nqt - 1 - qti) : qti;
  const int kvh = h / p.gqa;
  const BwdSeq sq = bwd_seq(p, b);
  const int SQ = sq.SQ, SK = sq.SK, delta = SK - SQ;
  const int qb = qt * C::BQ;
  const int dbase = dpass * C::NDB * 32;
  if (qb >= SQ) return;

  const T* Qg = (const T*)p.Q + (long long)b * p.qs.b + sq.qo * p.qs.s + (long long)h * p.qs.h;
  const T* dOg = (const T*)p.dO + (long long)b * p.dos.b + sq.qo * p.dos.s + (long long)h * p.dos.h;
  const T* Og = (const T*)p.O + (long long)b * p.os.b + sq.qo * p.os.s + (long long)h * p.os.h;
  const T* Kg = (const T*)p.K + (long long)b * p.ks.b + sq.ko * p.ks.s + (long long)kvh * p.ks.h;
  const T* Vg = (const T*)p.V + (long long)b * p.vs.b + sq.ko * p.vs.s + (long long)kvh * p.vs.h;
  T* dQg = (T*)p.dQ + (long long)b * p.dqs.b + sq.qo * p.dqs.s + (long long)h * p.dqs.h;
  const long long row0 = (long long)b * p.lse_sb + (long long)h * p.lse_sh + sq.qo;

  const int qw = qb + 32 * wave, qi = qw + l32;
  const bool wave_rows = qw < SQ;
  int bk0, bk1, wk0 = 0, wk1 = 0;
  key_range_b<CAUSAL, FEAT>(p, qb, min(qb + C::BQ, SQ) - 1, delta, SK, bk0, bk1);
  if (wave_rows) key_range_b<CAUSAL, FEAT>(p, qw, min(qw + 32, SQ) - 1, delta, SK, wk0, wk1);
  const int kstart = (bk0 / C::BC) * C::BC;
  const int ntiles = bk1 > bk0 ? (bk1 - kstart + C::BC - 1) / C::BC : 0;

  // Q, dO rows as B operands; D = rowsum(O*dO). A head dim p.D below C::HD (a multiple of 8)
  // runs with zero columns p.D..C::HD-1 in every operand (they add nothing to any product) and
  // stores only the first p.D columns.
  const int HDr = p.D;
  V8 qreg[C::NDS], doreg[C::NDS];
  float dpart = 0.0f;
#pragma unroll
  for (int ds = 0; ds < C::NDS; ds++) {
    const int d0 = 16 * ds + 8 * hh;
    if (qi < SQ && d0 < HDr) {
      qreg[ds] = *(const V8*)(Qg + (long long)qi * p.qs.s + d0);
      doreg[ds] = *(const V8*)(dOg + (long long)qi * p.dos.s + d0);
      const V8 o = *(const V8*)(Og + (long long)qi * p.os.s + d0);
#pragma unroll
      for (int e = 0; e < 8; e++) dpart += (float)o[e] * (float)doreg[ds][e];
    } else {
      qreg[ds] = bitcast<V8>(u32x4{0, 0, 0, 0});
      doreg[ds] = qreg[ds];
    }
  }
  const float Di = half_sum(dpart);
  float lse2 = INFINITY;  // rows past SQ and rows without visible keys contribute nothing
  if (qi < SQ) {
    const float l = p.lse[row0 + qi];
    lse2 = l == -INFINITY ? INFINITY : l * kLog2e;
    if (hh == 0 && dpass == 0) p.dsum[row0 + qi] = Di;
  }
  const float c_log2 = p.scale * kLog2e;
  const float slope = (FEAT && p.alibi) ? p.alibi[h] : 0.0f;

  f32x16 dqacc[C::NDB];
#pragma unroll
  for (int db = 0; db < C::NDB; db++) dqacc[db] = f32x16{};

  // K/V tiles through buffer descriptors over rows kb..SK-1 (rows past SK read as zeros):
  // no per-lane condition, loop-invariant lane offsets, prefetch stays in flight.
  const bool kloader = wave < C::NW / 2;
  const int lt = kloader ? tid : tid - C::HALF;
  const long long sstride = kloader ? p.ks.s : p.vs.s;
  // chunks in the zero columns (>= p.D) load from kBufZero, which reads zeros
  int voff[C::PER];
#pragma unroll
  for (int j = 0; j < C::PER; j++) {
    const int idx = lt + j * C::HALF, r = idx / C::DCH, c = idx % C::DCH;
    voff[j] = 8 * c < HDr ? r * (int)(sstride * 2) + 16 * c : kBufZero;
  }
  u32x4 ld[C::PER];
  auto gload = [&](int kb) {
    const auto rs = kloader ? buf_rsrc(Kg + (long long)kb * p.ks.s, (long long)(SK - kb) * p.ks.s * 2)
                            : buf_rsrc(Vg + (long long)kb * p.vs.s, (long long)(SK - kb) * p.vs.s * 2);
#pragma unroll
    for (int j = 0; j < C::PER; j++) ld[j] = buf_load16(rs, voff[j]);
  };
  auto lstore = [&](int stage) {
    T* base = lds + stage * C::STAGE + (kloader ? 0 : C::KT);
#pragma unroll
    for (int j = 0; j < C::PER; j++) {
      const int idx = lt + j * C::HALF, r = idx / C::DCH, c = idx % C::DCH;
      *(u32x4*)(base + bofs<C::HD>(r, c)) = ld[j];
    }
  };

  if (ntiles > 0) {
    gload(kstart);
    lstore(0);
  }
  __syncthreads();
  for (int t = 0; t < ntiles; t++) {
    const int kb = kstart + t * C::BC;
    const int stage = t & 1;
    gload(kb + C::BC);  // past the last tile the descriptor is empty: zeros, no condition
    const bool active = wave_rows && kb < wk1 && kb + C::BC > wk0;
    if (active) {
      const T* ks = lds + stage * C::STAGE;
      const T* vs = ks + C::KT;
      f32x16 s[C::NB], dp[C::NB];
#pragma unroll
      for (int jb = 0; jb < C::NB; jb++) {
        s[jb] = f32x16{};
        dp[jb] = f32x16{};
      }
#pragma unroll
      for (int ds = 0; ds < C::NDS; ds++)
#pragma unroll
        for (int jb = 0; jb < C::NB; jb++) {
          const int off = bofs<C::HD>(jb * 32 + l32, 2 * ds + hh);
          s[jb] = Dt<T>::mma32(*(const V8*)(ks + off), qreg[ds], s[jb]);
          dp[jb] = Dt<T>::mma32(*(const V8*)(vs + off), doreg[ds], dp[jb]);
        }
      const bool edge = FEAT || (CAUSAL ? (kb + C::BC - 1 > qw + delta) : (kb + C::BC > SK));
      const int kq = kb + 4 * hh;
#pragma unroll
      for (int jb = 0; jb < C::NB; jb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int key = kq + jb * 32 + 8 * (r >> 2) + (r & 3);
          float deriv;
          const float x = bwd_logit2<FEAT>(p, s[jb][r], c_log2, slope, qi, key, deriv);
          float pr = exp2_fast(x - lse2);
          if (edge && !visible_b<CAUSAL, FEAT>(p, qi, key, delta, SQ, SK)) pr = 0.0f;
          const float z = DROP ? dropout_z(p.drop_seed, ((uint64_t)h * SQ + qi) * SK + key,
                                                          p.dropout_p, p.keep_scale)
                                              : 1.0f;
          s[jb][r] = pr * (z * dp[jb][r] - Di) * deriv;  // dS^T (backward.hip:170-176)
        }
      V8 pb[C::NG];
#pragma unroll
      for (int jb = 0; jb < C::NB; jb++)
#pragma unroll
        for (int sh = 0; sh < 2; sh++)
#pragma unroll
          for (int e = 0; e < 8; e++) pb[2 * jb + sh][e] = (T)s[jb][8 * sh + e];
      // dQ^T += K^T . dS^T: lane j16 of group (mh, hh) addresses key row 16g+8a+4hh+j16/4,
      // head-dim 32db+16mh+4*(j16%4)
#pragma unroll
      for (int db = 0; db < C::NDB; db++) {
        const int col = dbase + 32 * db + 16 * mh + 4 * (j16 & 3);
#pragma unroll
        for (int g = 0; g < C::NG; g++) {
          V4 part[2];
#pragma unroll
          for (int a = 0; a < 2; a++) {
            const int row = 16 * g + 8 * a + 4 * hh + (j16 >> 2);
            part[a] = lds_read_tr<T>(ks + bofs<C::HD>(row, col >> 3) + (col & 7));
          }
          V8 av;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            av[e] = part[0][e];
            av[4 + e] = part[1][e];
          }
          dqacc[db] = Dt<T>::mma32(av, pb[g], dqacc[db]);
        }
      }
    }
    lstore(stage ^ 1);
    __syncthreads();
  }
  {
    T* row = dQg + (long long)qi * p.dqs.s;
#pragma unroll
    for (int db = 0; db < C::NDB; db++)
      store_cblock<T>(row + dbase + 32 * db, dqacc[db], p.scale, hh, qi < SQ, HDr - dbase - 32 * db);
  }
}

// ---------------------------------------------------------------------------------- dK, dV
template <int HD_, int NW_, int WPE_, int DSPLIT_ = 1>
struct BwdKVCfg {
  static constexpr bool PAIR = false;
  static constexpr int HD = HD_, NW = NW_, WPE = WPE_, DSPLIT = DSPLIT_;
  static constexpr int NT = NW * 64;
  static constexpr int BQ = 32;         // queries per stage
  static constexpr int BK = NW * 32;    // keys per workgroup
  static constexpr int NDS = HD / 16;
  static constexpr int NDB = HD / 32 / DSPLIT;  // 32-row blocks of dK^T/dV^T owned by one pass
  static constexpr int DCH = HD / 8;
  static constexpr int TT = BQ * HD;    // halfs per Q (or dO) tile
  static constexpr int STAGE = 2 * TT;
  static constexpr int CH = 2 * BQ * DCH;  // chunks per stage (Q and dO)
  static constexpr int PER = (CH + NT - 1) / NT;
};

template <typename T, class C, bool CAUSAL, bool FEAT, bool DROP = false, bool DSW = false>
__global__ __attribute__((amdgpu_flat_work_group_size(C::NT, C::NT),
                          amdgpu_waves_per_eu(C::WPE, C::WPE))) void
bwd_dkdv_kernel(FableBwdParams p, int nkt) {
  using V8 = typename Dt<T>::V8;
  using V4 = typename Dt<T>::V4;
  __shared__ __attribute__((aligned(16))) T lds[2 * C::STAGE];
  __shared__ __attribute__((aligned(16))) float rowv[2][2][C::BQ];  // [stage][lse2 | D][q]
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5, j16 = lane & 15, mh = (lane >> 4) & 1;

  const int w = xcd_group_remap(blockIdx.x, gridDim.x, C::DSPLIT * nkt, 1, kBwdUMajor);
  const int dpass = w % C::DSPLIT, w2 = w / C::DSPLIT;  // head-dim slice of dK/dV owned here
  const int kt = w2 % nkt, zh = w2 / nkt;
  const int kvh = zh % p.Hk, b = zh / p.Hk;
  const int dbase = dpass * C::NDB * 32;
  const BwdSeq sq = bwd_seq(p, b);
  const int SQ = sq.SQ, SK = sq.SK, delta = SK - SQ;
  const int kb0 = kt * C::BK;
  if (kb0 >= SK) return;

  const T* Kg = (const T*)p.K + (long long)b * p.ks.b + sq.ko * p.ks.s + (long long)kvh * p.ks.h;
  const T* Vg = (const T*)p.V + (long long)b * p.vs.b + sq.ko * p.vs.s + (long long)kvh * p.vs.h;
  const int kw = kb0 + 32 * wave, key = kw + l32;
  const bool wave_keys = kw < SK;

  // a head dim p.D below C::HD runs with zero columns (see bwd_dq_kernel)
  const int HDr = p.D;
  V8 kreg[C::NDS], vreg[C::NDS];
#pragma unroll
  for (int ds = 0; ds < C::NDS; ds++) {
    const int d0 = 16 * ds + 8 * hh;
    if (key < SK && d0 < HDr) {
      kreg[ds] = *(const V8*)(Kg + (long long)key * p.ks.s + d0);
      vreg[ds] = *(const V8*)(Vg + (long long)key * p.vs.s + d0);
    } else {
      kreg[ds] = bitcast<V8>(u32x4{0, 0, 0, 0});
      vreg[ds] = kreg[ds];
    }
  }
  f32x16 dkacc[C::NDB], dvacc[C::NDB];
#pragma unroll
  for (int db = 0; db < C::NDB; db++) {
    dkacc[db] = f32x16{};
    dvacc[db] = f32x16{};
  }
  int bq0, bq1, wq0 = 0, wq1 = 0;
  query_range_b<CAUSAL, FEAT>(p, kb0, min(kb0 + C::BK, SK) - 1, delta, SQ, bq0, bq1);
  if (wave_keys) query_range_b<CAUSAL, FEAT>(p, kw, min(kw + 32, SK) - 1, delta, SQ, wq0, wq1);
  const int qstart = (max(bq0, 0) / C::BQ) * C::BQ;
  const int ntq = bq1 > bq0 ? (bq1 - qstart + C::BQ - 1) / C::BQ : 0;
  const int total = ntq * p.gqa;
  const float c_log2 = p.scale * kLog2e;
  // dS workspace (the head-dim pass 0 of each key block stores it): this wave's 32-key block
  // in the compacted layout, a cursor over the tiles in the loop's order (q tiles of a head,
  // then the next head), as in the pair kernel
  T* ds_cur = nullptr;
  long long ds_wrap = 0;
  if constexpr (DSW) {
    const int nkb = (p.SK + 31) >> 5;
    const int* tbl = (const int*)p.ds_ws;
    const int ds_T = tbl[nkb];
    ds_cur = ds_head_tiles<T>(p, b, kvh * p.gqa, ds_T) + (long long)(tbl[min(kw >> 5, nkb - 1)] + (qstart >> 5)) * 1024;
    ds_wrap = ((long long)ds_T - (ntq - 1)) * 1024;
  }

  // Q/dO tiles through buffer descriptors over rows qt0..SQ-1 (rows past SQ read as zeros);
  // each thread's first QJ chunk slots are Q, the rest dO. The LSE/D row values are loaded
  // unconditionally (clamped row) and turned into log2-domain LSE / D at store time.
  static_assert((C::BQ * C::DCH) % C::NT == 0, "Q/dO slot split");
  constexpr int QJ = C::BQ * C::DCH / C::NT;
  int voff[C::PER];  // zero-column chunks load from kBufZero, which reads zeros
#pragma unroll
  for (int j = 0; j < C::PER; j++) {
    const int ci = tid + (j < QJ ? j : j - QJ) * C::NT, r = ci / C::DCH, c = ci % C::DCH;
    voff[j] = 8 * c < HDr ? r * (int)((j < QJ ? p.qs.s : p.dos.s) * 2) + 16 * c : kBufZero;
  }
  u32x4 ld[C::PER];
  float lraw = 0.0f;
  bool lok = false;
  const int rsel = tid % (2 * C::BQ);  // row value slot: [0,BQ) LSE, [BQ,2BQ) D
  auto gload = [&](int it) {
    const int hg = min(it / ntq, p.gqa - 1), qt0 = qstart + (it % ntq) * C::BQ;
    const int h = kvh * p.gqa + hg;
    const long long rows = it < total ? (long long)(SQ - qt0) : 0;  // past the end: all zeros
    const auto rq = buf_rsrc((const T*)p.Q + (long long)b * p.qs.b + (long long)h * p.qs.h + (sq.qo + qt0) * p.qs.s,
                             rows * p.qs.s * 2);
    const auto rd = buf_rsrc((const T*)p.dO + (long long)b * p.dos.b + (long long)h * p.dos.h + (sq.qo + qt0) * p.dos.s,
                             rows * p.dos.s * 2);
#pragma unroll
    for (int j = 0; j < C::PER; j++) ld[j] = buf_load16(j < QJ ? rq : rd, voff[j]);
    const int q = qt0 + (rsel % C::BQ);
    lok = it < total && q < SQ;
    const long long ri = (long long)b * p.lse_sb + (long long)h * p.lse_sh + sq.qo + min(q, SQ - 1);
    lraw = rsel < C::BQ ? p.lse[ri] : p.dsum[ri];
  };
  auto lstore = [&](int stage) {
    T* base = lds + stage * C::STAGE;
#pragma unroll
    for (int j = 0; j < C::PER; j++) {
      const int ci = tid + (j < QJ ? j : j - QJ) * C::NT, r = ci / C::DCH, c = ci % C::DCH;
      *(u32x4*)(base + (j < QJ ? 0 : C::TT) + bofs<C::HD>(r, c)) = ld[j];
    }
    if (tid < 2 * C::BQ) {
      // rows past SQ and rows without visible keys (LSE = -inf) get P = 0 through LSE = +inf
      const float lv = rsel < C::BQ ? ((lok && lraw != -INFINITY) ? lraw * kLog2e : INFINITY)
                                    : (lok ? lraw : 0.0f);
      rowv[stage][rsel / C::BQ][rsel % C::BQ] = lv;
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
    gload(it + 1);  // past the last stage the descriptors are empty: zeros, no condition
    const bool active = wave_keys && qt0 < wq1 && qt0 + C::BQ > wq0;
    if (active) {
      const int h = kvh * p.gqa + hg;
      const float slope = (FEAT && p.alibi) ? p.alibi[h] : 0.0f;
      const T* qs = lds + stage * C::STAGE;
      const T* dos = qs + C::TT;
      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int ds = 0; ds < C::NDS; ds++) {
        const int off = bofs<C::HD>(l32, 2 * ds + hh);
        s = Dt<T>::mma32(*(const V8*)(qs + off), kreg[ds], s);
        dp = Dt<T>::mma32(*(const V8*)(dos + off), vreg[ds], dp);
      }
      // s[r] is query qt0 + 8*(r/4) + 4*hh + (r%4), key `key`
      const bool edge = FEAT || (CAUSAL ? (kw + 31 > qt0 + delta) : false) || qt0 + C::BQ > SQ || kw + 32 > SK;
      V8 pP[2], pS[2];
#pragma unroll
      for (int rq = 0; rq < 4; rq++) {
        const f32x4 l4 = *(const f32x4*)&rowv[stage][0][8 * rq + 4 * hh];
        const f32x4 d4 = *(const f32x4*)&rowv[stage][1][8 * rq + 4 * hh];
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const int r = 4 * rq + c, q = qt0 + 8 * rq + 4 * hh + c;
          float deriv;
          const float x = bwd_logit2<FEAT>(p, s[r], c_log2, slope, q, key, deriv);
          float pr = exp2_fast(x - l4[c]);
          if (edge && !visible_b<CAUSAL, FEAT>(p, q, key, delta, SQ, SK)) pr = 0.0f;
          const float z = DROP ? dropout_z(p.drop_seed, ((uint64_t)h * SQ + q) * SK + key,
                                                          p.dropout_p, p.keep_scale)
                                              : 1.0f;
          const float dsv = pr * (z * dp[r] - d4[c]) * deriv;
          pP[r >> 3][r & 7] = (T)(z * pr);
          pS[r >> 3][r & 7] = (T)dsv;
        }
      }
      if constexpr (DSW) {  // the dS tile (32 queries x this wave's 32 keys), streaming stores
        if (dpass == 0) {
          T* dst = ds_cur + 16 * l32 + 8 * hh;
          __builtin_nontemporal_store(pS[0], (V8*)dst);
          __builtin_nontemporal_store(pS[1], (V8*)(dst + 512));
        }
      }
      // dV^T += dO^T . P, dK^T += Q^T . dS (A operands by transposing reads of the tiles)
#pragma unroll
      for (int db = 0; db < C::NDB; db++) {
        const int col = dbase + 32 * db + 16 * mh + 4 * (j16 & 3);
#pragma unroll
        for (int st = 0; st < 2; st++) {
          V4 po[2], pq[2];
#pragma unroll
          for (int a = 0; a < 2; a++) {
            const int row = 16 * st + 8 * a + 4 * hh + (j16 >> 2);
            const int off = bofs<C::HD>(row, col >> 3) + (col & 7);
            po[a] = lds_read_tr<T>(dos + off);
            pq[a] = lds_read_tr<T>(qs + off);
          }
          V8 ao, aq;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            ao[e] = po[0][e];
            ao[4 + e] = po[1][e];
            aq[e] = pq[0][e];
            aq[4 + e] = pq[1][e];
          }
          dvacc[db] = Dt<T>::mma32(ao, pP[st], dvacc[db]);
          dkacc[db] = Dt<T>::mma32(aq, pS[st], dkacc[db]);
        }
      }
    }
    if constexpr (DSW) ds_cur += (it % ntq) + 1 == ntq ? ds_wrap : 1024;
    lstore(stage ^ 1);
    __syncthreads();
  }
  {
    T* krow = (T*)p.dK + (long long)b * p.dks.b + (long long)kvh * p.dks.h + (sq.ko + key) * p.dks.s;
    T* vrow = (T*)p.dV + (long long)b * p.dvs.b + (long long)kvh * p.dvs.h + (sq.ko + key) * p.dvs.s;
#pragma unroll
    for (int db = 0; db < C::NDB; db++) {
      store_cblock<T>(krow + dbase + 32 * db, dkacc[db], p.scale, hh, key < SK, HDr - dbase - 32 * db);
      store_cblock<T>(vrow + dbase + 32 * db, dvacc[db], 1.0f, hh, key < SK, HDr - dbase - 32 * db);
    }
  }
}

// f(integral_constant<int, I>) for I in the sequence, in order (compile-time register-set index)
template <int... I, typename F>
__device__ __forceinline__ void for_sets(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}

// ------------------------------------------------------------------- dK, dV with wave pairs
// Each 32-key block belongs to a pair of waves on the same SIMD slot pattern (wave w and w+NP):
// the S-wave holds K and computes S = Q K^T, P, and dV += dO^T P; the dP-wave holds V and, one
// tile behind, computes dP = dO V^T, dS = P deriv (dP - D) and dK += Q^T dS, taking P deriv
// (fp32) from the S-wave through LDS. No product is computed twice, and each wave needs about
// half the registers of a wave that owns both accumulators, so two waves fit per SIMD and
// one's VALU work overlaps the other's MFMAs. The Q/dO tiles sit in a 4-stage LDS ring (the
// S-wave reads tile t, the dP-wave tile t-1, tile t+1 is stored) and tiles t+2 .. t+NSET are in
// flight in the S-waves' registers; one barrier per tile.
// Query split of the pair dK/dV kernel on a grid of one round (dS-workspace path, dense or
// packed varlen batches): `n` workgroups per key block each take a contiguous run of its query
// tiles and write fp32 partial dK and dV rows, at row r = item * bk + (key within the block)
// (item: the key block's work item, sequence-head-major as the grid); bwd_split_merge_kernel
// sums them in share order and writes each row through the sequence's key offset.
struct BwdSplit {
  int n;           // shares per key block; 1: no split, the kernel writes dK and dV itself
  int nkt, bk;     // key blocks per (sequence, kv head) and keys per block of the launch
  long long rows;  // work items * bk
  float* part;     // [n][dK | dV][rows][p.D]
};

// WPE_: waves per SIMD (two; three at head dims 32 and 64, whose kernels fit 168 registers)
template <int HD_, int NP_, int NSET_, int WPE_ = 2>
struct BwdKVPCfg {
  static constexpr bool PAIR = true;
  static constexpr int HD = HD_, NP = NP_, NW = 2 * NP_, WPE = WPE_, DSPLIT = 1;
  static constexpr int NSET = NSET_;       // global-load prefetch distance (tiles), 2 or 3
  static_assert(NSET == 2 || NSET == 3, "prefetch distance");
  static constexpr int NT = NW * 64;
  static constexpr int BQ = 32;            // queries per stage
  static constexpr int BK = NP * 32;       // keys per workgroup
  static constexpr int NDS = HD / 16;
  static constexpr int NDB = HD / 32;
  static constexpr int DCH = HD / 8;
  static constexpr int TT = BQ * HD;       // elements per Q (or dO) tile
  static constexpr int STAGE = 2 * TT;
  static constexpr int CH = 2 * BQ * DCH;  // chunks per stage (Q and dO)
  // loader threads: the S-waves. The dP-waves load nothing and only store dS tiles: loads and
  // stores share one in-order completion counter, so a dP-wave that also loaded waited on
  // its earlier dS stores whenever it waited for a tile (C3 +3% with the S-waves loading)
  static constexpr int LT = NP * 64;
  static constexpr int PER = CH / LT;
  static constexpr int QJ = BQ * DCH / LT; // Q chunk slots per thread (the rest are dO)
  static_assert(CH % LT == 0 && (BQ * DCH) % LT == 0, "loader split");
};

// One work item of the pair kernel: key block w % nkt of K/V group w / nkt, query share `share`
// (LOOP: called from the persistent kernel's item loop)
template <typename T, class C, bool CAUSAL, bool FEAT, bool DROP, bool DSW, bool LOOP>
__device__ __forceinline__ void bwd_pair_item(const FableBwdParams& p, int nkt, const BwdSplit& sp, int w, int share) {
  using V8 = typename Dt<T>::V8;
  using V4 = typename Dt<T>::V4;
  __shared__ __attribute__((aligned(16))) T lds[4 * C::STAGE];
  __shared__ __attribute__((aligned(16))) float rowv[4][2][C::BQ];  // [stage][lse2 | D][q]
  // P deriv hand-over, [buffer][pair][rq][lane] x 4 floats: lane-contiguous 16-byte records
  __shared__ __attribute__((aligned(16))) f32x4 pdx[2][C::NP][4][64];
  // (in the item loop the thread index passes through an empty asm: the compiler otherwise
  // computes the per-lane offsets once, ahead of the loop, and holds them in registers the
  // steps need; D=128 then spilled)
  int tid_ = threadIdx.x;
  if constexpr (LOOP) asm volatile("" : "+v"(tid_));
  const int tid = tid_, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5, j16 = lane & 15, mh = (lane >> 4) & 1;
  const bool dpw = wave >= C::NP;  // dP-wave (holds V, accumulates dK)
  const int pair = dpw ? wave - C::NP : wave;

  const int kt = w % nkt, zh = w / nkt;
  const int kvh = zh % p.Hk, b = zh / p.Hk;
  const BwdSeq sq = bwd_seq(p, b);
  const int SQ = sq.SQ, SK = sq.SK, delta = SK - SQ;
  const int kb0 = kt * C::BK;
  if (kb0 >= SK) return;

  const int kw = kb0 + 32 * pair, key = kw + l32;
  const bool pair_keys = kw < SK;
  // dS workspace: this pair's key block in the compacted layout (table built by the dsum kernel)
  int ds_row = 0, ds_T = 0;
  if constexpr (DSW) {
    const int nkb = (p.SK + 31) >> 5;
    const int* tbl = (const int*)p.ds_ws;
    ds_row = tbl[min(kw >> 5, nkb - 1)];
    ds_T = tbl[nkb];
  }
  // B operand rows of this wave's product with the Q (or dO) tile: K for the S-wave, V for the
  // dP-wave; lane holds key `key`, head-dim 16*ds + 8*hh .. +7
  const T* Rg = dpw ? (const T*)p.V + (long long)b * p.vs.b + sq.ko * p.vs.s + (long long)kvh * p.vs.h
                    : (const T*)p.K + (long long)b * p.ks.b + sq.ko * p.ks.s + (long long)kvh * p.ks.h;
  const long long rstride = dpw ? p.vs.s : p.ks.s;
  // a head dim p.D below C::HD runs with zero columns (see bwd_dq_kernel)
  const int HDr = p.D;
  V8 kv[C::NDS];
#pragma unroll
  for (int ds = 0; ds < C::NDS; ds++)
    kv[ds] = key < SK && 16 * ds + 8 * hh < HDr ? *(const V8*)(Rg + (long long)key * rstride + 16 * ds + 8 * hh)
                                                : bitcast<V8>(u32x4{0, 0, 0, 0});
  f32x16 acc[C::NDB];  // dV^T (S-wave) or dK^T (dP-wave)
#pragma unroll
  for (int db = 0; db < C::NDB; db++) acc[db] = f32x16{};

  int bq0, bq1, wq0 = 0, wq1 = 0;
  query_range_b<CAUSAL, FEAT>(p, kb0, min(kb0 + C::BK, SK) - 1, delta, SQ, bq0, bq1);
  if (pair_keys) query_range_b<CAUSAL, FEAT>(p, kw, min(kw + 32, SK) - 1, delta, SQ, wq0, wq1);
  const int qstart = (max(bq0, 0) / C::BQ) * C::BQ;
  const int ntq = bq1 > bq0 ? (bq1 - qstart + C::BQ - 1) / C::BQ : 0;
  // this workgroup's steps: `total` tiles of the block's ntq*gqa, from tile it0 on (a query
  // split gives each share a contiguous run of them)
  int it0 = 0, total = ntq * p.gqa;
  if (sp.n > 1) {
    const int per = (total + sp.n - 1) / sp.n;
    it0 = min(share * per, total);
    total = min(it0 + per, total) - it0;
  }
  const int qi0 = ntq > 0 ? it0 % ntq : 0, hg0 = ntq > 0 ? it0 / ntq : 0;  // its first tile
  const float c_log2 = p.scale * kLog2e;

  // Q/dO tiles through buffer descriptors over rows qt0..SQ-1 (rows past SQ read as zeros);
  // each thread's first QJ chunk slots are Q, the rest dO. LSE/D row values are loaded
  // unconditionally (clamped row) and turned into log2-domain LSE / D at store time.
  // chunks in the zero columns (>= p.D) load from kBufZero, which reads zeros
  int voff[C::PER];
#pragma unroll
  for (int j = 0; j < C::PER; j++) {
    const int ci = tid + (j < C::QJ ? j : j - C::QJ) * C::LT, r = ci / C::DCH, c = ci % C::DCH;
    voff[j] = 8 * c < HDr ? r * (int)((j < C::QJ ? p.qs.s : p.dos.s) * 2) + 16 * c : kBufZero;
  }
  // NSET register sets: tile it+NSET is loaded while tile it+1 (loaded NSET-1 iterations
  // earlier) is stored, so every global load has NSET iterations to land
  constexpr int NSET = C::NSET;
  u32x4 ld[NSET][C::PER];
  float lraw[NSET];
  bool lok[NSET];
  const int rsel = tid % (2 * C::BQ);  // row value slot: [0,BQ) LSE, [BQ,2BQ) D
  // Tiles are loaded in order (tile g = head hg of the group, q tile qi), through a cursor
  // whose pointers, byte counts and row index advance by additions: the 64-bit products of a
  // from-scratch address cost ~90 scalar instructions per tile, which the scalar issue port
  // cannot hide. Past the last tile the cursor stays on it and the loads are emptied.
  const long long q_step = (long long)C::BQ * p.qs.s, do_step = (long long)C::BQ * p.dos.s;
  const long long q_wrap = p.qs.h - ntq * q_step, do_wrap = p.dos.h - ntq * do_step;
  const long long l_wrap = p.lse_sh - (long long)ntq * C::BQ;
  const long long q_left0 = (long long)(SQ - qstart) * p.qs.s * 2, do_left0 = (long long)(SQ - qstart) * p.dos.s * 2;
  const int hfirst = kvh * p.gqa + hg0;
  const T* g_q = (const T*)p.Q + (long long)b * p.qs.b + (long long)hfirst * p.qs.h + (sq.qo + qstart) * p.qs.s + qi0 * q_step;
  const T* g_do = (const T*)p.dO + (long long)b * p.dos.b + (long long)hfirst * p.dos.h + (sq.qo + qstart) * p.dos.s +
                  qi0 * do_step;
  long long g_l = (long long)b * p.lse_sb + (long long)hfirst * p.lse_sh + sq.qo + qstart + qi0 * C::BQ;
  long long g_qleft = q_left0 - 2 * qi0 * q_step, g_doleft = do_left0 - 2 * qi0 * do_step;
  int g_qi = qi0, g_t = 0;  // q tile index within the head, tile number (from it0)
  auto gload = [&](auto set) {
    constexpr int S = decltype(set)::value;
    const bool in = g_t < total;
    const auto rq = buf_rsrc(g_q, in ? g_qleft : 0);  // past the end: all zeros
    const auto rd = buf_rsrc(g_do, in ? g_doleft : 0);
#pragma unroll
    for (int j = 0; j < C::PER; j++) ld[S][j] = buf_load16(j < C::QJ ? rq : rd, voff[j]);
    const int qr = qstart + g_qi * C::BQ + (rsel % C::BQ);
    lok[S] = in && qr < SQ;
    // unconditional (clamped row; SQ >= 1 whenever the loop runs), so the memory waits of
    // the tile loads stay exact
    const long long ri = g_l + min(rsel % C::BQ, SQ - 1 - qstart - g_qi * C::BQ);
    lraw[S] = rsel < C::BQ ? p.lse[ri] : p.dsum[ri];
    if (g_t + 1 < total) {  // advance (uniform, scalar)
      if (++g_qi == ntq) {
        g_qi = 0;
        g_q += q_step + q_wrap;
        g_do += do_step + do_wrap;
        g_l += C::BQ + l_wrap;
        g_qleft = q_left0;
        g_doleft = do_left0;
      } else {
        g_q += q_step;
        g_do += do_step;
        g_l += C::BQ;
        g_qleft -= 2 * q_step;
        g_doleft -= 2 * do_step;
      }
    }
    ++g_t;
  };
  auto lstore = [&](auto set, int stage) {
    constexpr int S = decltype(set)::value;
    T* base = lds + stage * C::STAGE;
#pragma unroll
    for (int j = 0; j < C::PER; j++) {
      const int ci = tid + (j < C::QJ ? j : j - C::QJ) * C::LT, r = ci / C::DCH, c = ci % C::DCH;
      *(u32x4*)(base + (j < C::QJ ? 0 : C::TT) + bofs<C::HD>(r, c)) = ld[S][j];
    }
    if (tid < 2 * C::BQ) {
      // rows past SQ and rows without visible keys (LSE = -inf) get P = 0 through LSE = +inf
      const float lv = rsel < C::BQ ? ((lok[S] && lraw[S] != -INFINITY) ? lraw[S] * kLog2e : INFINITY)
                                    : (lok[S] ? lraw[S] : 0.0f);
      rowv[stage][rsel / C::BQ][rsel % C::BQ] = lv;
    }
  };
  auto active = [&](int qt0) { return pair_keys && qt0 < wq1 && qt0 + C::BQ > wq0; };
  // this wave's product of a tile with its B rows: S (S-wave, with Q) or dP (dP-wave, with
  // dO); x[r] is query qt0 + 8*(r/4) + 4*hh + (r%4), key `key`
  // (one accumulation chain: dependent MFMAs of one shape issue back to back, and a second
  // chain would cost 16 VALU adds per product). Both products read all their LDS operands
  // first: the scheduler otherwise put each read right before its product, through one
  // register set, so every product waited out a read; with the reads first the kernel takes
  // 6 fewer registers and runs as fast (the second wave of the SIMD hid those waits).
  auto rowprod = [&](const T* tile) {
    V8 a[C::NDS];
#pragma unroll
    for (int ds = 0; ds < C::NDS; ds++) a[ds] = *(const V8*)(tile + bofs<C::HD>(l32, 2 * ds + hh));
    __builtin_amdgcn_sched_barrier(0);
    f32x16 x = f32x16{};
#pragma unroll
    for (int ds = 0; ds < C::NDS; ds++) x = Dt<T>::mma32(a[ds], kv[ds], x);
    return x;
  };
  // acc^T += tile^T . B (A operand by transposing reads of the tile; B = P or dS)
  auto tprod = [&](const T* tile, const V8 (&bop)[2]) {
    V4 part[C::NDB][2][2];
#pragma unroll
    for (int db = 0; db < C::NDB; db++) {
      const int col = 32 * db + 16 * mh + 4 * (j16 & 3);
#pragma unroll
      for (int sq = 0; sq < 2; sq++)
#pragma unroll
        for (int a = 0; a < 2; a++) {
          const int row = 16 * sq + 8 * a + 4 * hh + (j16 >> 2);
          part[db][sq][a] = lds_read_tr<T>(tile + bofs<C::HD>(row, col >> 3) + (col & 7));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int db = 0; db < C::NDB; db++) {
#pragma unroll
      for (int sq = 0; sq < 2; sq++) {
        V8 av;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          av[e] = part[db][sq][0][e];
          av[4 + e] = part[db][sq][1][e];
        }
        acc[db] = Dt<T>::mma32(av, bop[sq], acc[db]);
      }
    }
  };

  // 4-stage ring (a power of two keeps the stage index cheap; three would do): the S-wave
  // reads tile it (stage it%4), the dP-wave tile it-1, tile it+1 is stored into the stage tile
  // it-3 used; tiles it+2 .. it+NSET are in flight in registers.
  // Each role runs its own loop of straight-line steps: a step whose tile this pair does not
  // see still multiplies, with exact zeros for its P (or dS) operand, so the accumulators never
  // sit behind a branch (which made the compiler copy them at every join). The zeros need no
  // select: a tile of the range that the pair does not see is masked by the edge test, a step
  // past the last tile has LSE = +inf (P = 0), and the dP-wave's dS = P deriv (dP - D) inherits
  // the zero. The ring, the LSE/D rows and the hand-over buffer start zeroed, so the first
  // dP-wave step (tile -1) and every masked step multiply finite values.
  {
    T* z = lds + 8 * tid;
#pragma unroll
    for (int i = 0; i < 4 * C::STAGE / (8 * C::NT); i++) *(u32x4*)(z + 8 * i * C::NT) = u32x4{0u, 0u, 0u, 0u};
    static_assert(4 * C::STAGE % (8 * C::NT) == 0, "ring zeroing split");
    for (int i = tid; i < (int)(sizeof(rowv) / 4); i += C::NT) (&rowv[0][0][0])[i] = 0.0f;
    for (int i = tid; i < (int)(sizeof(pdx) / 16); i += C::NT) (&pdx[0][0][0][0])[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  __syncthreads();  // zeroed before the first tile is stored
  if (total > 0 && !dpw) {
    gload(std::integral_constant<int, 0>{});
    lstore(std::integral_constant<int, 0>{}, 0);
    gload(std::integral_constant<int, 1>{});
    if constexpr (NSET > 2) gload(std::integral_constant<int, 2>{});
  }
  __syncthreads();
  // the tile a role works on: head hg of the group, q tile qi (advanced once per tile)
  int w_qi = qi0, w_hg = hg0;
  auto w_next = [&]() {
    if (++w_qi == ntq) {
      w_qi = 0;
      w_hg = min(w_hg + 1, p.gqa - 1);
    }
  };
  // S-wave step `it` (set S holds tile it, stored an iteration ago): S, P, dV += dO^T . P
  auto s_step = [&](auto set, int it) {
    constexpr int S = decltype(set)::value;
    gload(set);
    const int st = it & 3, hg = w_hg, qt0 = qstart + w_qi * C::BQ;
    w_next();
    const float slope = (FEAT && p.alibi) ? p.alibi[kvh * p.gqa + hg] : 0.0f;
    const T* qs = lds + st * C::STAGE;
    const f32x16 sv = rowprod(qs);
    const bool edge = FEAT || (CAUSAL && kw + 31 > qt0 + delta) || qt0 + C::BQ > SQ || kw + 32 > SK;
    // probabilities; on an edge tile (one uniform branch, no per-score branches) the scores a
    // query does not see are zeroed
    float pr[16], dv[16];
#pragma unroll
    for (int rq = 0; rq < 4; rq++) {
      const f32x4 l4 = *(const f32x4*)&rowv[st][0][8 * rq + 4 * hh];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int r = 4 * rq + c, q = qt0 + 8 * rq + 4 * hh + c;
        const float x = bwd_logit2<FEAT>(p, sv[r], c_log2, slope, q, key, dv[r]);
        pr[r] = exp2_fast(x - l4[c]);
      }
    }
    if (edge) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int q = qt0 + 8 * (r >> 2) + 4 * hh + (r & 3);
        pr[r] = visible_b<CAUSAL, FEAT>(p, q, key, delta, SQ, SK) ? pr[r] : 0.0f;
      }
    }
    V8 pP[2];
#pragma unroll
    for (int rq = 0; rq < 4; rq++) {
      f32x4 pd4;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int r = 4 * rq + c, q = qt0 + 8 * rq + 4 * hh + c;
        const float z = DROP ? dropout_z(p.drop_seed, ((uint64_t)(kvh * p.gqa + hg) * SQ + q) * SK + key,
                                         p.dropout_p, p.keep_scale)
                             : 1.0f;
        pP[r >> 3][r & 7] = (T)(z * pr[r]);
        // p * deriv >= 0; a dropped score hands it over negated, so the dP-wave knows z
        pd4[c] = z == 0.0f ? -(pr[r] * dv[r]) : pr[r] * dv[r];
      }
      pdx[it & 1][pair][rq][lane] = pd4;
    }
    tprod(qs + C::TT, pP);  // dV^T += dO^T . P
    lstore(std::integral_constant<int, (S + 1) % NSET>{}, (it + 1) & 3);  // tile it+1
    __syncthreads();
  };
  // dP-wave step `it`: tile t = it-1 (a step behind the S-wave): dP, dS; dK += Q^T . dS of
  // tile t-1 (the dS of the step before). Both waves of a SIMD start a step with matrix-core
  // work after the barrier; deferring the dK product puts the dP-wave's two products first and
  // its dS VALU work last, beside the S-wave's dV product, instead of both waves running
  // their VALU work at once. The Q tile of t-1 is still in its stage: the stage is refilled
  // with tile t+3 at the end of step it+1.
  V8 pS[2] = {bitcast<V8>(u32x4{0, 0, 0, 0}), bitcast<V8>(u32x4{0, 0, 0, 0})};
  // dS workspace cursor (wave-uniform): the tile of step t, advanced like the tile order (the
  // next q tile of the head, or the first of the next head); rebuilding the address every step
  // from 64-bit products cost ~25 scalar instructions
  T* ds_cur = nullptr;
  long long ds_wrap = 0;
  if constexpr (DSW) {
    ds_cur = ds_head_tiles<T>(p, b, hfirst, ds_T) + (long long)(ds_row + (qstart >> 5) + qi0) * 1024;
    ds_wrap = ((long long)ds_T - (ntq - 1)) * 1024;
  }
  auto d_step = [&](auto set, int it) {
    const int t = it - 1;
    const int qt0 = qstart + w_qi * C::BQ;
    const bool act = t >= 0 && t < total && active(qt0);
    T* const ds_tile = ds_cur;
    if (t >= 0) {
      if constexpr (DSW) ds_cur += w_qi + 1 == ntq ? ds_wrap : 1024;
      w_next();
    }
    const int st = t & 3;
    const T* qs = lds + st * C::STAGE;
    tprod(lds + ((t - 1) & 3) * C::STAGE, pS);  // dK^T += Q^T . dS (tile t-1)
    const f32x16 dpv = rowprod(qs + C::TT);
#pragma unroll
    for (int rq = 0; rq < 4; rq++) {
      const f32x4 d4 = *(const f32x4*)&rowv[st][1][8 * rq + 4 * hh];
      const f32x4 pd4 = pdx[t & 1][pair][rq][lane];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int r = 4 * rq + c;
        float ds;
        if constexpr (DROP) {  // dS = p (z dP - D) deriv (backward.hip:170-176)
          const float z = pd4[c] < 0.0f ? 0.0f : p.keep_scale;
          ds = fabsf(pd4[c]) * (z * dpv[r] - d4[c]);
        } else {
          ds = pd4[c] * (dpv[r] - d4[c]);
        }
        pS[r >> 3][r & 7] = (T)ds;
      }
    }
    if constexpr (DSW) {  // dS tile (32 queries x this pair's 32 keys) to the workspace
      if (act) {
        T* dst = ds_tile + 16 * l32 + 8 * hh;
        // streaming stores: the tiles are read once, by the dQ kernel, and must not push the
        // Q/dO tiles this kernel re-reads out of L2
        __builtin_nontemporal_store(pS[0], (V8*)dst);
        __builtin_nontemporal_store(pS[1], (V8*)(dst + 512));
      }
    }
    __syncthreads();
  };
  // steps 0 .. total (the dP-wave's last tile is total-1), rounded up to whole register-set
  // rounds; both roles run the same number of barriers
  if (total > 0) {
    if (dpw) {
      int it = 0;
      for (; it <= total; it += NSET)
        for_sets(std::make_integer_sequence<int, NSET>{}, [&](auto set) { d_step(set, it + decltype(set)::value); });
      tprod(lds + ((it - 2) & 3) * C::STAGE, pS);  // the last step's tile (it-1 was the last step)
    } else {
      for (int it = 0; it <= total; it += NSET)
        for_sets(std::make_integer_sequence<int, NSET>{}, [&](auto set) { s_step(set, it + decltype(set)::value); });
    }
  }
  const float sc = dpw ? p.scale : 1.0f;
  if (sp.n > 1) {  // a query split: this share's fp32 partial dK (or dV) rows
    const long long r = ((long long)(2 * share + (dpw ? 0 : 1)) * sp.rows + (long long)w * C::BK + (key - kb0)) * HDr;
#pragma unroll
    for (int db = 0; db < C::NDB; db++) store_cblock_f32(sp.part + r + 32 * db, acc[db], sc, hh, key < SK, HDr - 32 * db);
    return;
  }
  {
    T* row = dpw ? (T*)p.dK + (long long)b * p.dks.b + (long long)kvh * p.dks.h + (sq.ko + key) * p.dks.s
                 : (T*)p.dV + (long long)b * p.dvs.b + (long long)kvh * p.dvs.h + (sq.ko + key) * p.dvs.s;
#pragma unroll
    for (int db = 0; db < C::NDB; db++) store_cblock<T>(row + 32 * db, acc[db], sc, hh, key < SK, HDr - 32 * db);
  }
}

// Workgroups of the persistent pair kernel per workgroup slot of a CU: the CUs of an MI355X
// (256 in 8 XCDs)
constexpr int kBwdPersistWG = 256, kBwdXcd = 8;
// The persistent kernel runs grids of at least two rounds of workgroups whose longest item has
// at most kBwdPersistMaxSteps query-tile steps (sequences of up to 512 queries, or packed
// batches whose longest sequence is), when the batch is packed (sequences of unequal length:
// many items are short or empty) or, for a dense batch, causal with one workgroup per CU:
// B=64 S=512 H=32 D=128 causal 1.14x, packed 1..512-row sequences 1.32x (D=128) and 1..256-row
// ones 1.17x (D=64, three workgroups per CU). Dense grids of three workgroups per CU (D=64
// S=512 0.97-0.99x), dense non-causal ones (0.97-0.98x) and longer items (S=1024 0.98x, S=4096
// 0.96x: the fixed item lists balance less well than the dispatcher once its gaps no longer
// matter) keep the dispatched grid.
constexpr long long kBwdPersistMinItems = 512;
constexpr long long kBwdPersistMaxSteps = 16;
// The pair kernel. Dispatched (PERSIST false): one work item per workgroup, the grid
// share-major (every key block's first share, then the second, ...) and mapped to items by
// xcd_group_remap. Persistent (PERSIST true, no query split): a fixed grid of kBwdPersistWG
// workgroups per CU slot, each running a fixed list of items. Workgroup L of the dispatched
// grid runs on XCD L % 8 (round-robin dispatch), so XCD x's share of the work is the items of
// L = x + 8 j, j = 0, 1, ..., in that order; the R persistent workgroups of XCD x (blockIdx % 8
// = x) take j in a snake, workgroup r the j = r, 2R-1-r, 2R+r, 4R-1-r, ...: a causal grid's
// key blocks alternate heavy and light along j, and the snake pairs them. Short items (a few
// query tiles per key block) otherwise leave CUs idle between workgroups: at B=64 S=512 H=32
// D=128 the dispatched grid's CUs sat idle a median 7 us between 24 us workgroups.
template <typename T, class C, bool CAUSAL, bool FEAT, bool DROP = false, bool DSW = false, bool PERSIST = false>
__global__ __attribute__((amdgpu_flat_work_group_size(C::NT, C::NT),
                          amdgpu_waves_per_eu(C::WPE, C::WPE))) void
bwd_dkdv_pair_kernel(FableBwdParams p, int nkt, BwdSplit sp) {
  if constexpr (!PERSIST) {
    const int nitems = gridDim.x / sp.n;
    const int share = blockIdx.x / nitems;
    bwd_pair_item<T, C, CAUSAL, FEAT, DROP, DSW, false>(p, nkt, sp, xcd_group_remap(blockIdx.x - share * nitems, nitems, nkt, 1, kBwdUMajor),
                                                        share);
  } else {
    const int x = blockIdx.x % kBwdXcd, r = blockIdx.x / kBwdXcd, R = gridDim.x / kBwdXcd;
    const long long nitems = (long long)nkt * p.Hk * p.B;
    for (long long k = 0;; k++) {
      const long long j = k * R + ((k & 1) ? R - 1 - r : r);
      const long long L = j * kBwdXcd + x;  // increases with k
      if (L >= nitems) break;
      if (k > 0) __syncthreads();  // the last item's LDS reads done before this one zeroes it
      bwd_pair_item<T, C, CAUSAL, FEAT, DROP, DSW, true>(p, nkt, sp, xcd_group_remap((int)L, (int)nitems, nkt, 1, kBwdUMajor), 0);
    }
  }
}

// most shares a key block's query tiles split into (bwd_split_count)
constexpr int kBwdMaxSplit = 8;

// Sum of the query-split partials of the pair dK/dV kernel, shares in order (bitwise
// reproducible): one thread per (row, 4 head dims), rows (dK | dV, work item, key in block);
// keys past the sequence's end are left alone.
template <typename T, int NMAX>
__global__ __launch_bounds__(256) void bwd_split_merge_kernel(FableBwdParams p, BwdSplit sp) {
  const int ch = p.D / 4;
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= 2 * sp.rows * ch) return;
  const long long r = gid / ch;
  const int c = (int)(gid - r * ch);
  const int which = (int)(r / sp.rows);  // 0 dK, 1 dV
  const long long rr = r - which * sp.rows;
  const int w = (int)(rr / sp.bk), kt = w % sp.nkt, zh = w / sp.nkt;
  const int kvh = zh % p.Hk, b = zh / p.Hk;
  const BwdSeq sq = bwd_seq(p, b);
  const int key = kt * sp.bk + (int)(rr - (long long)w * sp.bk);
  if (key >= sq.SK) return;
  // every share's partial loaded before any is added (NMAX >= n; indices past the last share
  // repeat it and are not added): one memory latency instead of one per share
  f32x4 v[NMAX];
#pragma unroll
  for (int k = 0; k < NMAX; k++)
    v[k] = *(const f32x4*)(sp.part + ((long long)(2 * min(k, sp.n - 1) + which) * sp.rows + rr) * p.D + 4 * c);
  f32x4 acc = v[0];
#pragma unroll
  for (int k = 1; k < NMAX; k++)
    if (k < sp.n) acc += v[k];
  typename Dt<T>::V4 o;
#pragma unroll
  for (int e = 0; e < 4; e++) o[e] = (T)acc[e];
  T* dst = which == 0 ? (T*)p.dK + (long long)b * p.dks.b + (long long)kvh * p.dks.h + (sq.ko + key) * p.dks.s
                      : (T*)p.dV + (long long)b * p.dvs.b + (long long)kvh * p.dvs.h + (sq.ko + key) * p.dvs.s;
  *(u32x2*)(dst + 4 * c) = __builtin_bit_cast(u32x2, o);
}

// ------------------------------------------------------------ dQ from a dS workspace
// D = rowsum(O*dO) for every (b, h, q) row: HD/8 lanes per row, one 16-byte chunk each, and
// DSUM_RPT rows per lane whose loads are all in flight before the first sum (one row per lane
// left each workgroup waiting on a single load pair: C3 33 us for 134 MB).
constexpr int DSUM_RPT = 4;
template <typename T, int HD>
__global__ __launch_bounds__(256) void bwd_dsum_kernel(FableBwdParams p, int rblocks) {
  constexpr int LPR = HD / 8, RPB = 256 / LPR;
  using V8 = typename Dt<T>::V8;
  const int tid = threadIdx.x;
  const int rb = blockIdx.x % rblocks, zh = blockIdx.x / rblocks;
  const int h = zh % p.Hq, b = zh / p.Hq;
  if (blockIdx.x == 0) ds_build_table(p);  // the dS workspace's tile table, for the next kernels
  const BwdSeq sq = bwd_seq(p, b);
  // (a packed batch's grid covers its longest sequence: the blocks past a shorter one's end)
  if (sq.SQ <= 0 || rb * DSUM_RPT * RPB >= sq.SQ) return;
  const int c = tid % LPR;
  // chunks past a head dim p.D below HD read the row's first chunk and add nothing
  const bool cok = 8 * c < p.D;
  const T* ob = (const T*)p.O + (long long)b * p.os.b + (long long)h * p.os.h + (cok ? 8 * c : 0);
  const T* db = (const T*)p.dO + (long long)b * p.dos.b + (long long)h * p.dos.h + (cok ? 8 * c : 0);
  V8 o[DSUM_RPT], d[DSUM_RPT];
#pragma unroll
  for (int r = 0; r < DSUM_RPT; r++) {
    // rows past the end load the last row (in bounds) and are not stored
    const int q = min((rb * DSUM_RPT + r) * RPB + tid / LPR, sq.SQ - 1);
    o[r] = *(const V8*)(ob + (sq.qo + q) * p.os.s);
    d[r] = *(const V8*)(db + (sq.qo + q) * p.dos.s);
  }
#pragma unroll
  for (int r = 0; r < DSUM_RPT; r++) {
    const int q = (rb * DSUM_RPT + r) * RPB + tid / LPR;
    float acc = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) acc += (float)o[r][e] * (float)d[r][e];
    acc = cok ? acc : 0.0f;
#pragma unroll
    for (int m = LPR / 2; m > 0; m >>= 1) acc += __shfl_xor(acc, m);
    if (c == 0 && q < sq.SQ) p.dsum[(long long)b * p.lse_sb + (long long)h * p.lse_sh + sq.qo + q] = acc;
  }
}

template <int HD_, int NW_, int WPE_, int NS_, int BC_ = 64>
struct BwdDsQCfg {
  static constexpr int HD = HD_, NW = NW_, WPE = WPE_;
  static constexpr int NS = NS_;       // dS register sets: dS loaded NS-1 tiles ahead (K one)
  static constexpr int NT = NW * 64;
  static constexpr int BQ = NW * 32;   // queries per workgroup (32 per wave)
  static constexpr int BC = BC_;       // keys per K tile
  static constexpr int NKB = BC / 32;  // workspace key blocks per K tile
  static constexpr int NDB = HD / 32;  // 32-row blocks of dQ^T
  static constexpr int DCH = HD / 8;
  static constexpr int KCH = BC * DCH;
  static constexpr int PER = KCH / NT;
  static constexpr int KT = BC * HD;
  static constexpr int DSTR = 32;      // LDS row of a wave's dS block: 32 query slots (64 B)
  static_assert(KCH % NT == 0, "loader split");
};

// Element offset of (key row r, query slot n) in a wave's dS block: 64-byte rows of four 16-byte
// chunks, chunk n/8 stored at position (n/8) ^ (2*(r.bit1 ^ r.bit3) + r.bit2). The 16-byte
// writes (one row per lane) then reach distinct 16-byte bank slots within every 8 consecutive
// rows of one parity (bits 1, 2 map one to one) and within every 16 consecutive rows (bits 2, 3
// map one to one for each r mod 4), and the transposing reads of rows R..R+3 find rows R and
// R+2 (and R+1, R+3) on disjoint chunk pairs. SQ_LDS_BANK_CONFLICT of the dQ kernel on C3: 8.9e6
// cycles per dispatch with the earlier 2*r.bit2 + r.bit3 (its 16-byte writes conflicted two
// ways), 0 with this one; the time did not change (the writes cost ~3% of the backward by
// their LDS latency, not by conflicts: a timing copy without them ran 1.03x faster).
__device__ __forceinline__ int dsl_ofs(int r, int n) {
  return r * 32 + 8 * ((n >> 3) ^ (2 * (((r >> 1) ^ (r >> 3)) & 1) + ((r >> 2) & 1))) + (n & 7);
}

// dQ^T = K^T . dS^T over the dS tiles the pair kernel wrote for this wave's 32 queries. K tiles
// are double-buffered through LDS and read transposed (A operand); each is loaded into
// registers one step ahead and stored to LDS at the end of that step. dS tiles are loaded NS-1
// K tiles ahead (16-byte loads into NS rotating register sets); the dS chunks are staged in
// a per-wave LDS block with keys as rows and read back transposed, so each lane gets 8 keys of
// one query slot (B operand), in the contraction order of the K^T reads. Column n of the product
// is query slot n, i.e. query ds_slot_query(n). A (key block, query block) tile is read exactly
// when the pair kernel wrote it: the same query range of the key block, intersected with the
// wave's rows.
template <typename T, class C, bool CAUSAL, bool FEAT>
__global__ __attribute__((amdgpu_flat_work_group_size(C::NT, C::NT),
                          amdgpu_waves_per_eu(C::WPE, C::WPE))) void
bwd_dq_ds_kernel(FableBwdParams p, int nqt) {
  using V8 = typename Dt<T>::V8;
  using V4 = typename Dt<T>::V4;
  __shared__ __attribute__((aligned(16))) T lds[2 * C::KT];
  __shared__ __attribute__((aligned(16))) T dsl[C::NW][C::BC * C::DSTR];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5, j16 = lane & 15, mh = (lane >> 4) & 1;

  const int w = xcd_group_remap(blockIdx.x, gridDim.x, nqt, p.gqa, kBwdUMajor);
  const int qti = w % nqt, zh = w / nqt;
  const int h = zh % p.Hq, b = zh / p.Hq;
  const int qt = CAUSAL ? (nqt - 1 - qti) : qti;
  const int kvh = h / p.gqa;
  const BwdSeq sq = bwd_seq(p, b);
  const int SQ = sq.SQ, SK = sq.SK, delta = SK - SQ;
  const int qb = qt * C::BQ;
  if (qb >= SQ) return;

  const T* Kg = (const T*)p.K + (long long)b * p.ks.b + sq.ko * p.ks.s + (long long)kvh * p.ks.h;
  T* dQg = (T*)p.dQ + (long long)b * p.dqs.b + sq.qo * p.dqs.s + (long long)h * p.dqs.h;
  const int qw = qb + 32 * wave;
  const bool wave_rows = qw < SQ;
  int bk0, bk1;
  key_range_b<CAUSAL, FEAT>(p, qb, min(qb + C::BQ, SQ) - 1, delta, SK, bk0, bk1);
  const int kstart = (bk0 / C::BC) * C::BC;
  const int ntiles = bk1 > bk0 ? (bk1 - kstart + C::BC - 1) / C::BC : 0;

  // the pair kernel wrote tile (key block kb32, this wave's query block) iff it is inside the
  // key range, and the queries that see some key of the block meet the wave's rows
  auto written = [&](int kb32) {
    const int k0 = 32 * kb32;
    if (!wave_rows || k0 >= SK) return false;
    int q0, q1;
    query_range_b<CAUSAL, FEAT>(p, k0, min(k0 + 32, SK) - 1, delta, SQ, q0, q1);
    return qw < q1 && qw + 32 > q0;
  };
  // Loads are issued unconditionally (from a clamped tile address when the tile was not written;
  // such data is never used), so the memory waits stay exact and the prefetch stays in flight.
  // Tiles of the compacted layout (bwd_common.hpp): key block kb's row starts at tbl[kb], and
  // tbl[kb+1] = tbl[kb] + qb1(kb) - qb0(kb+1), so after one table read per workgroup the row
  // advances by scalar integer steps. A tile that was not written is read from a clamped index
  // inside this head's tiles (its data is never used).
  const int nkb = (p.SK + 31) >> 5;
  const int* tbl = (const int*)p.ds_ws;
  const int ds_T = tbl[nkb];
  const int dlane = (16 * l32 + 8 * hh) * (int)sizeof(T);
  constexpr int NS = C::NS;
  V8 dsr[NS][2 * C::NKB];  // [register set][key block jb, query half sh] chunks of one K tile
  bool dact[NS][C::NKB];
  int d_kb32 = kstart >> 5;
  // tile (key block d_kb32, this wave's query block): a wave-uniform cursor that advances by
  // the next row's offset, qb1(kb) - qb0(kb + 1) tiles, from the span of the current key block
  // (kept) and of the next. It points outside the head's tiles where the tile was not written;
  // such a tile is never read (below).
  const T* ds_cur = ds_head_tiles<T>(p, b, h, ds_T) + (long long)(tbl[min(d_kb32, nkb - 1)] + (qw >> 5)) * 1024;
  int sp1;  // qb1 of key block d_kb32
  {
    int sp0;
    ds_span_k<CAUSAL, FEAT>(p, min(d_kb32, nkb - 1), sp0, sp1);
  }
  auto dsload = [&](auto set, int t) {
    constexpr int S = decltype(set)::value;
#pragma unroll
    for (int jb = 0; jb < C::NKB; jb++) {
      const int kb = d_kb32 + jb;
      dact[S][jb] = t < ntiles && written(kb);
      // a tile that is not used (past the last one, or not written for this wave's rows on
      // the diagonal) loads through an empty descriptor: zeros, and no memory traffic (its
      // clamped reads had been ~14% of the dS bytes); its address is never dereferenced
      const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(ds_cur), (short)0, dact[S][jb] ? 2048 : 0, 0x00020000);
      dsr[S][2 * jb] = bitcast<V8>(buf_load16_nt(rs, dlane));
      dsr[S][2 * jb + 1] = bitcast<V8>(buf_load16_nt(rs, dlane + 1024));
      if (kb + 1 < nkb) {  // the next key block's row (past the last one: stay)
        int n0, n1;
        ds_span_k<CAUSAL, FEAT>(p, kb + 1, n0, n1);
        ds_cur += (long long)(sp1 - n0) * 1024;
        sp1 = n1;
      }
    }
    d_kb32 += C::NKB;
  };

  // a head dim p.D below C::HD runs with zero columns (see bwd_dq_kernel): their chunks load
  // from kBufZero, which reads zeros
  const int HDr = p.D;
  int voff[C::PER];
#pragma unroll
  for (int j = 0; j < C::PER; j++) {
    const int idx = tid + j * C::NT, r = idx / C::DCH, c = idx % C::DCH;
    voff[j] = 8 * c < HDr ? r * (int)(p.ks.s * 2) + 16 * c : kBufZero;
  }
  u32x4 ld[C::PER];
  const T* k_ptr = Kg + (long long)kstart * p.ks.s;
  long long k_left = (long long)(SK - kstart) * p.ks.s * 2;
  const long long k_step = (long long)C::BC * p.ks.s;
  auto gload = [&]() {
    const auto rs = buf_rsrc(k_ptr, k_left);  // past the last tile the descriptor is empty: zeros
#pragma unroll
    for (int j = 0; j < C::PER; j++) ld[j] = buf_load16(rs, voff[j]);
    k_ptr += k_step;
    k_left -= 2 * k_step;
  };
  auto lstore = [&](int stage) {
    T* base = lds + stage * C::KT;
#pragma unroll
    for (int j = 0; j < C::PER; j++) {
      const int idx = tid + j * C::NT, r = idx / C::DCH, c = idx % C::DCH;
      *(u32x4*)(base + bofs<C::HD>(r, c)) = ld[j];
    }
  };

  f32x16 dqacc[C::NDB];
#pragma unroll
  for (int db = 0; db < C::NDB; db++) dqacc[db] = f32x16{};
  T* my = dsl[wave];
  // tile t: K in LDS stage t&1, dS in register set S; K tile t+1 is loaded into registers and
  // goes to LDS stage (t+1)&1 at the end of the step, dS tile t+NS-1 is loaded into set
  // (S+NS-1)%NS
  auto step = [&](auto set, int t) {
    constexpr int S = decltype(set)::value;
    gload();
    dsload(std::integral_constant<int, (S + NS - 1) % NS>{}, t + NS - 1);
    // this wave's dS chunks (key rows 32jb + l32, query slots 16sh + 8hh ..) into its LDS block
#pragma unroll
    for (int jb = 0; jb < C::NKB; jb++)
#pragma unroll
      for (int sh = 0; sh < 2; sh++) *(V8*)(my + dsl_ofs(32 * jb + l32, 16 * sh + 8 * hh)) = dsr[S][2 * jb + sh];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const T* ks = lds + (t & 1) * C::KT;
#pragma unroll
    for (int jb = 0; jb < C::NKB; jb++) {
      if (!dact[S][jb]) continue;
#pragma unroll
      for (int g2 = 0; g2 < 2; g2++) {
        const int g = 2 * jb + g2;
        // B: keys 16g + 8(e/4) + 4hh + e%4 (e = 0..7) of query slot l32
        V8 bop;
        {
          const int row = 16 * g + 4 * hh + (j16 >> 2), col = 16 * mh + 4 * (j16 & 3);
          const V4 lo = lds_read_tr<T>(my + dsl_ofs(row, col)), hi = lds_read_tr<T>(my + dsl_ofs(row + 8, col));
#pragma unroll
          for (int e = 0; e < 4; e++) {
            bop[e] = lo[e];
            bop[4 + e] = hi[e];
          }
        }
#pragma unroll
        for (int db = 0; db < C::NDB; db++) {
          // A: K^T, head-dim 32db + l32, the same keys
          const int col = 32 * db + 16 * mh + 4 * (j16 & 3);
          V4 part[2];
#pragma unroll
          for (int a = 0; a < 2; a++) {
            const int row = 16 * g + 8 * a + 4 * hh + (j16 >> 2);
            part[a] = lds_read_tr<T>(ks + bofs<C::HD>(row, col >> 3) + (col & 7));
          }
          V8 av;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            av[e] = part[0][e];
            av[4 + e] = part[1][e];
          }
          dqacc[db] = Dt<T>::mma32(av, bop, dqacc[db]);
        }
      }
    }
    lstore((t + 1) & 1);
    __syncthreads();
  };

  if (ntiles > 0) {
    gload();
    for_sets(std::make_integer_sequence<int, NS - 1>{}, [&](auto set) { dsload(set, decltype(set)::value); });
    lstore(0);
  }
  __syncthreads();
  // whole groups of NS steps (a step past the last tile multiplies nothing): no branch around a
  // step, so the waits for each register set's loads are exact
  for (int t = 0; t < ntiles; t += NS)
    for_sets(std::make_integer_sequence<int, NS>{}, [&](auto set) { step(set, t + decltype(set)::value); });
  const int qi = qw + ds_slot_query(l32);
  {
    T* row = dQg + (long long)qi * p.dqs.s;
#pragma unroll
    for (int db = 0; db < C::NDB; db++) store_cblock<T>(row + 32 * db, dqacc[db], p.scale, hh, qi < SQ, HDr - 32 * db);
  }
}

// dS register sets of the dQ-from-dS kernel
#ifndef DSQ_SETS
#define DSQ_SETS 2
#endif
constexpr int kDsqSets = DSQ_SETS;
// bytes of the compacted dS workspace (bwd_common.hpp): the table, then every (b, h)'s tiles
// keys per workgroup of the pair dK/dV kernel at each width (the BwdKVPCfg of bwd_d32.hip ..
// bwd_d128.hip; 0: the width has no pair kernel); the launcher checks it against the config
inline int bwd_pair_bk(int D) {
  const int w = bwd_width(D);
  return w > 128 ? 0 : (w == 128 ? 128 : 64);
}
// Shares per key block of the pair kernel's query split. A causal grid of at most one
// workgroup per CU runs as long as its longest key block (the first sees every query): halving
// the blocks of at least 32 query-tile steps pays for the fp32 partials and their merge. A
// grid filling at most half the CUs splits up to one workgroup per CU, at least 16 steps each.
inline int bwd_split_count(const FableBwdParams& p) {
  const int bk = bwd_pair_bk(p.D);
  if (bk == 0 || p.B <= 0 || p.Hk <= 0 || p.SQ <= 0 || p.SK <= 0) return 1;
  const long long gkv = (long long)((p.SK + bk - 1) / bk) * p.Hk * p.B;
  const long long steps = (long long)((p.SQ + 31) / 32) * p.gqa;  // the most a key block takes
  if (gkv > 256) return 1;
  if (2 * gkv > 256) return (p.causal && steps >= 32) ? 2 : 1;
  long long n = 256 / gkv;
  n = n < steps / 16 ? n : steps / 16;
  n = n < kBwdMaxSplit ? n : kBwdMaxSplit;
  return n >= 2 ? (int)n : 1;
}
// partial rows of the split: every key block's work item times its keys
inline long long bwd_split_rows(const FableBwdParams& p) {
  const int bk = bwd_pair_bk(p.D);
  return bk > 0 ? (long long)((p.SK + bk - 1) / bk) * p.Hk * p.B * bk : 0;
}
inline long long ds_split_offset(const FableBwdParams& p, long long tiles) {
  return (ds_header_bytes((p.SK + 31) >> 5) + (long long)p.B * p.Hq * tiles * 2048 + 255) / 256 * 256;
}
// bytes of the compacted dS workspace: the table, every (b, h)'s tiles, and the pair kernel's
// split partials when it splits
inline long long ds_bytes(const FableBwdParams& p) {
  if (p.SQ <= 0 || p.SK <= 0) return 0;
  const long long t = ds_tiles_per_head(p);  // 0: no query sees any key, the recomputing path serves
  if (t <= 0) return 0;
  const int n = bwd_split_count(p);
  const long long part = n > 1 ? (long long)n * 2 * bwd_split_rows(p) * p.D * 4 : 0;
  return n > 1 ? ds_split_offset(p, t) + part : ds_header_bytes((p.SK + 31) >> 5) + (long long)p.B * p.Hq * t * 2048;
}

// backward through the dS workspace: D rows, then dK/dV (writing dS), then dQ = dS.K
template <typename T, class CKV, bool CAUSAL, bool FEAT, bool DROP>
static int launch_bwd_ds(const FableBwdParams& p, hipStream_t st, int nkt) {
  // up to 128 wide: 8 waves where a K tile's chunks split evenly over them (widths that are
  // multiples of 64); wider: 4 waves. Two waves per SIMD up to 192 wide; at 256 one (the dQ
  // accumulators of a 256-wide row take 128 registers, the kernel 268)
  constexpr bool kWide = CKV::HD > 128;
  using CD = BwdDsQCfg<CKV::HD, (!kWide && (CKV::HD / 8) % 8 == 0) ? 8 : 4, (CKV::HD > 192) ? 1 : 2, kDsqSets>;
  // the D-row kernel reduces over a power-of-two count of lanes per row (chunks past the head
  // dim add zero)
  constexpr int DW = CKV::HD <= 32 ? 32 : (CKV::HD <= 64 ? 64 : (CKV::HD <= 128 ? 128 : 256));
  constexpr int RPB = 256 / (DW / 8) * DSUM_RPT;  // rows per dsum workgroup
  const long long gd = (long long)((p.SQ + RPB - 1) / RPB) * p.Hq * p.B;
  // grids of fewer 8-wave workgroups than CUs run 4-wave ones (twice as many, half the rows)
  using CDS = BwdDsQCfg<CKV::HD, 4, CD::WPE, kDsqSets>;
  const int nqt = (p.SQ + CD::BQ - 1) / CD::BQ;
  const bool small = CD::NW == 8 && (long long)nqt * p.Hq * p.B < 256;
  const int nqts = (p.SQ + CDS::BQ - 1) / CDS::BQ;
  const long long gq = (long long)(small ? nqts : nqt) * p.Hq * p.B;
  const long long gkv = (long long)nkt * p.Hk * p.B * CKV::DSPLIT;
  if (gd > 0x7FFFFFFF || gq > 0x7FFFFFFF || gkv > 0x7FFFFFFF) return fail(FA_ERR_ARG, "fable_attn_bwd: grid too large");
  hipLaunchKernelGGL((bwd_dsum_kernel<T, DW>), dim3((unsigned)gd), dim3(256), 0, st, p, (p.SQ + RPB - 1) / RPB);
  if (int rc = launch_status("fable_attn_bwd (dsum)")) return rc;
  if constexpr (CKV::PAIR) {
    BwdSplit sp{1, nkt, CKV::BK, 0, nullptr};
    const int n = CKV::BK == bwd_pair_bk(p.D) ? bwd_split_count(p) : 1;
    if (n > 1 && (long long)p.D % 4 == 0) {
      const long long t = ds_tiles_per_head(p);
      const long long off = ds_split_offset(p, t);
      if (p.ds_ws_bytes >= off + (long long)n * 2 * bwd_split_rows(p) * p.D * 4)
        sp = BwdSplit{n, nkt, CKV::BK, bwd_split_rows(p), (float*)((char*)p.ds_ws + off)};
    }
    // workgroups of the config that fit one CU at once (its waves per SIMD over its waves per CU)
    constexpr int kPerCu = 4 * CKV::WPE / CKV::NW > 0 ? 4 * CKV::WPE / CKV::NW : 1;
    const long long item_steps = (long long)((p.SQ + 31) / 32) * p.gqa;  // the most an item takes
    const bool persist_shape = p.cu_q != nullptr || (CAUSAL && kPerCu == 1);
    if (sp.n == 1 && persist_shape && gkv >= kBwdPersistMinItems * kPerCu && item_steps <= kBwdPersistMaxSteps)
      hipLaunchKernelGGL((bwd_dkdv_pair_kernel<T, CKV, CAUSAL, FEAT, DROP, true, true>), dim3((unsigned)(kBwdPersistWG * kPerCu)),
                         dim3(CKV::NT), 0, st, p, nkt, sp);
    else
      hipLaunchKernelGGL((bwd_dkdv_pair_kernel<T, CKV, CAUSAL, FEAT, DROP, true>), dim3((unsigned)(gkv * sp.n)),
                         dim3(CKV::NT), 0, st, p, nkt, sp);
    if (int rc = launch_status("fable_attn_bwd (dkdv)")) return rc;
    if (sp.n > 1) {
      const long long items = 2 * sp.rows * (p.D / 4);
      const dim3 mg((unsigned)((items + 255) / 256));
      if (sp.n <= 2)
        hipLaunchKernelGGL((bwd_split_merge_kernel<T, 2>), mg, dim3(256), 0, st, p, sp);
      else if (sp.n <= 4)
        hipLaunchKernelGGL((bwd_split_merge_kernel<T, 4>), mg, dim3(256), 0, st, p, sp);
      else
        hipLaunchKernelGGL((bwd_split_merge_kernel<T, kBwdMaxSplit>), mg, dim3(256), 0, st, p, sp);
      if (int rc = launch_status("fable_attn_bwd (dkdv merge)")) return rc;
    }
  } else {
    hipLaunchKernelGGL((bwd_dkdv_kernel<T, CKV, CAUSAL, FEAT, DROP, true>), dim3((unsigned)gkv), dim3(CKV::NT), 0, st, p, nkt);
    if (int rc = launch_status("fable_attn_bwd (dkdv)")) return rc;
  }
  if constexpr (CD::NW == 8) {
    if (small) {
      hipLaunchKernelGGL((bwd_dq_ds_kernel<T, CDS, CAUSAL, FEAT>), dim3((unsigned)gq), dim3(CDS::NT), 0, st, p, nqts);
      return launch_status("fable_attn_bwd (dq)");
    }
  }
  hipLaunchKernelGGL((bwd_dq_ds_kernel<T, CD, CAUSAL, FEAT>), dim3((unsigned)gq), dim3(CD::NT), 0, st, p, nqt);
  return launch_status("fable_attn_bwd (dq)");
}

template <typename T, class CQ, class CKV, bool CAUSAL, bool FEAT, bool DROP = false>
static int launch_bwd2(const FableBwdParams& p, hipStream_t st) {
  const int nqt = (p.SQ + CQ::BQ - 1) / CQ::BQ;
  const int nkt = (p.SK + CKV::BK - 1) / CKV::BK;
  const long long gq = (long long)nqt * p.Hq * p.B * CQ::DSPLIT;
  const long long gkv = (long long)nkt * p.Hk * p.B * CKV::DSPLIT;
  if (gq > 0x7FFFFFFF || gkv > 0x7FFFFFFF) return fail(FA_ERR_ARG, "fable_attn_bwd: grid too large");
  {
    const long long need = ds_bytes(p);
    // (the tiles are moved with 16-byte accesses: an unaligned workspace is not used)
    if (p.ds_ws && ((uintptr_t)p.ds_ws & 15) == 0 && need > 0 && p.ds_ws_bytes >= need)
      return launch_bwd_ds<T, CKV, CAUSAL, FEAT, DROP>(p, st, nkt);
  }
  if (gq > 0) {
    hipLaunchKernelGGL((bwd_dq_kernel<T, CQ, CAUSAL, FEAT, DROP>), dim3((unsigned)gq), dim3(CQ::NT), 0, st, p, nqt);
    if (int rc = launch_status("fable_attn_bwd (dq)")) return rc;
  }
  if (gkv > 0) {
    if constexpr (CKV::PAIR)
      hipLaunchKernelGGL((bwd_dkdv_pair_kernel<T, CKV, CAUSAL, FEAT, DROP>), dim3((unsigned)gkv), dim3(CKV::NT), 0, st, p, nkt,
                         BwdSplit{1, nkt, CKV::BK, 0, nullptr});
    else
      hipLaunchKernelGGL((bwd_dkdv_kernel<T, CKV, CAUSAL, FEAT, DROP>), dim3((unsigned)gkv), dim3(CKV::NT), 0, st, p, nkt);
    if (int rc = launch_status("fable_attn_bwd (dkdv)")) return rc;
  }
  return FA_OK;
}

template <typename T, class CQ, class CKV>
static int launch_bwd(const FableBwdParams& p, hipStream_t st) {
  const bool feat = p.softcap > 0.0f || p.alibi != nullptr || p.win_left >= 0 ||
                    (p.win_right >= 0 && !(p.win_right == 0 && p.causal));
  // dropout has kernels of its own (the Philox rounds cost the other features no registers)
  if (p.dropout)
    return p.causal ? launch_bwd2<T, CQ, CKV, true, true, true>(p, st) : launch_bwd2<T, CQ, CKV, false, true, true>(p, st);
  if (p.causal)
    return feat ? launch_bwd2<T, CQ, CKV, true, true>(p, st) : launch_bwd2<T, CQ, CKV, true, false>(p, st);
  return feat ? launch_bwd2<T, CQ, CKV, false, true>(p, st) : launch_bwd2<T, CQ, CKV, false, false>(p, st);
}
}  // namespace fa
