// fwd_kernel.hpp — exact attention forward for gfx950 (MI355X), fp16 and bf16: the kernel and
// its launcher, instantiated per kernel width by fwd_d32.hip .. fwd_d256.hip (one translation
// unit each, so they compile in parallel).
//
// Replaces the reference forward (kernels/fa_forward.hip:52-313 kernel, :424-451 launcher);
// same math and masking contract (FableFwdParams in include/fable_attn_abi.h), new design:
//
//  * workgroup = NW waves; wave w owns 32 query rows, so a workgroup covers BR = 32*NW rows of
//    one (batch, head). Q for those rows lives in registers for the whole kernel, laid out as
//    the B operand of v_mfma_f32_32x32x16 (lane l holds query l%32, 8 head-dim values).
//  * scores are computed transposed, S^T = K . Q^T (A = K rows from LDS), so each lane holds
//    one query and BC/2 of its keys: the row max needs a single cross-half exchange
//    (v_permlane32_swap) and the probabilities P^T are already laid out as the B operand of
//    O^T = V^T . P^T. P never touches LDS.
//  * software pipeline: iteration j computes S(j+1) = K(j+1) . Q^T, then the PV product of tile
//    j and the softmax of tile j+1 in one branch-free block, so the VALU work of one tile runs
//    under the matrix-core work of the other. K and V have their own double buffers in LDS
//    (K is loaded two tiles ahead, V one) and there is one barrier per tile.
//  * LDS rows are padded (K by 16 bytes, V by 64 bytes) so that the 16-byte K reads of 16 rows
//    and the transposing V reads (ds_read_b64_tr_b16, 4 rows x 64 bytes per half-wave) hit
//    distinct banks, and every read address is a per-lane base plus an immediate offset.
//  * tile loads go through buffer descriptors (rows past the last needed key read as zeros),
//    so they carry no per-lane condition and stay in flight across a whole iteration.
//  * online softmax in the log2 domain (one FMA + v_exp_f32 per score). The running max only
//    moves when a tile raises it by more than 2^8 (probabilities then stay <= 256, exact in
//    fp16/bf16 range), so the O rescale is rare; it is skipped when no lane needs it. Row sums
//    add the fp32 probabilities.
//  * tiles entirely outside the causal / window / chunk range are never loaded; the leading
//    tiles every row of the workgroup sees in full run without mask code (template CAUSAL/FEAT
//    split as in the reference's launch_cfg, fa_forward.hip:409-421).
//  * the workgroup -> (q tile, head, batch) map is XCD-aware (the q tiles of one K/V head of
//    one sequence run on one XCD, whose L2 they share; heads are dealt round-robin to the XCDs)
//    and, for causal, starts with the heaviest q tiles.
#pragma once
#include <type_traits>

#include "attn_device.hpp"
#include "fwd_common.hpp"
#include "status.hpp"

namespace fa {

template <int HD_, int BC_, int NW_, int WPE_, int QB_ = 1>
struct FwdCfg {
  static constexpr int HD = HD_, BC = BC_, NW = NW_, WPE = WPE_;
  static constexpr int QB = QB_;            // 32-query blocks per wave
  static constexpr int NT = NW * 64;
  static constexpr int BR = NW * 32 * QB;
  static constexpr int NB = BC / 32;        // 32-key blocks per tile
  static constexpr int NG = BC / 16;        // 16-key groups per tile (PV contraction steps)
  static constexpr int NDS = HD / 16;       // Q.K contraction steps
  static constexpr int NDB = HD / 32;       // 32-row blocks of O^T
  static constexpr int DCH = HD / 8;        // 16-byte chunks per K/V row
  static constexpr int KSTR = HD + 8;       // LDS row strides (elements)
  static constexpr int VSTR = HD + 32;
  static constexpr int KTILE = BC * KSTR;
  static constexpr int VTILE = BC * VSTR;
  static constexpr int KCH = BC * DCH;      // chunks per K (or V) tile
  static constexpr int KJ = (KCH + NT - 1) / NT;  // chunks each thread loads per K (or V) tile
  static constexpr bool KTAIL = KCH % NT != 0;    // the last round leaves some threads idle
  static_assert(HD % 32 == 0 && BC % 32 == 0, "shape");
};

template <typename T, class C, bool CAUSAL, bool FEAT, bool DROP = false>
__global__ __attribute__((amdgpu_flat_work_group_size(C::NT, C::NT),
                          amdgpu_waves_per_eu(C::WPE, C::WPE))) void
fwd_kernel(FableFwdParams p, int nqt, FwdSplit sp) {
  using V8 = typename Dt<T>::V8;
  using V4 = typename Dt<T>::V4;
  // K/V rings of NST stages, a barrier every BP tiles. Iteration t reads K tile t+1 and V tile t
  // and stores K tile t+BP+1 and V tile t+BP, so what it reads was stored BP iterations earlier
  // and what it overwrites was last read BP iterations earlier: a barrier in every BP
  // consecutive iterations orders both. With BP = 2 the waves may drift up to two tiles apart
  // between barriers, so the two waves of a SIMD fall out of step and one's softmax runs under
  // the other's products. Used by the 8-wave D=128 shape (151.5 KB of LDS, one workgroup per
  // CU either way): C2 +0.4-1.9%, bf16 +1.9%, window 4096 +7.6%. The 8-wave D=64 shape was
  // 3.7% slower with it; the shorter shapes would lose workgroups per CU to the LDS.
  constexpr int NST = (C::NW == 8 && C::HD == 128) ? 4 : 2;
  constexpr int BP = NST / 2;
  __shared__ __attribute__((aligned(16))) T kl[NST * C::KTILE];
  __shared__ __attribute__((aligned(16))) T vl[NST * C::VTILE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5, j16 = lane & 15, mh = (lane >> 4) & 1;

  // ---- work item -> (sequence z, head h, q tile), and the key split (grid split-major)
  const int nitems = gridDim.x / sp.n;
  const int split = blockIdx.x / nitems;
  // (rows over 2048 keys stop at half the causal limit: B8 S4096 D128 1.04x and B4 S8192 1.03x
  // head after head at 512 items per XCD, whose K/V per head then stays in L2; at 2048 keys
  // u-major kept 1.04-1.17x there)
  const int umax = (CAUSAL && !FEAT && C::HD <= 128 && !p.cu_q) ? (p.SK <= 2048 ? kFwdUMajorCausal : kFwdUMajorCausal / 2)
                                                                : kFwdUMajor;
  const int w = xcd_group_remap(blockIdx.x - split * nitems, nitems, nqt, p.gqa, umax);
  const int qti = w % nqt, zh = w / nqt;
  const int h = zh % p.NH, z = zh / p.NH;
  const int qt = CAUSAL ? (nqt - 1 - qti) : qti;
  const int kvh = h / p.gqa;

  const SeqView sv = seq_view(p, z, h);
  const int SQ = sv.SQ, SK = sv.SK;
  const int qb = qt * C::BR;
  if (qb >= SQ) return;
  const int delta = SK - SQ;

  const T* Qg = (const T*)p.Q + sv.q0 + (long long)h * p.sQ.h;
  const T* Kg = (const T*)p.K + sv.k0 + (long long)kvh * p.sK.h;
  const T* Vg = (const T*)p.V + sv.v0 + (long long)kvh * p.sV.h;
  T* Og = (T*)p.O + sv.o0 + (long long)h * p.sO.h;

  // ---- block and wave key ranges
  constexpr int QB = C::QB;
  int bk0, bk1;
  key_range<CAUSAL, FEAT>(p, qb, min(qb + C::BR, SQ) - 1, delta, SK, bk0, bk1);
  const int qw = qb + wave * 32 * QB;  // first row of this wave; block i = rows qw+32i..+31
  const bool wave_rows = qw < SQ;
  int wk0 = 0, wk1 = 0;
  if (wave_rows) key_range<CAUSAL, FEAT>(p, qw, min(qw + 32 * QB, SQ) - 1, delta, SK, wk0, wk1);
  int kstart = (bk0 / C::BC) * C::BC;
  int ntiles = bk1 > bk0 ? (bk1 - kstart + C::BC - 1) / C::BC : 0;
  if (sp.n > 1) {  // this workgroup's share of the key tiles: a contiguous run of them
    const int per = (ntiles + sp.n - 1) / sp.n;
    const int t0 = min(split * per, ntiles), t1 = min(t0 + per, ntiles);
    kstart += t0 * C::BC;
    ntiles = t1 - t0;
  }

  // ---- Q (B operands) in registers: lane holds query qw + 32i + l32, head-dim 16ds + 8hh..+7.
  // A head dim p.HD below the kernel's C::HD (a multiple of 8) runs with zero columns
  // p.HD..C::HD-1 in Q, K and V: they add nothing to q.k, and the O columns they produce are
  // not stored.
  const int HDr = p.HD;
  V8 qreg[QB][C::NDS];
#pragma unroll
  for (int i = 0; i < QB; i++) {
    const int qi = qw + 32 * i + l32;
#pragma unroll
    for (int ds = 0; ds < C::NDS; ds++) {
      if (qi < SQ && 16 * ds + 8 * hh < HDr)
        qreg[i][ds] = *(const V8*)(Qg + (long long)qi * p.sQ.s + 16 * ds + 8 * hh);
      else
        qreg[i][ds] = bitcast<V8>(u32x4{0, 0, 0, 0});
    }
  }

  // Fixed softmax offset (bf16 softcap without alibi, cap c <= kFixCap): every logit, in log2
  // units c*tanh(.)*log2(e), lies in [-lcap, lcap] with lcap = c*log2(e), so the logits are
  // formed as x - lcap <= 0 and each probability 2^(x - lcap) lies in [2^(-2 lcap), 1], at
  // least 2^-95.3, inside the bf16 and fp32 normal ranges. The row max, its exchange and the
  // rescale test drop out, the subtraction folds into the transform's last FMA, and the LSE
  // adds c. (fp16 would flush such probabilities to zero; alibi leaves the logits unbounded.)
  constexpr float kFixCap = 33.0f;
  constexpr bool kFixT = FEAT && !DROP && std::is_same<T, __bf16>::value;
  const bool fixm = kFixT && p.softcap > 0.0f && p.softcap <= kFixCap && !p.alibi_slopes;
  f32x16 oacc[QB][C::NDB];
  float m_run[QB], l_run[QB];
#pragma unroll
  for (int i = 0; i < QB; i++) {
#pragma unroll
    for (int db = 0; db < C::NDB; db++) oacc[i][db] = f32x16{};
    m_run[i] = fixm ? 0.0f : -INFINITY;
    l_run[i] = 0.0f;
  }
  // FEAT masks: every mask (sequence end, causal, window, chunk) leaves row qi a single
  // visible key interval [rlo, rhi), so the edge-tile test per score is one unsigned compare,
  // with no uniform branches inside the score loop
  int rlo[QB], rspan[QB];
  if constexpr (FEAT) {
#pragma unroll
    for (int i = 0; i < QB; i++) {
      // (64-bit: window and chunk sizes up to INT_MAX must not wrap)
      const long long qd = qw + 32 * i + l32 + delta;
      long long lo = 0, hi = SK;
      if (CAUSAL) hi = min(hi, qd + 1);
      if (p.win_left >= 0) lo = max(lo, qd - p.win_left);
      if (p.win_right >= 0) hi = min(hi, qd + p.win_right + 1);
      if (p.attn_chunk > 0) {
        const long long cs = (max(qd, 0LL) / p.attn_chunk) * p.attn_chunk;
        lo = max(lo, cs);
        hi = min(hi, cs + p.attn_chunk);
      }
      rlo[i] = (int)lo;
      rspan[i] = (int)max(hi - lo, 0LL);
    }
  }
  const float c_log2 = p.scale * kLog2e;
  const float aslope = (FEAT && p.alibi_slopes) ? p.alibi_slopes[h] : 0.0f;

  // leading tiles that every row of the workgroup sees in full: no mask code for them
  int nint = 0;
  if (!FEAT) {
    int lim = SK;
    if (CAUSAL) lim = min(lim, qb + delta + 1);
    nint = min(max((lim - kstart) / C::BC, 0), ntiles);
  }

  // ---- global -> register loads of one tile through buffer descriptors spanning the rows
  // kb .. kvalid-1 of this head: rows past the last needed key read as zeros without a
  // per-lane condition (a conditional load would make the compiler wait for it at once), and
  // the per-lane byte offsets are loop invariant.
  const int kvalid = min(SK, kstart + ntiles * C::BC);
  // chunk j of this thread: ci = tid + j*NT, row ci / DCH, 16-byte column chunk ci % DCH. In the
  // last round (KTAIL) threads past the tile's chunks load row 0 again and store nothing;
  // chunks in the zero columns (>= p.HD) load from kBufZero, past the descriptor's range, which
  // reads zeros: no load depends on a lane condition and nothing is selected afterwards.
  // When NT is a multiple of DCH (every shape whose head dim is a power of two) a thread's
  // chunks share one column and sit RSTEP rows apart, so the LDS addresses are one base plus
  // immediate offsets; other shapes keep one address per chunk.
  constexpr bool kRowStep = C::NT % C::DCH == 0 && !C::KTAIL;
  constexpr int RSTEP = kRowStep ? C::NT / C::DCH : 0;
  int koff[C::KJ], voff[C::KJ], lko[C::KJ], lvo[C::KJ];
#pragma unroll
  for (int j = 0; j < C::KJ; j++) {
    const int ci = tid + j * C::NT;
    const bool live = !C::KTAIL || ci < C::KCH;
    const int r = live ? ci / C::DCH : 0, c = live ? ci % C::DCH : 0;
    const bool cok = 8 * c < HDr;
    koff[j] = cok ? r * (int)(p.sK.s * 2) + 16 * c : kBufZero;
    voff[j] = cok ? r * (int)(p.sV.s * 2) + 16 * c : kBufZero;
    if constexpr (kRowStep) {
      lko[j] = (tid / C::DCH) * C::KSTR + 8 * (tid % C::DCH) + j * RSTEP * C::KSTR;
      lvo[j] = (tid / C::DCH) * C::VSTR + 8 * (tid % C::DCH) + j * RSTEP * C::VSTR;
    } else {
      lko[j] = live ? r * C::KSTR + 8 * c : -1;
      lvo[j] = live ? r * C::VSTR + 8 * c : -1;
    }
  }
  u32x4 ldk[C::KJ], ldv[C::KJ];
  // K and V tiles are loaded in key order, kstart, kstart+BC, ... (each through its own
  // cursor): the descriptor advances by additions instead of 64-bit products of the tile's key
  const long long k_step = (long long)C::BC * p.sK.s, v_step = (long long)C::BC * p.sV.s;
  const T* k_cur = Kg + (long long)kstart * p.sK.s;
  const T* v_cur = Vg + (long long)kstart * p.sV.s;
  long long k_left = (long long)(kvalid - kstart) * p.sK.s * 2, v_left = (long long)(kvalid - kstart) * p.sV.s * 2;
  auto gload_k = [&]() {
    const auto r = buf_rsrc(k_cur, k_left);
#pragma unroll
    for (int j = 0; j < C::KJ; j++) ldk[j] = buf_load16(r, koff[j]);
    k_cur += k_step;
    k_left -= 2 * k_step;
  };
  auto gload_v = [&]() {
    const auto r = buf_rsrc(v_cur, v_left);
#pragma unroll
    for (int j = 0; j < C::KJ; j++) ldv[j] = buf_load16(r, voff[j]);
    v_cur += v_step;
    v_left -= 2 * v_step;
  };
  auto lstore_k = [&](int st) {
    T* b = kl + st * C::KTILE;
#pragma unroll
    for (int j = 0; j < C::KJ; j++)
      if (!C::KTAIL || j < C::KJ - 1 || lko[j] >= 0) *(u32x4*)(b + lko[j]) = ldk[j];
  };
  auto lstore_v = [&](int st) {
    T* b = vl + st * C::VTILE;
#pragma unroll
    for (int j = 0; j < C::KJ; j++)
      if (!C::KTAIL || j < C::KJ - 1 || lvo[j] >= 0) *(u32x4*)(b + lvo[j]) = ldv[j];
  };

  // S^T = K . Q^T for the K tile in stage st, every query block: lane reads key row
  // 32*jb + l32, head-dim 16*ds + 8*hh .. +7 (the A operand of v_mfma_f32_32x32x16), shared by
  // the blocks
  const int kro = l32 * C::KSTR + 8 * hh;
  auto qk = [&](int st, f32x16 (&s)[QB][C::NB]) {
    const T* kp = kl + st * C::KTILE + kro;
#pragma unroll
    for (int i = 0; i < QB; i++)
#pragma unroll
      for (int jb = 0; jb < C::NB; jb++) s[i][jb] = f32x16{};
    if constexpr (C::WPE == 1) {
      // One wave per SIMD: no other wave runs while this one waits on LDS, so the K fragments
      // are read in chunks of 16 before their products (read one product ahead, each product
      // of the dependent chain waited on its own read)
      // (contraction steps per chunk: at most 16 fragments, and the head dim's NDS steps,
      // which need not be a multiple of it)
      constexpr int CH = 16 / C::NB < C::NDS ? 16 / C::NB : C::NDS;
#pragma unroll
      for (int d0 = 0; d0 < C::NDS; d0 += CH) {
        V8 a[CH][C::NB];
#pragma unroll
        for (int ds = 0; ds < CH; ds++)
          if (d0 + ds < C::NDS)
#pragma unroll
            for (int jb = 0; jb < C::NB; jb++) a[ds][jb] = *(const V8*)(kp + jb * 32 * C::KSTR + 16 * (d0 + ds));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ds = 0; ds < CH; ds++)
          if (d0 + ds < C::NDS)
#pragma unroll
            for (int jb = 0; jb < C::NB; jb++)
#pragma unroll
              for (int i = 0; i < QB; i++) s[i][jb] = Dt<T>::mma32(a[ds][jb], qreg[i][d0 + ds], s[i][jb]);
      }
    } else {
#pragma unroll
      for (int ds = 0; ds < C::NDS; ds++)
#pragma unroll
        for (int jb = 0; jb < C::NB; jb++) {
          const V8 a = *(const V8*)(kp + jb * 32 * C::KSTR + 16 * ds);
#pragma unroll
          for (int i = 0; i < QB; i++) s[i][jb] = Dt<T>::mma32(a, qreg[i][ds], s[i][jb]);
        }
    }
  };
  // O^T += V^T . P^T for the V tile in stage st. A operand by transposing reads: lane j16 of
  // 16-lane group (mh, hh) addresses key row 16g+8a+4hh+j16/4, head-dim 32db+16mh+4*(j16%4)
  // and receives head-dim 32db+16mh+j16 of keys 16g+8a+4hh+0..3 (the keys of its P^T items
  // 4a..4a+3).
  const int vro = (4 * hh + (j16 >> 2)) * C::VSTR + 16 * mh + 4 * (j16 & 3);
  auto pv = [&](int st, const V8 (&pb)[QB][C::NG]) {
    const T* vp = vl + st * C::VTILE + vro;
#pragma unroll
    for (int db = 0; db < C::NDB; db++)
#pragma unroll
      for (int g = 0; g < C::NG; g++) {
        const V4 lo = lds_read_tr<T>(vp + 16 * g * C::VSTR + 32 * db);
        const V4 hi = lds_read_tr<T>(vp + (16 * g + 8) * C::VSTR + 32 * db);
        V8 av;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          av[e] = lo[e];
          av[4 + e] = hi[e];
        }
#pragma unroll
        for (int i = 0; i < QB; i++) oacc[i][db] = Dt<T>::mma32(av, pb[i][g], oacc[i][db]);
      }
  };
  // Softmax of one tile (keys kb..kb+BC-1) of query block i in s -> probabilities pb (the B
  // operands of the PV product), running max/sum update. Returns the factor the block's O
  // accumulators must be scaled by once every earlier tile's PV product is in them; `resc` is
  // set when any lane's is not 1. Branch-free, so the compiler can interleave it with
  // independent matrix-core work.
  // FEAT logits in log2 units. softcap: c * tanh(x / c) with x = scale * q.k, tanh(y) =
  // 1 - 2 / (exp(2y) + 1); exp(2y) = exp2(q.k * kcap), so no division per score
  const float kcap = p.softcap > 0.0f ? 2.0f * kLog2e * p.scale / p.softcap : 0.0f;
  const float lcap = p.softcap * kLog2e;
  // Polynomial softcap (transform bit 3; the one-wave loop of 32-key tiles below): tanh(y) =
  // y P(y^2) on |y| <= kPolyY, y = scale*s/c, odd degree 7, minimax coefficients from Lawson's
  // iteratively reweighted least squares: |error| <= 1.9e-8 exactly, 5e-8 evaluated in fp32,
  // against 1.8e-7 for the exp/rcp form above, with no transcendental; the logit (log2 units)
  // is u (a1 + u^2 (a3 + u^2 (a5 + u^2 a7))), u = s * kpoly, a_i = c_i * c * log2(e)
  constexpr float kPolyY = 0.4f;
  const float kpoly = p.softcap > 0.0f ? p.scale / p.softcap : 0.0f;
  const float prange = p.softcap > 0.0f ? kPolyY * p.softcap / p.scale : 0.0f;  // largest |s|
  const float pa1 = 0.9999995735192077f * lcap, pa3 = -0.3332972661781136f * lcap;
  const float pa5 = 0.1325057420337534f * lcap, pa7 = -0.046826030150687044f * lcap;
  const float aslope2 = aslope * kLog2e;
  // dropout: probabilities are scaled after the row sum, O = sum z p V / sum p
  const float keep_scale = DROP ? 1.0f / (1.0f - p.dropout_p) : 1.0f;
  // masked tiles: the lane's 16 keys of 32-key block jb sit at offsets 8*(r/4) + r%4 from
  // kb + 4*hh + 32*jb; the word has bit o set iff offset o is inside the row's interval
  // [rlo, rlo + rspan), so each score takes one bit extract and one bitfield insert (the
  // per-score add, compare and select cost one more instruction each)
  auto vis_word = [&](int i, int kb, int jb) -> unsigned {
    const int base = kb + 4 * hh + 32 * jb - rlo[i];
    const int a = min(max(-base, 0), 32), b = min(max(rspan[i] - base, 0), 32);
    return (unsigned)(((1ull << b) - 1ull) & ~((1ull << a) - 1ull));
  };
  // FEAT logit (log2 units) of score r of block jb of query block i: the transform `cap`
  // (bit 0 softcap, bit 1 alibi), then the interval mask
  auto logit = [&](auto masked, auto cap, int i, float sv, int kb, int jb, int r, unsigned vis) -> float {
    float x;
    // (bit 4: the fixed offset, the logit less lcap)
    constexpr bool kFix = (decltype(cap)::value & 16) != 0;
    if constexpr ((decltype(cap)::value & 8) != 0) {
      const float u = sv * kpoly, u2 = u * u;
      const float pu = fmaf(u2, fmaf(u2, fmaf(u2, pa7, pa5), pa3), pa1);
      x = kFix ? fmaf(u, pu, -lcap) : u * pu;
    } else if constexpr ((decltype(cap)::value & 1) != 0) {
      const float e = exp2_fast(sv * kcap);
      x = kFix ? (-2.0f * lcap) * __builtin_amdgcn_rcpf(e + 1.0f)
               : fmaf(-2.0f * lcap, __builtin_amdgcn_rcpf(e + 1.0f), lcap);
    } else {
      x = sv * c_log2;
    }
    if constexpr ((decltype(cap)::value & 2) != 0) {
      const int key = kb + 4 * hh + jb * 32 + 8 * (r >> 2) + (r & 3);
      x = fmaf(aslope2, (float)(key - (qw + 32 * i + l32)), x);
    }
    if constexpr (decltype(masked)::value) {
      const unsigned keep = (unsigned)__builtin_amdgcn_sbfe((int)vis, 8 * (r >> 2) + (r & 3), 1);
      x = __builtin_bit_cast(float, (__builtin_bit_cast(unsigned, x) & keep) | (0xFF800000u & ~keep));
    }
    return x;
  };
  // cap bit 2: the scores already hold their FEAT logits (transformed and masked by the caller)
  auto softmax = [&](auto masked, auto cap, int i, f32x16 (&s)[C::NB], int kb, V8 (&pb)[C::NG], bool& resc) {
    const int qi = qw + 32 * i + l32;
    const int kq = kb + 4 * hh;  // key of s[jb][r] = kq + 32*jb + 8*(r/4) + (r%4)
    if constexpr (FEAT && (decltype(cap)::value & 4) == 0) {
#pragma unroll
      for (int jb = 0; jb < C::NB; jb++) {
        const unsigned vis = decltype(masked)::value ? vis_word(i, kb, jb) : 0u;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          s[jb][r] = logit(masked, cap, i, s[jb][r], kb, jb, r, vis);
          // bound how many scores the scheduler transforms at once (the softcap transform's
          // register pressure); plain logits are left to the scheduler
          if constexpr ((decltype(cap)::value & 1) != 0)
            if ((r & 7) == 7) __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else if constexpr (!FEAT && decltype(masked)::value) {
#pragma unroll
      for (int jb = 0; jb < C::NB; jb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int key = kq + jb * 32 + 8 * (r >> 2) + (r & 3);
          const bool ok = CAUSAL ? (key < SK && key <= qi + delta) : key < SK;
          if (!ok) s[jb][r] = -INFINITY;
        }
    }
    // cap bit 4: the fixed offset (the logits are already shifted; m_run stays 0, no rescale)
    float corr = 1.0f, m_use = 0.0f;
    if constexpr ((decltype(cap)::value & 16) != 0) {
      resc = false;
    } else {
      float mx = -INFINITY;
#pragma unroll
      for (int jb = 0; jb < C::NB; jb++)
#pragma unroll
        for (int r = 0; r < 16; r++) mx = fmaxf(mx, s[jb][r]);
      mx = half_max(mx);
      const float m_cand = fmaxf(m_run[i], FEAT ? mx : mx * c_log2);
      const bool need = m_cand > m_run[i] + kLazyMax;
      corr = need ? exp2_fast(m_run[i] - m_cand) : 1.0f;
      // While a row's running max is -inf no key has been visible to it and its O accumulators
      // are still zero: the first tile a row sees moves the max but needs no rescale. The
      // feature kernels skip it (at head dim 256 a rescale is 384 VALU instructions, a tenth of
      // a 512-key window's work: C5 +1.3%); on the long rows of the plain kernels the extra
      // test per tile cost more than the one rescale (D=160/192 0.98x)
      const bool scale_o = FEAT ? need && m_run[i] != -INFINITY : need;
      m_run[i] = need ? m_cand : m_run[i];
      resc = __builtin_amdgcn_ballot_w64(scale_o) != 0;
      m_use = m_run[i] == -INFINITY ? 0.0f : m_run[i];
    }
    // The row sum adds the fp32 probabilities (not the rounded ones the PV product takes): the
    // LSE is then exact to fp32 rounding, and the backward, which rebuilds P = exp(s - LSE),
    // sees probabilities that sum to 1. Summing the fp16-rounded values pairwise (v_dot2) ran at
    // the same speed but left the LSE off by up to 2e-4, a row-wide scale error of every P the
    // fp16 backward rebuilt (its dQ/dK error against exact gradients rose from 3.7e-4 to 5.5e-4
    // on short causal rows). Dropout scales the probabilities after the sum either way.
    constexpr bool kPairSum = false;
    float r0 = 0.0f, r1 = 0.0f;
#pragma unroll
    for (int jb = 0; jb < C::NB; jb++)
#pragma unroll
      for (int sh = 0; sh < 2; sh++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float x = s[jb][8 * sh + e];
          const float pe = FEAT ? exp2_fast(x - m_use) : exp2_fast(fmaf(x, c_log2, -m_use));
          float pz = pe;
          if constexpr (DROP) {
            const int r = 8 * sh + e, key = kq + 32 * jb + 8 * (r >> 2) + (r & 3);
            pz *= dropout_z(p.philox_seed, ((uint64_t)h * SQ + qi) * SK + key, p.dropout_p, keep_scale);
          }
          pb[2 * jb + sh][e] = (T)pz;
          if (!kPairSum) (e & 1 ? r1 : r0) += pe;
        }
    if (kPairSum) {
#pragma unroll
      for (int g = 0; g < C::NG; g++)
#pragma unroll
        for (int e = 0; e < 8; e += 4) {
          r0 = Dt<T>::sum2(typename Dt<T>::V2{pb[g][e], pb[g][e + 1]}, r0);
          r1 = Dt<T>::sum2(typename Dt<T>::V2{pb[g][e + 2], pb[g][e + 3]}, r1);
        }
    }
    l_run[i] = l_run[i] * corr + (r0 + r1);
    return corr;
  };
  auto active = [&](int t) {
    const int kb = kstart + t * C::BC;
    return wave_rows && kb < wk1 && kb + C::BC > wk0;
  };
  // FEAT tiles that every row of this wave sees in full (no mask code); chunked attention
  // always takes the masked path
  auto interior = [&](int t) {
    const int kb = kstart + t * C::BC, ke = kb + C::BC - 1;
    const int r0 = qw + delta, r1 = qw + 32 * QB - 1 + delta;
    bool ok = ke < SK && p.attn_chunk <= 0;
    if (CAUSAL) ok = ok && ke <= r0;
    if (p.win_right >= 0) ok = ok && ke <= r0 + p.win_right;
    if (p.win_left >= 0) ok = ok && kb >= r1 - p.win_left;
    return ok;
  };
  using Plain = std::integral_constant<bool, false>;
  using Masked = std::integral_constant<bool, true>;
  // logit transform of the feature kernels: bit 0 softcap, bit 1 alibi; bit 4 (with bit 0 alone)
  // the fixed softmax offset of the bf16 softcap kernels (fixm)
  using Cap0 = std::integral_constant<int, 0>;
  const int fmode = FEAT ? (p.softcap > 0.0f ? 1 : 0) | (p.alibi_slopes ? 2 : 0) : 0;
  auto with_fmode = [&](auto f) {
    switch (fmode) {
      case 1:
        if constexpr (kFixT) {
          if (fixm) {
            f(std::integral_constant<int, 1 | 16>{});
            break;
          }
        }
        f(std::integral_constant<int, 1>{});
        break;
      case 2: f(std::integral_constant<int, 2>{}); break;
      case 3: f(std::integral_constant<int, 3>{}); break;
      default: f(Cap0{}); break;
    }
  };

  // ---- prologue: K tiles 0 and 1, V tile 0 in LDS; S and P of tile 0
  V8 pb[QB][C::NG];
  if (ntiles > 0) {
#pragma unroll
    for (int j = 0; j < BP; j++) {
      gload_k();  // tile j
      gload_v();  // tile j
      lstore_k(j);
      lstore_v(j);
    }
    gload_k();  // tile BP
    lstore_k(BP);
  }
  __syncthreads();
  bool a_cur = false;
  // a pending O rescale (from the softmax of the tile whose PV product comes next) is applied
  // at the top of the next iteration, so the softmax shares a basic block with the PV product
  bool resc[QB];
  float corr[QB];
#pragma unroll
  for (int i = 0; i < QB; i++) {
    resc[i] = false;
    corr[i] = 1.0f;
  }
  // resc is wave-uniform (a ballot); readfirstlane states it, so the branch is a scalar one.
  // As a divergent (exec-mask) branch, the compiler read every AGPR-held O accumulator into
  // VGPRs ahead of it on every tile (128 extra VALU per tile at head dim 256) and used the
  // copies only when the branch was taken.
  auto rescale = [&]() {
#pragma unroll
    for (int i = 0; i < QB; i++)
      if (__builtin_amdgcn_readfirstlane((int)resc[i])) {
#pragma unroll
        for (int db = 0; db < C::NDB; db++) oacc[i][db] *= corr[i];
        resc[i] = false;
      }
  };
  if (ntiles > 0) {
    f32x16 s[QB][C::NB];
    if (nint > 0) {
      a_cur = true;
      qk(0, s);
#pragma unroll
      for (int i = 0; i < QB; i++) corr[i] = softmax(Plain{}, Cap0{}, i, s[i], kstart, pb[i], resc[i]);
    } else if ((a_cur = active(0))) {
      qk(0, s);
      with_fmode([&](auto cap) {
#pragma unroll
        for (int i = 0; i < QB; i++) corr[i] = softmax(Masked{}, cap, i, s[i], kstart, pb[i], resc[i]);
      });
    }
  }
  __syncthreads();  // every wave has read K stage 0 before iteration 0 refills it

  // ---- iteration t: S of tile t+1, PV of tile t, softmax of tile t+1; then K tile t+2 and
  // V tile t+1 go to the stages tiles t and t-1 used.
  int t = 0;
  for (; t + 1 < nint; t++) {
    rescale();
    const int kb1 = kstart + (t + 1) * C::BC;
    gload_k();  // tile t+1+BP
    gload_v();  // tile t+BP
    f32x16 s[QB][C::NB];
    // raised wave priority over the S product: +1-3% at D=128; 1.5-6% slower at D=64 and 4-6%
    // slower at D=256 (one wave per SIMD there: nothing to take priority over), so not there
    if constexpr (C::HD == 128) __builtin_amdgcn_s_setprio(1);
    qk((t + 1) & (NST - 1), s);
    if constexpr (C::HD == 128) __builtin_amdgcn_s_setprio(0);
    pv(t & (NST - 1), pb);
#pragma unroll
    for (int i = 0; i < QB; i++) corr[i] = softmax(Plain{}, Cap0{}, i, s[i], kb1, pb[i], resc[i]);
    lstore_k((t + BP + 1) & (NST - 1));
    lstore_v((t + BP) & (NST - 1));
    if (BP == 1 || t % BP == BP - 1) __syncthreads();
  }
  if (t < ntiles && t > 0) a_cur = active(t);
  if constexpr (FEAT && !DROP && C::WPE == 1) {
    // One wave per SIMD (D=256): no second wave fills the matrix cores while this one runs
    // its softmax, so the overlap has to come from within the wave, which the branches of the
    // general iteration below (tile active? next tile masked?) prevent: they split the S
    // product, the PV product and the softmax into separate basic blocks. Here every
    // iteration is one basic block: every tile goes through the interval mask, and a tile
    // this wave does not see gives all-masked scores, zero probabilities and a PV product
    // that adds exact zeros. D=256 window 512: 275 -> 298 TFLOP/s, with softcap 259 -> 271.
    // (With two waves per SIMD the same loop is no faster, and the 64-key D=128 shape spills.)
    if (!a_cur) {
#pragma unroll
      for (int i = 0; i < QB; i++)
#pragma unroll
        for (int g = 0; g < C::NG; g++) pb[i][g] = bitcast<V8>(u32x4{0, 0, 0, 0});
    }
    with_fmode([&](auto cap) {
      for (; t + 1 < ntiles; t++) {
        rescale();
        const int kb1 = kstart + (t + 1) * C::BC;
        gload_k();  // tile t+1+BP
        gload_v();  // tile t+BP
        f32x16 s[QB][C::NB];
        qk((t + 1) & (NST - 1), s);
        if constexpr (QB == 1 && C::NDB * C::NG == 16 * C::NB) {
          // The PV products of tile t in steps of SPS, each step beside the logit transforms of
          // SPS scores of tile t+1 (head dim 256 has as many products as a lane has scores):
          // left to itself, the scheduler ran the transforms and the products one after the
          // other. The barrier after each step holds the order; the V reads run a step ahead.
          constexpr int NPV = C::NDB * C::NG;
          // products (and scores) per step: 4 lets four scores' dependent transform chains
          // overlap (C5 +2.8% and dense softcap +5% over the unordered schedule; 1, 2 and 8
          // measured 0.98-1.03x)
          constexpr int SPS = 4;
          const T* vp = vl + (t & (NST - 1)) * C::VTILE + vro;
          unsigned vis[C::NB];
#pragma unroll
          for (int jb = 0; jb < C::NB; jb++) vis[jb] = vis_word(0, kb1, jb);
          // Softcap by the polynomial on 32-key tiles (C5: 0.58 instead of 1.53 transcendentals
          // per MFMA, the same time); the 64-key softcap shape keeps the exp/rcp form (with the
          // polynomial it held 40 more registers, 491 of 512, and ran 0.96-0.97x). The raw
          // scores stay in registers for the rare tile outside the polynomial's range.
          constexpr bool kPoly = (decltype(cap)::value & 1) != 0 && C::NB == 1;
          using CapP = std::integral_constant<int, decltype(cap)::value | (kPoly ? 8 : 0)>;
          float raw[kPoly ? 16 * C::NB : 1];
          float amax = 0.0f;  // largest |raw score| of the lane's tile
          V4 rd[2][SPS][2];
          auto vread = [&](int k, V4 (&r)[2]) {
            const int db = k / C::NG, g = k % C::NG;
            r[0] = lds_read_tr<T>(vp + 16 * g * C::VSTR + 32 * db);
            r[1] = lds_read_tr<T>(vp + (16 * g + 8) * C::VSTR + 32 * db);
          };
#pragma unroll
          for (int u = 0; u < SPS; u++) vread(u, rd[0][u]);
#pragma unroll
          for (int k = 0; k < NPV; k += SPS) {
            const int b = (k / SPS) & 1;
#pragma unroll
            for (int u = 0; u < SPS; u++) {
              if (k + SPS + u < NPV) vread(k + SPS + u, rd[b ^ 1][u]);
              V8 av;
#pragma unroll
              for (int e = 0; e < 4; e++) {
                av[e] = rd[b][u][0][e];
                av[4 + e] = rd[b][u][1][e];
              }
              oacc[0][(k + u) / C::NG] = Dt<T>::mma32(av, pb[0][(k + u) % C::NG], oacc[0][(k + u) / C::NG]);
            }
            // the empty asm ties the scores to this step (pure arithmetic moves freely across
            // the scheduling barrier before instruction selection)
#pragma unroll
            for (int u = 0; u < SPS; u++) {
              const int kk = k + u;
              float sk = s[0][kk / 16][kk % 16];
              asm volatile("" : "+v"(sk));
              if constexpr (kPoly) {
                raw[kk] = sk;
                amax = fmaxf(amax, fabsf(sk));
              }
              s[0][kk / 16][kk % 16] = logit(Masked{}, CapP{}, 0, sk, kb1, kk / 16, kk % 16, vis[kk / 16]);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
          const float m_keep = m_run[0], l_keep = l_run[0];
          corr[0] = softmax(Masked{}, std::integral_constant<int, 4 | (decltype(cap)::value & 16)>{}, 0, s[0], kb1, pb[0], resc[0]);
          if constexpr (kPoly && (decltype(cap)::value & 16) != 0) {
            // With the fixed offset nothing in the softmax waits for the row max, and the
            // compiler moved the exponentials past the range test below (on its fallback path
            // they are dead): formed here, they stay in the block of the products.
#pragma unroll
            for (int g = 0; g < C::NG; g++) asm volatile("" : "+v"(pb[0][g]));
            asm volatile("" : "+v"(l_run[0]));
          }
          if constexpr (kPoly) {
            // A score outside the polynomial's range anywhere in the wave: the row state goes
            // back to before this tile, and the tile is redone with the exp/rcp form. The test
            // comes after the softmax, so the common path keeps the products and the whole
            // softmax in one basic block (tested before it, the softmax moved to a block of its
            // own and C5 ran 0.98-0.99x)
            if (__builtin_amdgcn_readfirstlane((int)(__builtin_amdgcn_ballot_w64(!(amax <= prange)) != 0))) {
              m_run[0] = m_keep;
              l_run[0] = l_keep;
#pragma unroll
              for (int kk = 0; kk < 16 * C::NB; kk++) {
                // (the exact form stays inside the branch: not hoisted ahead of the test)
                float rv = raw[kk];
                asm volatile("" : "+v"(rv));
                s[0][kk / 16][kk % 16] = logit(Masked{}, cap, 0, rv, kb1, kk / 16, kk % 16, vis[kk / 16]);
              }
              corr[0] = softmax(Masked{}, std::integral_constant<int, 4 | (decltype(cap)::value & 16)>{}, 0, s[0], kb1, pb[0], resc[0]);
            }
          }
        } else {
          pv(t & (NST - 1), pb);
#pragma unroll
          for (int i = 0; i < QB; i++) corr[i] = softmax(Masked{}, cap, i, s[i], kb1, pb[i], resc[i]);
        }
        lstore_k((t + BP + 1) & (NST - 1));
        lstore_v((t + BP) & (NST - 1));
        if (BP == 1 || t % BP == BP - 1) __syncthreads();
      }
    });
    // the last tile: its PV product only (the loop's S product and softmax of the tile after
    // it would score keys past the range: C5 spent ~4% of its work there)
    if (t < ntiles) {
      rescale();
      pv(t & (NST - 1), pb);
      t++;
    }
  }
  for (; t < ntiles; t++) {
    rescale();
    const int kb1 = kstart + (t + 1) * C::BC;
    gload_k();  // tile t+1+BP
    gload_v();  // tile t+BP
    const bool a_next = t + 1 < ntiles && active(t + 1);
    f32x16 s[QB][C::NB];
    if (a_next) qk((t + 1) & (NST - 1), s);
    if (a_cur) pv(t & (NST - 1), pb);
    if (a_next) {
      // FEAT tiles every row of the wave sees in full skip the mask code
      auto sm = [&](auto masked, auto cap) {
#pragma unroll
        for (int i = 0; i < QB; i++) corr[i] = softmax(masked, cap, i, s[i], kb1, pb[i], resc[i]);
      };
      if (FEAT && interior(t + 1))
        with_fmode([&](auto cap) { sm(Plain{}, cap); });
      else
        with_fmode([&](auto cap) { sm(Masked{}, cap); });
    }
    a_cur = a_next;
    lstore_k((t + BP + 1) & (NST - 1));
    lstore_v((t + BP) & (NST - 1));
    if (BP == 1 || t % BP == BP - 1) __syncthreads();
  }

  // ---- epilogue: O = acc / l, LSE (a key split: the fp32 partial O and LSE of its keys); with
  // the fixed offset the logits were formed less lcap
  const float m_base = fixm ? lcap : 0.0f;
#pragma unroll
  for (int i = 0; i < QB; i++) {
    const int qi = qw + 32 * i + l32;
    const float l_tot = half_sum(l_run[i]);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (sp.n > 1) {
      const long long r = (long long)split * sp.rows + (long long)w * C::BR + (qi - qb);
#pragma unroll
      for (int db = 0; db < C::NDB; db++)
        store_cblock_f32(sp.o + r * HDr + db * 32, oacc[i][db], inv, hh, qi < SQ, HDr - db * 32);
      if (qi < SQ && hh == 0) sp.lse[r] = l_tot > 0.0f ? (m_run[i] + m_base) * kLn2 + __logf(l_tot) : -INFINITY;
      continue;
    }
    T* orow = Og + (long long)qi * p.sO.s;
#pragma unroll
    for (int db = 0; db < C::NDB; db++)
      store_cblock<T>(orow + db * 32, oacc[i][db], inv, hh, qi < SQ, HDr - db * 32);
    if (qi < SQ) {
      if (p.LSE && hh == 0)
        p.LSE[sv.lse0 + qi] = l_tot > 0.0f ? (m_run[i] + m_base) * kLn2 + __logf(l_tot) : -INFINITY;
    }
  }
}

// Workgroup shapes per head dim: C (the widest) runs the plain masks (causal / sequence end)
// and the wide-window / alibi feature kernels; CS the plain masks when C's grid would give
// fewer than 4 workgroups per CU (short sequences: more, shorter workgroups balance better);
// CF the softcap and dropout kernels, whose per-score work needs a different register
// balance; CN the narrow masks (a window or chunk under 2048 keys), where a tall workgroup's
// key span would be mostly masked and its fixed costs (Q rows, pipeline fill, output) are paid
// over few tiles, so shorter workgroups, more of them per CU, win; CL and CR the plain masks
// on long and on short causal rows (below, at launch_fwd). Dropout has kernels of its own, so its Philox rounds cost the
// other features no registers.
template <class K>
struct CfgTag {
  using type = K;
};

// Key split of a small grid: splits per query tile when the tiles fill at most half the CUs,
// up to one workgroup per CU, at least kSplitMinTiles key tiles per split, at most 16. A causal
// grid of one round (at most one workgroup per CU) with rows of kSplitLongRow key tiles or more
// splits in two: its longest rows set the time (B1 H8 S8192 D128 1.27-1.30x, H6 1.17x, H4
// S16384 1.12x); with shorter rows the halves of a grid over 128 workgroups take a second round
// (H12 S4096, 64 tiles: 0.87x).
constexpr long long kSplitSlots = 256;
constexpr int kSplitMinTiles = 4, kSplitLongRow = 128;

template <class K>
static int fwd_split_count(const FableFwdParams& p, long long nblk) {
  if (p.dropout_p > 0.0f || p.win_left >= 0 || p.attn_chunk > 0) return 1;
  if (nblk <= 0) return 1;
  const int tiles = (p.SK + K::BC - 1) / K::BC;  // the most any query tile reads
  if (2 * nblk > kSplitSlots) return (p.causal && nblk <= kSplitSlots && tiles >= kSplitLongRow) ? 2 : 1;
  long long n = (kSplitSlots + nblk - 1) / nblk;
  n = n < tiles / kSplitMinTiles ? n : tiles / kSplitMinTiles;
  n = n < 16 ? n : 16;
  return n >= 2 ? (int)n : 1;
}

// CL: the plain masks on long rows (no causal mask, or a causal one over at least kLongKeys
// keys) when its grid gives at least 4 workgroups per CU (D=64: 4-wave workgroups at three
// waves per SIMD, 1.04-1.12x over the 8-wave shape there; 0.90-0.97x on causal rows of 2048 and
// 4096 keys, whose shorter workgroups pay the diagonal tiles and the K/V loads of half as many
// rows more often)
constexpr int kLongKeys = 8192;
// CR: the plain masks on short causal rows (at head dim 96 non-causal ones too; at most
// kShortKeys keys) when C's grid gives at
// least 4 workgroups per CU (D=128: 2-wave workgroups of 64 rows and 32-key tiles; on a row of
// 512 keys half the tiles of a 256-row workgroup straddle the diagonal. Varlen batches of
// 64-1024-token sequences 1.53-1.58x, dense B16 S1024 H32 1.22x, B64 S512 1.16x; on a grid of
// 512 workgroups (B8 S1024 H16) 0.81x, so larger grids only)
constexpr int kShortKeys = 1024;

template <typename T, class C, class CF, class CN, class CS = C, class CL = C, class CR = C>
static int launch_fwd(const FableFwdParams& p, hipStream_t st, FwdWs& ws) {
  const bool drop = p.dropout_p > 0.0f;
  const bool feat = drop || p.softcap > 0.0f || p.alibi_slopes != nullptr || p.attn_chunk > 0 ||
                    p.win_left >= 0 || (p.win_right >= 0 && !(p.win_right == 0 && p.causal));
  auto short_span = [](int w) { return w >= 0 && w < 2048; };
  const bool narrow = short_span(p.win_left) || (p.attn_chunk > 0 && p.attn_chunk < 2048) ||
                      (short_span(p.win_right) && !(p.win_right == 0 && p.causal));
  const bool heavy = drop || p.softcap > 0.0f;
  auto go = [&](auto cfg, auto causal, auto ft, auto dr) -> int {
    using K = typename decltype(cfg)::type;
    const int nqt = (p.SQ + K::BR - 1) / K::BR;
    const long long nblk = (long long)nqt * p.NH * p.batch;
    FwdSplit sp{1, nqt, K::BR, 0, nullptr, nullptr};
    const int n = fwd_split_count<K>(p, nblk);
    if (n > 1) {
      const long long rows = nblk * K::BR;
      const long long obytes = ((long long)n * rows * p.HD * 4 + 255) / 256 * 256;
      const long long need = obytes + (long long)n * rows * 4;
      if (ws.query) {
        ws.need = need;
        return FA_OK;
      }
      if (ws.ptr && ws.bytes >= need && ((uintptr_t)ws.ptr & 255) == 0)
        sp = FwdSplit{n, nqt, K::BR, rows, (float*)ws.ptr, (float*)((char*)ws.ptr + obytes)};
    }
    if (ws.query) {
      ws.need = 0;
      return FA_OK;
    }
    if (nblk <= 0) return FA_OK;
    if (nblk * sp.n > 0x7FFFFFFF) return fail(FA_ERR_ARG, "fable_attn_fwd: grid too large");
    hipLaunchKernelGGL((fwd_kernel<T, K, decltype(causal)::value, decltype(ft)::value, decltype(dr)::value>),
                       dim3((unsigned)(nblk * sp.n)), dim3(K::NT), 0, st, p, nqt, sp);
    const int rc = launch_status("fable_attn_fwd");
    if (rc != FA_OK || sp.n == 1) return rc;
    return launch_fwd_split_combine(p, std::is_same<T, _Float16>::value ? FA_F16 : FA_BF16, sp, st);
  };
  auto pick = [&](auto causal) -> int {
    using Y = std::integral_constant<bool, true>;
    using N = std::integral_constant<bool, false>;
    if (narrow) {
      if (drop) return go(CfgTag<CN>{}, causal, Y{}, Y{});
      return go(CfgTag<CN>{}, causal, Y{}, N{});
    }
    if (heavy) {
      if (drop) return go(CfgTag<CF>{}, causal, Y{}, Y{});
      return go(CfgTag<CF>{}, causal, Y{}, N{});
    }
    if (feat) return go(CfgTag<C>{}, causal, Y{}, N{});
    if constexpr (!std::is_same<CR, C>::value) {
      const long long nc = (long long)((p.SQ + C::BR - 1) / C::BR) * p.NH * p.batch;
      // (non-causal short rows too at head dim 96: B64 S512 H32 1.14x, B16 S1024 1.07x; at 32, 64
      // and 128 they ran 0.69-0.97x)
      if ((p.causal || C::HD == 96) && p.SK <= kShortKeys && nc >= 4 * 256) return go(CfgTag<CR>{}, causal, N{}, N{});
    }
    if constexpr (!std::is_same<CL, C>::value) {
      const long long nl = (long long)((p.SQ + CL::BR - 1) / CL::BR) * p.NH * p.batch;
      if ((!p.causal || p.SK >= kLongKeys) && nl >= 4 * 256) return go(CfgTag<CL>{}, causal, N{}, N{});
    }
    if constexpr (!std::is_same<CS, C>::value) {
      constexpr long long kSmallGrid = 4 * 256;  // 4 workgroups of shape C per CU
      if ((long long)((p.SQ + C::BR - 1) / C::BR) * p.NH * p.batch < kSmallGrid)
        return go(CfgTag<CS>{}, causal, N{}, N{});
    }
    return go(CfgTag<C>{}, causal, N{}, N{});
  };
  return p.causal ? pick(std::integral_constant<bool, true>{}) : pick(std::integral_constant<bool, false>{});
}

}  // namespace fa
