/*
 * oracle.c — fp64 CPU restatement of the reference's attention oracles.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library links, loads or calls this code; it
 * is the checker used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 *
 * Every routine accumulates in double, takes inputs that the caller has already rounded to the
 * storage dtype (fp16/bf16 values held in float), and follows a reference routine:
 *   oracle_fwd      kernels/fa_common.hpp:102-134 (ref_attention): mask order causal,
 *                   window left/right, chunk; softcap before alibi; alibi slope*(j-i);
 *                   a row with no visible key gives O = 0 and LSE = -inf.
 *                   Batch/GQA indexing as kernels/fa_forward_gate.inc:33-47.
 *   oracle_bwd      kernels/backward.hip:566-597 (fp64 backward of the gate): recompute P from
 *                   the exact forward, Di = sum(O*dO), dS = P*(z*dP - Di)*softcap'(.), dQ,dK,dV
 *                   with dropout multiplier z (1 when dropout_p == 0).
 *   oracle_bwd_model the same gradients with only the roundings a 16-bit-operand backward must
 *                   make (O before Di, or Di from a given stored O; z*P before dV; dS before
 *                   dK/dQ); not a reference routine: it measures the floor of fp16/bf16
 *                   kernels against oracle_bwd.
 *   dropout         kernels/fa_common.hpp:71-88: Philox4x32-10 (Salmon, Moraes, Dror, Shaw,
 *                   "Parallel random numbers: as easy as 1, 2, 3", SC 2011) on counter
 *                   (idx, 0, 0) and key = seed; u = (word0 >> 8) * 2^-24; kept (z = 1/(1-p))
 *                   iff u >= p; idx = (h*SQ + i)*SK + j with no batch term
 *                   (fa_forward.hip:255-259, backward.hip:172). The forward normalises with
 *                   the undropped sum: O = sum_j z_j p_j V_j, LSE unchanged.
 *   oracle_decode   kernels/fa_decode_gate.inc:19-25 (rot_at) and :66-96 (oracle loop): new
 *                   tokens at ctx+tk, causal among new tokens via append, window lo =
 *                   qpos-window+1, leftpad, softcap, alibi slope*(pos-qpos), rotary (neox /
 *                   interleaved) applied to q and to appended k at their positions.
 *
 * Layouts (all contiguous, float):
 *   fwd/bwd: Q,O,dO,dQ [B][H][SQ][D]; K,V,dK,dV [B][Hk][SK][D]; LSE [B][H][SQ].
 *   decode:  q,o [B][nq][H][D]; Kc,Vc [nblocks][page][Hk][D]; block_table [B][max_blocks];
 *            new_k,new_v [B][nq][Hk][D]; cos,sin [seqlen_ro][rdim/2]; lse [B][nq][H].
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct OracleCfg {
  int B, H, Hk, SQ, SK, D;
  double scale, softcap;
  int win_left, win_right, causal, attn_chunk;
  const float* alibi; /* [H] or NULL */
  double dropout_p;   /* 0: no dropout */
  uint64_t seed;
} OracleCfg;

/* Philox4x32-10: 10 rounds of the published round function with multipliers 0xD2511F53 and
 * 0xCD9E8D57 and key bumps 0x9E3779B9, 0xBB67AE85 (Salmon et al. 2011, Random123). */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; r++) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n1 = (uint32_t)p1;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1, n3 = (uint32_t)p0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* dropout multiplier of (h, i, j): 0 or 1/(1-p) — fa_common.hpp:84-88 */
double oracle_drop_mul(uint64_t seed, uint64_t idx, double p) {
  const uint32_t ctr[4] = {(uint32_t)idx, (uint32_t)(idx >> 32), 0u, 0u};
  const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t out[4];
  oracle_philox4x32_10(ctr, key, out);
  const float u = (float)(out[0] >> 8) * (1.0f / 16777216.0f);
  return u >= (float)p ? 1.0 / (1.0 - p) : 0.0;
}

/* z[h][i][j] for h < H, i < SQ, j < SK (the dropout multipliers of one sequence) */
void oracle_dropout_mask(uint64_t seed, double p, int H, int SQ, int SK, double* z) {
  for (int h = 0; h < H; h++)
    for (int i = 0; i < SQ; i++)
      for (int j = 0; j < SK; j++) {
        const uint64_t idx = ((uint64_t)h * (uint64_t)SQ + (uint64_t)i) * (uint64_t)SK + (uint64_t)j;
        z[((size_t)h * SQ + i) * SK + j] = oracle_drop_mul(seed, idx, p);
      }
}

static double drop_mul(const OracleCfg* c, int h, int i, int j) {
  if (c->dropout_p <= 0) return 1.0;
  const uint64_t idx = ((uint64_t)h * (uint64_t)c->SQ + (uint64_t)i) * (uint64_t)c->SK + (uint64_t)j;
  return oracle_drop_mul(c->seed, idx, c->dropout_p);
}

/* visibility of key j to query i — fa_common.hpp:111-118 */
static int visible(const OracleCfg* c, int i, int j) {
  const int delta = c->SK - c->SQ;
  if (c->causal && j > i + delta) return 0;
  if (c->win_left >= 0 && j < i + delta - c->win_left) return 0;
  if (c->win_right >= 0 && j > i + delta + c->win_right) return 0;
  if (c->attn_chunk > 0) {
    int pp = i + delta;
    if (pp < 0) pp = 0;
    int cs = (pp / c->attn_chunk) * c->attn_chunk;
    if (j < cs || j >= cs + c->attn_chunk) return 0;
  }
  return 1;
}

/* logit of (i, j) — fa_common.hpp:119-123; also returns d(logit)/d(scale*qk) for softcap */
static double logit(const OracleCfg* c, int h, int i, int j, const float* q, const float* k,
                    double* deriv) {
  double s = 0.0;
  for (int d = 0; d < c->D; d++) s += (double)q[d] * (double)k[d];
  s *= c->scale;
  double dv = 1.0;
  if (c->softcap > 0) {
    double t = tanh(s / c->softcap);
    s = c->softcap * t;
    dv = 1.0 - t * t;
  }
  if (c->alibi) s += (double)c->alibi[h] * (double)(j - i);
  if (deriv) *deriv = dv;
  return s;
}

/* Forward. rows: optional list of query indices (n_rows entries) to evaluate for every (b,h);
 * NULL means all SQ rows. Rows not evaluated are left untouched in O/LSE. */
void oracle_fwd(const float* Q, const float* K, const float* V, float* O, float* LSE,
                const OracleCfg* c, const int32_t* rows, int n_rows) {
  const int gqa = c->H / c->Hk;
  const int nr = rows ? n_rows : c->SQ;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < c->B; b++)
    for (int h = 0; h < c->H; h++) {
      const int kvh = h / gqa;
      double* pr = (double*)malloc(sizeof(double) * (size_t)(c->SK > 0 ? c->SK : 1));
      const float* Kb = K + ((size_t)b * c->Hk + kvh) * (size_t)c->SK * c->D;
      const float* Vb = V + ((size_t)b * c->Hk + kvh) * (size_t)c->SK * c->D;
      for (int r = 0; r < nr; r++) {
        const int i = rows ? rows[r] : r;
        const float* q = Q + (((size_t)b * c->H + h) * c->SQ + i) * c->D;
        double mx = -INFINITY;
        int cnt = 0;
        for (int j = 0; j < c->SK; j++) {
          if (!visible(c, i, j)) { pr[j] = -INFINITY; continue; }
          double s = logit(c, h, i, j, q, Kb + (size_t)j * c->D, NULL);
          pr[j] = s;
          if (s > mx) mx = s;
          cnt++;
        }
        double sum = 0.0;
        for (int j = 0; j < c->SK; j++) {
          if (pr[j] == -INFINITY) { pr[j] = 0.0; continue; }
          pr[j] = exp(pr[j] - mx);
          sum += pr[j];
        }
        if (c->dropout_p > 0)
          for (int j = 0; j < c->SK; j++) pr[j] *= drop_mul(c, h, i, j);  /* after the sum */
        float* o = O + (((size_t)b * c->H + h) * c->SQ + i) * c->D;
        for (int d = 0; d < c->D; d++) {
          double acc = 0.0;
          for (int j = 0; j < c->SK; j++) acc += pr[j] * (double)Vb[(size_t)j * c->D + d];
          o[d] = (float)(cnt ? acc / sum : 0.0);
        }
        if (LSE) LSE[((size_t)b * c->H + h) * c->SQ + i] = cnt ? (float)(mx + log(sum)) : -INFINITY;
      }
      free(pr);
    }
}

/* Backward (exact fp64 gradients of the forward above). dQ/dK/dV are double outputs,
 * overwritten. dO [B][H][SQ][D]. */
static float round_f16(float x);
static float round_bf16(float x);

/* Round a double to the storage dtype of `mode` (0 keep, 1 fp16, 2 bf16), back to double. */
static double round_mode(double x, int mode) {
  if (mode == 1) return (double)round_f16((float)x);
  if (mode == 2) return (double)round_bf16((float)x);
  return x;
}

/* mode 0: exact fp64 gradients. mode 1/2 (fp16/bf16): the same gradients with the roundings a
 * kernel that feeds 16-bit matrix products must make, and nothing else: O is rounded to the
 * dtype before Di = sum(O*dO) (the kernels read D from the stored O), the dropped probability
 * z*P is rounded before dV += (z*P)^T dO, and dS is rounded (before the softmax scale) before
 * dK += scale*dS^T Q and dQ += scale*dS K. Accumulation stays in double. The distance of this
 * model from mode 0 is the floor that any 16-bit-operand backward shows against the exact
 * gradients. */
static void bwd_impl(const float* Q, const float* K, const float* V, const float* dO, double* dQ,
                     double* dK, double* dV, const OracleCfg* c, int mode, const float* Ost) {
  const int gqa = c->H / c->Hk;
  const size_t nq = (size_t)c->B * c->H * c->SQ * c->D, nk = (size_t)c->B * c->Hk * c->SK * c->D;
  memset(dQ, 0, nq * sizeof(double));
  memset(dK, 0, nk * sizeof(double));
  memset(dV, 0, nk * sizeof(double));
  /* parallel over (b, kv head): each task owns dK/dV of its kv head and dQ of its q heads */
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < c->B; b++)
    for (int kvh = 0; kvh < c->Hk; kvh++) {
      double* P = (double*)malloc(sizeof(double) * (size_t)(c->SK > 0 ? c->SK : 1));
      double* Dv = (double*)malloc(sizeof(double) * (size_t)(c->SK > 0 ? c->SK : 1));
      double* o = (double*)malloc(sizeof(double) * (size_t)c->D);
      const float* Kb = K + ((size_t)b * c->Hk + kvh) * (size_t)c->SK * c->D;
      const float* Vb = V + ((size_t)b * c->Hk + kvh) * (size_t)c->SK * c->D;
      double* dKb = dK + ((size_t)b * c->Hk + kvh) * (size_t)c->SK * c->D;
      double* dVb = dV + ((size_t)b * c->Hk + kvh) * (size_t)c->SK * c->D;
      for (int h = kvh * gqa; h < (kvh + 1) * gqa; h++)
        for (int i = 0; i < c->SQ; i++) {
          const size_t qo = (((size_t)b * c->H + h) * c->SQ + i) * c->D;
          const float* q = Q + qo;
          const float* g = dO + qo;
          double mx = -INFINITY;
          int cnt = 0;
          for (int j = 0; j < c->SK; j++) {
            if (!visible(c, i, j)) { P[j] = -INFINITY; continue; }
            double dv;
            P[j] = logit(c, h, i, j, q, Kb + (size_t)j * c->D, &dv);
            Dv[j] = dv;
            if (P[j] > mx) mx = P[j];
            cnt++;
          }
          if (!cnt) continue;
          double sum = 0.0;
          for (int j = 0; j < c->SK; j++) {
            if (P[j] == -INFINITY) { P[j] = 0.0; continue; }
            P[j] = exp(P[j] - mx);
            sum += P[j];
          }
          for (int j = 0; j < c->SK; j++) P[j] /= sum;
          /* O (exact, with dropout) and Di = sum_d O*dO — backward.hip:576-579 */
          double Di = 0.0;
          for (int d = 0; d < c->D; d++) {
            double acc = 0.0;
            for (int j = 0; j < c->SK; j++)
              acc += P[j] * drop_mul(c, h, i, j) * (double)Vb[(size_t)j * c->D + d];
            o[d] = Ost ? (double)Ost[qo + d] : round_mode(acc, mode);
            Di += o[d] * (double)g[d];
          }
          double* dq = dQ + qo;
          for (int j = 0; j < c->SK; j++) {
            if (P[j] == 0.0 && !visible(c, i, j)) continue;
            const double z = drop_mul(c, h, i, j);
            double dp = 0.0;
            for (int d = 0; d < c->D; d++) dp += (double)g[d] * (double)Vb[(size_t)j * c->D + d];
            const double dS = round_mode(P[j] * (z * dp - Di) * Dv[j], mode); /* backward.hip:170-176 */
            const double zp = round_mode(z * P[j], mode);
            for (int d = 0; d < c->D; d++) {
              dVb[(size_t)j * c->D + d] += zp * (double)g[d];
              dKb[(size_t)j * c->D + d] += c->scale * dS * (double)q[d];
              dq[d] += c->scale * dS * (double)Kb[(size_t)j * c->D + d];
            }
          }
        }
      free(P);
      free(Dv);
      free(o);
    }
}

/* exact fp64 gradients */
void oracle_bwd(const float* Q, const float* K, const float* V, const float* dO, double* dQ,
                double* dK, double* dV, const OracleCfg* c) {
  bwd_impl(Q, K, V, dO, dQ, dK, dV, c, 0, NULL);
}

/* rounding model of a 16-bit-operand backward (mode 1 fp16, 2 bf16), see bwd_impl; Ost (or
 * NULL) is a stored forward output [B][H][SQ][D] to take D = rowsum(O*dO) from, as a backward
 * that reads the forward's stored O does */
void oracle_bwd_model(const float* Q, const float* K, const float* V, const float* dO,
                      double* dQ, double* dK, double* dV, const OracleCfg* c, int mode,
                      const float* Ost) {
  bwd_impl(Q, K, V, dO, dQ, dK, dV, c, mode, Ost);
}

typedef struct OracleDecCfg {
  int B, nq, H, Hk, D, page, max_blocks;
  double scale, softcap;
  int window;  /* <0 off: number of keys back from the query position */
  int rotary;  /* 0 none, 1 neox, 2 interleaved */
  int rdim;    /* rotary dim (0 => D) */
  int append;  /* new_k/new_v present */
  const float* alibi; /* [H] or NULL */
  int round_append; /* 0: keep the rotated appended k exact; 1: round it to fp16; 2: to bf16 */
} OracleDecCfg;

/* Round a float to the nearest fp16 value (ties to even), overflow to inf, subnormals kept. */
static float round_f16(float x) {
  const float ax = fabsf(x);
  if (x != x) return x;
  if (!(ax < 65520.0f)) return copysignf(INFINITY, x);
  float q;
  if (ax < 6.103515625e-05f) {
    q = 5.9604644775390625e-08f; /* 2^-24: fp16 subnormal quantum */
  } else {
    int e;
    frexpf(ax, &e);
    q = ldexpf(1.0f, e - 11); /* 10 stored mantissa bits */
  }
  return copysignf(nearbyintf(ax / q) * q, x);
}

/* Round a float to bf16 (ties to even), as fa_forward_gate.inc:4-5. */
static float round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7F800000u) == 0x7F800000u) return x;
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

/* rot_at — fa_decode_gate.inc:20-25, generalised to rotary_dim <= D */
static void rot_at(double* v, int rdim, const float* cs, const float* sn, int mode, int pos) {
  const int half = rdim / 2;
  const float* c = cs + (size_t)pos * half;
  const float* s = sn + (size_t)pos * half;
  if (mode == 1) {
    for (int d = 0; d < half; d++) {
      double x = v[d], y = v[d + half];
      v[d] = x * c[d] - y * s[d];
      v[d + half] = y * c[d] + x * s[d];
    }
  } else if (mode == 2) {
    for (int d = 0; d < half; d++) {
      double x = v[2 * d], y = v[2 * d + 1];
      v[2 * d] = x * c[d] - y * s[d];
      v[2 * d + 1] = y * c[d] + x * s[d];
    }
  }
}

/* Decode oracle — fa_decode_gate.inc:66-96. leftpad/rotary_pos may be NULL. */
void oracle_decode(const float* q, const float* Kc, const float* Vc, const int32_t* block_table,
                   const int32_t* ctx_len, const float* new_k, const float* new_v,
                   const float* cos_t, const float* sin_t, const int32_t* leftpad,
                   const int32_t* rotary_pos, float* o, float* lse, const OracleDecCfg* c) {
  const int gqa = c->H / c->Hk;
  const int rdim = c->rdim > 0 ? c->rdim : c->D;
#pragma omp parallel for collapse(3) schedule(dynamic)
  for (int b = 0; b < c->B; b++)
    for (int tk = 0; tk < c->nq; tk++)
      for (int h = 0; h < c->H; h++) {
        const int kvh = h / gqa;
        const int ctx = ctx_len[b];
        const int qpos = ctx + tk;
        const int rp = (rotary_pos ? rotary_pos[b] : ctx) + tk;
        const int cend = ctx + (c->append ? tk + 1 : 0);
        int lo = 0;
        if (c->window >= 0 && qpos - c->window + 1 > lo) lo = qpos - c->window + 1;
        if (leftpad && leftpad[b] > lo) lo = leftpad[b];
        double* qr = (double*)malloc(sizeof(double) * c->D);
        double* kk = (double*)malloc(sizeof(double) * c->D);
        double* pr = (double*)malloc(sizeof(double) * (size_t)(cend > 0 ? cend : 1));
        const float* qs = q + (((size_t)b * c->nq + tk) * c->H + h) * c->D;
        for (int d = 0; d < c->D; d++) qr[d] = qs[d];
        if (c->rotary) rot_at(qr, rdim, cos_t, sin_t, c->rotary, rp);
        double mx = -INFINITY;
        for (int pos = 0; pos < cend; pos++) {
          pr[pos] = -INFINITY;
          if (pos < lo) continue;
          if (c->append && pos >= ctx) {
            const float* nk = new_k + (((size_t)b * c->nq + (pos - ctx)) * c->Hk + kvh) * c->D;
            for (int d = 0; d < c->D; d++) kk[d] = nk[d];
            if (c->rotary) rot_at(kk, rdim, cos_t, sin_t, c->rotary, rp - tk + (pos - ctx));
            /* the cache stores the rotated key in its dtype before attention reads it
               (fa_decode.hip:298-300, fd_append) */
            if (c->round_append == 1)
              for (int d = 0; d < c->D; d++) kk[d] = round_f16((float)kk[d]);
            else if (c->round_append == 2)
              for (int d = 0; d < c->D; d++) kk[d] = round_bf16((float)kk[d]);
          } else {
            const int blk = block_table[(size_t)b * c->max_blocks + pos / c->page];
            const float* kp = Kc + (((size_t)blk * c->page + pos % c->page) * c->Hk + kvh) * c->D;
            for (int d = 0; d < c->D; d++) kk[d] = kp[d];
          }
          double s = 0.0;
          for (int d = 0; d < c->D; d++) s += qr[d] * kk[d];
          s *= c->scale;
          if (c->softcap > 0) s = c->softcap * tanh(s / c->softcap);
          if (c->alibi) s += (double)c->alibi[h] * (double)(pos - qpos);
          pr[pos] = s;
          if (s > mx) mx = s;
        }
        double sum = 0.0;
        for (int pos = 0; pos < cend; pos++) {
          if (pr[pos] == -INFINITY) { pr[pos] = 0.0; continue; }
          pr[pos] = exp(pr[pos] - mx);
          sum += pr[pos];
        }
        float* os = o + (((size_t)b * c->nq + tk) * c->H + h) * c->D;
        for (int d = 0; d < c->D; d++) {
          double acc = 0.0;
          for (int pos = 0; pos < cend; pos++) {
            if (pr[pos] == 0.0) continue;
            float vv;
            if (c->append && pos >= ctx)
              vv = new_v[(((size_t)b * c->nq + (pos - ctx)) * c->Hk + kvh) * c->D + d];
            else {
              const int blk = block_table[(size_t)b * c->max_blocks + pos / c->page];
              vv = Vc[(((size_t)blk * c->page + pos % c->page) * c->Hk + kvh) * c->D + d];
            }
            acc += pr[pos] * (double)vv;
          }
          os[d] = (float)(sum > 0 ? acc / sum : 0.0);
        }
        if (lse) lse[((size_t)b * c->nq + tk) * c->H + h] = sum > 0 ? (float)(mx + log(sum)) : -INFINITY;
        free(qr);
        free(kk);
        free(pr);
      }
}

/* exported for tests: y[i] = round(x[i]) to fp16 (mode 1) or bf16 (mode 2) */
void oracle_round(const float* x, float* y, size_t n, int mode) {
  for (size_t i = 0; i < n; i++) y[i] = mode == 1 ? round_f16(x[i]) : mode == 2 ? round_bf16(x[i]) : x[i];
}

/* rel_rms — fa_common.hpp:136-139 (||got-ref||_2 / ||ref||_2) */
double oracle_rel_rms(const float* got, const float* ref, size_t n) {
  double e = 0, r = 0;
  for (size_t i = 0; i < n; i++) {
    double d = (double)got[i] - ref[i];
    e += d * d;
    r += (double)ref[i] * ref[i];
  }
  return r > 0 ? sqrt(e / r) : sqrt(e);
}
