// fwd.hip — exact attention forward for gfx950 (MI355X), fp16 and bf16.
//
// Replaces the reference forward (kernels/fa_forward.hip:52-313 kernel, :424-451 launcher);
// same math and masking contract (FwdParams in include/fable_attn_abi.h), new design:
//
//  * workgroup = NW waves; wave w owns 32 query rows, so a workgroup covers BR = 32*NW rows of
//    one (batch, head). Q for those rows lives in registers for the whole kernel, laid out as
//    the B operand of v_mfma_f32_32x32x16 (lane l holds query l%32, 8 head-dim values).
//  * scores are computed transposed, S^T = K . Q^T (A = K rows from LDS), so each lane holds
//    one query and BC/2 of its keys: the row max needs a single cross-half exchange
//    (v_permlane32_swap) and the probabilities P^T are already laid out as the B operand of
//    O^T = V^T . P^T. P never touches LDS.
//  * K and V tiles of BC keys are double-buffered in LDS with one barrier per tile, both
//    row-major with a 16-byte-chunk XOR swizzle. V^T, the A operand of the PV product, comes
//    from transposing LDS reads (ds_read_b64_tr_b16), so nothing is transposed on the way in.
//  * tile loads go through buffer descriptors (rows past the sequence end read as zeros), so
//    they carry no per-lane condition and the prefetch of tile t+1 stays in flight during
//    tile t.
//  * online softmax in the log2 domain (one FMA + v_exp_f32 per score); rescaling of the O
//    accumulator is skipped when no lane's running max moved.
//  * tiles entirely outside the causal / window / chunk range are never loaded; masking code
//    runs only on tiles that straddle a boundary (template CAUSAL/FEAT split as in the
//    reference's launch_cfg, fa_forward.hip:409-421).
//  * the workgroup -> (q tile, head, batch) map is XCD-aware (consecutive work items of one
//    head share an XCD's L2) and, for causal, starts with the heaviest q tiles.
#include "attn_device.hpp"
#include "status.hpp"

namespace fa {

template <int HD_, int BC_, int NW_, int WPE_>
struct FwdCfg {
  static constexpr int HD = HD_, BC = BC_, NW = NW_, WPE = WPE_;
  static constexpr int NT = NW * 64;
  static constexpr int BR = NW * 32;
  static constexpr int NB = BC / 32;        // 32-key blocks per tile
  static constexpr int NG = BC / 16;        // 16-key groups per tile (PV contraction steps)
  static constexpr int NDS = HD / 16;       // Q.K contraction steps
  static constexpr int NDB = HD / 32;       // 32-row blocks of O^T
  static constexpr int DCH = HD / 8;        // 16-byte chunks per K/V row
  static constexpr int KSW = DCH < 16 ? DCH : 16;
  static constexpr int KCH = BC * DCH;      // chunks per K (or V) tile
  static constexpr int PER = 2 * KCH / NT;  // chunks each thread loads per tile (K and V)
  static constexpr int KT = BC * HD;        // elements per K (or V) tile
  static constexpr int STAGE = 2 * KT;
  static_assert(HD % 32 == 0 && BC % 32 == 0, "shape");
  static_assert((2 * KCH) % NT == 0 && KCH % NT == 0, "loader split");
};

struct SeqView {
  int SQ, SK;
  long long q0, k0, v0, o0;  // element offsets of row 0 of this sequence (batch folded in)
  long long lse0;            // element offset of row 0 in LSE
};

// visible key range [k0, k1) for query rows [r0, r1] (reference mask contract)
template <bool CAUSAL, bool FEAT>
__device__ __forceinline__ void key_range(const FwdParams& p, int r0, int r1, int delta, int SK,
                                          int& k0, int& k1) {
  k0 = 0;
  k1 = SK;
  if (CAUSAL) k1 = min(k1, r1 + delta + 1);
  if (FEAT) {
    if (p.win_left >= 0) k0 = max(k0, r0 + delta - p.win_left);
    if (p.win_right >= 0) k1 = min(k1, r1 + delta + p.win_right + 1);
    if (p.attn_chunk > 0) {
      const int a = max(r0 + delta, 0), b = max(r1 + delta, 0);
      k0 = max(k0, (a / p.attn_chunk) * p.attn_chunk);
      k1 = min(k1, (b / p.attn_chunk + 1) * p.attn_chunk);
    }
  }
}

template <typename T, class C, bool CAUSAL, bool FEAT>
__global__ __attribute__((amdgpu_flat_work_group_size(C::NT, C::NT),
                          amdgpu_waves_per_eu(C::WPE, C::WPE))) void
fwd_kernel(FwdParams p, int nqt) {
  using V8 = typename Dt<T>::V8;
  using V4 = typename Dt<T>::V4;
  __shared__ __attribute__((aligned(16))) T lds[2 * C::STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5, j16 = lane & 15, mh = (lane >> 4) & 1;

  // ---- work item -> (sequence z, head h, q tile)
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const int qti = w % nqt, zh = w / nqt;
  const int h = zh % p.NH, z = zh / p.NH;
  const int qt = CAUSAL ? (nqt - 1 - qti) : qti;
  const int kvh = h / p.gqa;

  SeqView sv;
  if (p.cu_q) {
    const int qs = p.cu_q[z], ks = p.cu_k[z];
    sv.SQ = p.cu_q[z + 1] - qs;
    sv.SK = p.cu_k[z + 1] - ks;
    if (p.seqused_q) sv.SQ = min(sv.SQ, p.seqused_q[z]);
    if (p.seqused_k) sv.SK = min(sv.SK, p.seqused_k[z]);
    sv.q0 = (long long)qs * p.sQ.s;
    sv.k0 = (long long)ks * p.sK.s;
    sv.v0 = (long long)ks * p.sV.s;
    sv.o0 = (long long)qs * p.sO.s;
    sv.lse0 = (long long)h * p.lse_sh + qs;
  } else {
    sv.SQ = p.SQ;
    sv.SK = p.SK;
    sv.q0 = (long long)z * p.sQ.b;
    sv.k0 = (long long)z * p.sK.b;
    sv.v0 = (long long)z * p.sV.b;
    sv.o0 = (long long)z * p.sO.b;
    sv.lse0 = (long long)z * p.lse_sb + (long long)h * p.lse_sh;
  }
  const int SQ = sv.SQ, SK = sv.SK;
  const int qb = qt * C::BR;
  if (qb >= SQ) return;
  const int delta = SK - SQ;

  const T* Qg = (const T*)p.Q + sv.q0 + (long long)h * p.sQ.h;
  const T* Kg = (const T*)p.K + sv.k0 + (long long)kvh * p.sK.h;
  const T* Vg = (const T*)p.V + sv.v0 + (long long)kvh * p.sV.h;
  T* Og = (T*)p.O + sv.o0 + (long long)h * p.sO.h;

  // ---- block and wave key ranges
  int bk0, bk1;
  key_range<CAUSAL, FEAT>(p, qb, min(qb + C::BR, SQ) - 1, delta, SK, bk0, bk1);
  const int qw = qb + wave * 32;
  const bool wave_rows = qw < SQ;
  int wk0 = 0, wk1 = 0;
  if (wave_rows) key_range<CAUSAL, FEAT>(p, qw, min(qw + 32, SQ) - 1, delta, SK, wk0, wk1);
  const int kstart = (bk0 / C::BC) * C::BC;
  const int ntiles = bk1 > bk0 ? (bk1 - kstart + C::BC - 1) / C::BC : 0;

  // ---- Q (B operand) in registers
  const int qi = qw + l32;
  V8 qreg[C::NDS];
#pragma unroll
  for (int ds = 0; ds < C::NDS; ds++) {
    if (qi < SQ)
      qreg[ds] = *(const V8*)(Qg + (long long)qi * p.sQ.s + 16 * ds + 8 * hh);
    else
      qreg[ds] = bitcast<V8>(u32x4{0, 0, 0, 0});
  }

  f32x16 oacc[C::NDB];
#pragma unroll
  for (int db = 0; db < C::NDB; db++) oacc[db] = f32x16{};
  float m_run = -INFINITY, l_run = 0.0f;
  const float c_log2 = p.scale * kLog2e;
  const float aslope = (FEAT && p.alibi_slopes) ? p.alibi_slopes[h] : 0.0f;

  // ---- global -> register loads of one tile through buffer descriptors spanning rows
  // kb..SK-1 of this head: rows past the sequence end read as zeros without a per-lane
  // condition (a conditional load would make the compiler wait for it at once), and the
  // per-lane byte offsets are loop invariant. The first KJ chunks of each thread are K.
  constexpr int KJ = C::KCH / C::NT;
  int voff[C::PER];
#pragma unroll
  for (int j = 0; j < C::PER; j++) {
    const bool isv = j >= KJ;
    const int ci = tid + (isv ? j - KJ : j) * C::NT;
    const int r = ci / C::DCH, c = ci % C::DCH;
    voff[j] = r * (int)((isv ? p.sV.s : p.sK.s) * 2) + 16 * c;
  }
  u32x4 ld[C::PER];
  auto gload = [&](int kb) {
    const auto rk = buf_rsrc(Kg + (long long)kb * p.sK.s, (long long)(SK - kb) * p.sK.s * 2);
    const auto rv = buf_rsrc(Vg + (long long)kb * p.sV.s, (long long)(SK - kb) * p.sV.s * 2);
#pragma unroll
    for (int j = 0; j < C::PER; j++) ld[j] = buf_load16(j >= KJ ? rv : rk, voff[j]);
  };
  auto lstore = [&](int stage) {
    T* base = lds + stage * C::STAGE;
#pragma unroll
    for (int j = 0; j < C::PER; j++) {
      const bool isv = j >= KJ;
      const int ci = tid + (isv ? j - KJ : j) * C::NT;
      const int r = ci / C::DCH, c = ci % C::DCH;
      *(u32x4*)(base + (isv ? C::KT : 0) + kofs(r, c, C::HD, C::KSW)) = ld[j];
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
    gload(kb + C::BC);  // past the last tile the descriptor is empty and the loads return zeros

    const bool active = wave_rows && kb < wk1 && kb + C::BC > wk0;
    if (active) {
      const T* ks = lds + stage * C::STAGE;
      const T* vt = ks + C::KT;
      // S^T = K . Q^T
      f32x16 s[C::NB];
#pragma unroll
      for (int jb = 0; jb < C::NB; jb++) s[jb] = f32x16{};
#pragma unroll
      for (int ds = 0; ds < C::NDS; ds++) {
#pragma unroll
        for (int jb = 0; jb < C::NB; jb++) {
          const int r = jb * 32 + l32;
          const V8 a = *(const V8*)(ks + kofs(r, 2 * ds + hh, C::HD, C::KSW));
          s[jb] = Dt<T>::mma32(a, qreg[ds], s[jb]);
        }
      }
      // logits (log2 domain for FEAT; raw dot products for the plain path) + masking
      const int kq = kb + 4 * hh;  // key of s[jb][r] = kq + jb*32 + 8*(r/4) + (r%4)
      if (FEAT) {
#pragma unroll
        for (int jb = 0; jb < C::NB; jb++)
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const int key = kq + jb * 32 + 8 * (r >> 2) + (r & 3);
            float x = s[jb][r] * p.scale;
            if (p.softcap > 0.0f) x = p.softcap * tanh_exp(x / p.softcap);
            x += aslope * (float)(key - qi);
            bool ok = key < SK;
            if (CAUSAL) ok = ok && key <= qi + delta;
            if (p.win_left >= 0) ok = ok && key >= qi + delta - p.win_left;
            if (p.win_right >= 0) ok = ok && key <= qi + delta + p.win_right;
            if (p.attn_chunk > 0) {
              const int cs = (max(qi + delta, 0) / p.attn_chunk) * p.attn_chunk;
              ok = ok && key >= cs && key < cs + p.attn_chunk;
            }
            s[jb][r] = ok ? x * kLog2e : -INFINITY;
          }
      } else {
        const bool edge = CAUSAL ? (kb + C::BC - 1 > qw + delta) : (kb + C::BC > SK);
        if (edge) {
#pragma unroll
          for (int jb = 0; jb < C::NB; jb++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
              const int key = kq + jb * 32 + 8 * (r >> 2) + (r & 3);
              const bool ok = CAUSAL ? key <= qi + delta : key < SK;
              if (!ok) s[jb][r] = -INFINITY;
            }
        }
      }
      // online softmax
      float mx = -INFINITY;
#pragma unroll
      for (int jb = 0; jb < C::NB; jb++)
#pragma unroll
        for (int r = 0; r < 16; r++) mx = fmaxf(mx, s[jb][r]);
      mx = half_max(mx);
      const float m_new = fmaxf(m_run, FEAT ? mx : mx * c_log2);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float corr = exp2_fast(m_run - m_use);
      float rs = 0.0f;
#pragma unroll
      for (int jb = 0; jb < C::NB; jb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const float e = FEAT ? exp2_fast(s[jb][r] - m_use) : exp2_fast(fmaf(s[jb][r], c_log2, -m_use));
          s[jb][r] = e;
          rs += e;
        }
      l_run = l_run * corr + rs;
      m_run = m_new;
      if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {
#pragma unroll
        for (int db = 0; db < C::NDB; db++) oacc[db] *= corr;
      }
      // P^T as B operands: group g = 2*jb + half covers accumulators 8*half .. 8*half+7
      V8 pb[C::NG];
#pragma unroll
      for (int jb = 0; jb < C::NB; jb++)
#pragma unroll
        for (int sh = 0; sh < 2; sh++)
#pragma unroll
          for (int e = 0; e < 8; e++) pb[2 * jb + sh][e] = (T)s[jb][8 * sh + e];
      // O^T += V^T . P^T. A operand by transposing reads: lane j16 of 16-lane group (mh, hh)
      // addresses key row 16g+8a+4hh+j16/4, head-dim 32db+16mh+4*(j16%4) and receives head-dim
      // 32db+16mh+j16 of keys 16g+8a+4hh+0..3 (the keys of its P^T items 4a..4a+3).
#pragma unroll
      for (int db = 0; db < C::NDB; db++) {
        const int col = 32 * db + 16 * mh + 4 * (j16 & 3);
#pragma unroll
        for (int g = 0; g < C::NG; g++) {
          V4 part[2];
#pragma unroll
          for (int a = 0; a < 2; a++) {
            const int row = 16 * g + 8 * a + 4 * hh + (j16 >> 2);
            part[a] = lds_read_tr<T>(vt + kofs(row, col >> 3, C::HD, C::KSW) + (col & 7));
          }
          V8 av;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            av[e] = part[0][e];
            av[4 + e] = part[1][e];
          }
          oacc[db] = Dt<T>::mma32(av, pb[g], oacc[db]);
        }
      }
    }
    lstore(stage ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O = acc / l, LSE
  const float l_tot = half_sum(l_run);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (qi < SQ) {
    T* orow = Og + (long long)qi * p.sO.s;
#pragma unroll
    for (int db = 0; db < C::NDB; db++)
#pragma unroll
      for (int rq = 0; rq < 4; rq++) {
        V4 v;
#pragma unroll
        for (int c = 0; c < 4; c++) v[c] = (T)(oacc[db][4 * rq + c] * inv);
        *(V4*)(orow + db * 32 + 8 * rq + 4 * hh) = v;
      }
    if (p.LSE && hh == 0)
      p.LSE[sv.lse0 + qi] = l_tot > 0.0f ? m_run * kLn2 + __logf(l_tot) : -INFINITY;
  }
}

template <typename T, class C>
static int launch_fwd(const FwdParams& p, hipStream_t st) {
  const int nqt = (p.SQ + C::BR - 1) / C::BR;
  const long long nblk = (long long)nqt * p.NH * p.batch;
  if (nblk <= 0) return FA_OK;
  if (nblk > 0x7FFFFFFF) return fail(FA_ERR_ARG, "fa_forward_launch: grid too large");
  const bool feat = p.softcap > 0.0f || p.alibi_slopes != nullptr || p.attn_chunk > 0 ||
                    p.win_left >= 0 || (p.win_right >= 0 && !(p.win_right == 0 && p.causal));
  dim3 grid((unsigned)nblk), block(C::NT);
  if (p.causal) {
    if (feat)
      hipLaunchKernelGGL((fwd_kernel<T, C, true, true>), grid, block, 0, st, p, nqt);
    else
      hipLaunchKernelGGL((fwd_kernel<T, C, true, false>), grid, block, 0, st, p, nqt);
  } else {
    if (feat)
      hipLaunchKernelGGL((fwd_kernel<T, C, false, true>), grid, block, 0, st, p, nqt);
    else
      hipLaunchKernelGGL((fwd_kernel<T, C, false, false>), grid, block, 0, st, p, nqt);
  }
  return launch_status("fa_forward_launch");
}

template <typename T>
static int dispatch_hd(const FwdParams& p, hipStream_t st) {
  switch (p.HD) {
    case 64: return launch_fwd<T, FwdCfg<64, 64, 4, 2>>(p, st);
    case 128: return launch_fwd<T, FwdCfg<128, 64, 8, 2>>(p, st);
    case 256: return launch_fwd<T, FwdCfg<256, 32, 4, 1>>(p, st);
    default: return fail(FA_ERR_HEADDIM, "fa_forward_launch: head_dim=%d has no kernel (64, 128, 256)", p.HD);
  }
}

}  // namespace fa

extern "C" int fa_forward_launch(FwdParams p, int dtype, void* stream) {
  using namespace fa;
  if (!p.Q || !p.K || !p.V || !p.O) return fail(FA_ERR_ARG, "fa_forward_launch: null tensor pointer");
  if (p.NH <= 0 || p.gqa <= 0 || p.NH % p.gqa) return fail(FA_ERR_ARG, "fa_forward_launch: NH=%d gqa=%d", p.NH, p.gqa);
  if (p.dropout_p > 0.0f) return fail(FA_ERR_UNSUPPORTED, "fa_forward_launch: dropout is not implemented");
  if ((p.cu_q == nullptr) != (p.cu_k == nullptr)) return fail(FA_ERR_ARG, "fa_forward_launch: cu_q and cu_k go together");
  if (!p.cu_q && p.batch <= 0) return FA_OK;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case FA_F16: return dispatch_hd<_Float16>(p, st);
    case FA_BF16: return dispatch_hd<__bf16>(p, st);
    default: return fail(FA_ERR_DTYPE, "fa_forward_launch: dtype %d not implemented (fp16/bf16)", dtype);
  }
}
