// decode.hip — paged-KV split-KV decode for gfx950: KV append, partial attention per split,
// LSE-weighted combine.
//
// Replaces the reference decode (kernels/fa_decode.hip: fd_partial :57-252, fd_combine
// :255-272, fd_append :275-302, launcher :319-362) with the same FableDecParams contract
// (include/fable_attn_abi.h) and a different design:
//  * one workgroup (4 waves) per (kv head, 16-head group, sequence*new token, split); the q
//    heads sharing the kv head are packed into the N=16 dimension of v_mfma_f32_16x16x32, so
//    K and V are read from HBM once per kv head whatever the GQA ratio;
//  * K and V rows are read from the paged cache in whole rows (consecutive lanes cover one
//    row) and staged per wave in LDS; S^T = K . Q^T reads its A operand (16 bytes of one key
//    row per lane) back from the K slice, and the 16x16 result leaves every lane with one head
//    and four keys;
//  * P^T is the B operand of O^T = V^T . P^T (v_mfma_f32_16x16x16) without leaving registers;
//    V is read back from its slice transposed with ds_read_b64_tr_b16;
//  * each wave streams its own 16-key chunks (fp32: 32-key) with no barriers in the loop; the
//    four waves merge in LDS at the end and write one (max, sum, acc[HD]) partial per head and
//    split;
//  * the combine kernel merges the splits (natural-log LSE optional);
//  * appending new_k/new_v (with rotary on k) is a kernel earlier in the same stream: the
//    reference's hipDeviceSynchronize() after the append (fa_decode.hip:348-351) is gone.
// Scores are handled in the log2 domain; partial maxima are stored in log2 units.
#include <mutex>
#include <type_traits>

#include "attn_device.hpp"
#include "status.hpp"

namespace fa {

static int dec_checked(FableDecParams p, int dtype, void* stream, const void* new_k, const void* new_v);

constexpr int kDecChunk = 32;  // keys per wave iteration of the fp32 kernel; splits are multiples
constexpr int kDecKeys = 16;   // keys per wave iteration of the fp16/bf16 kernel
constexpr int kDecWaves = 4;
static_assert(kDecKeys <= 16, "a chunk spans at most two pages of >= 16 rows (SPT)");

__device__ __forceinline__ float xor16_max(float x) {
  return fmaxf(x, __shfl_xor(x, 16));
}
__device__ __forceinline__ float xor16_sum(float x) { return x + __shfl_xor(x, 16); }

struct DecRange {
  int qpos, hi, lo, start, end;
};

__device__ __forceinline__ DecRange dec_range(const FableDecParams& p, int b, int tk, int sp, int append) {
  DecRange r;
  const int ctx = p.ctx_len[b];
  r.qpos = ctx + tk;
  r.hi = min(ctx + (append ? tk + 1 : 0), p.max_blocks * p.page);
  int lo = p.leftpad ? p.leftpad[b] : 0;
  if (p.window >= 0) lo = max(lo, r.qpos - p.window + 1);
  r.lo = max(lo, 0);
  const int n = max(r.hi - r.lo, 0);
  const int chunk = (((n + p.nsplit - 1) / p.nsplit) + kDecChunk - 1) / kDecChunk * kDecChunk;
  r.start = r.lo + sp * chunk;
  r.end = min(r.start + chunk, r.hi);
  return r;
}

// SPT (page >= 16): the block-table entries of a chunk are fetched by scalar loads. A chunk of
// 16 keys touches at most two pages then, and each lane selects its row's entry from the two.
// Per-lane table loads share the in-order vector-memory counter with the row loads, so a wave
// waiting for its next entries also waited for the rows issued before them (the chunk in
// flight): C4 +1% with the scalar loads (+4% in a read probe). Smaller pages (a dense cache of
// fewer than 16 rows) keep per-lane loads.
// flags: bit 0 new keys were appended (kDecAppend), bit 1 the kernel writes the final output and
// LSE itself (kDecFinal: one split, no combine launch)
constexpr int kDecAppend = 1, kDecFinal = 2;
template <typename T, int HD, bool FEAT, bool SPT>
__global__ __launch_bounds__(256) void dec_partial_kernel(FableDecParams p, int page_shift, int ngrp, int flags) {
  const int append = flags & kDecAppend;
  using V8 = typename Dt<T>::V8;
  constexpr int NDS = HD / 32;  // S^T contraction steps
  constexpr int NDB = HD / 16;  // 16-row blocks of O^T
  constexpr int RCH = HD / 8;   // 16-byte chunks per key row
  static_assert(RCH >= 8, "swizzle needs >= 8 chunks per row");
  // one LDS region, reused: q staging (fp32) before the loop, per-wave V chunks in the loop,
  // the four waves' accumulators after it; per-wave K chunks in a region of their own
  __shared__ __attribute__((aligned(16))) char vraw[kDecWaves * 16 * HD * 4];
  __shared__ __attribute__((aligned(16))) char kraw[kDecWaves * kDecKeys * HD * 2];
  __shared__ float red_m[kDecWaves][16], red_l[kDecWaves][16];
  static_assert(16 * HD * 4 <= sizeof(vraw), "q staging fits the V region");
  static_assert(kDecWaves * kDecKeys * HD * 2 <= sizeof(vraw), "the V slices fit the V region");
  float (*qsh)[HD] = (float (*)[HD])vraw;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lg = lane >> 4, lh = lane & 15;  // lane group (0..3), lane in group
  // grid x = (kv head, head group) fastest: the workgroups reading the interleaved heads of the
  // same cache pages are dispatched together
  const int b = blockIdx.y / p.nq, tk = blockIdx.y % p.nq;
  const int kvh = blockIdx.x / ngrp, hgi = blockIdx.x % ngrp;
  const int h0 = kvh * p.gqa + 16 * hgi, hg = min(16, p.gqa - 16 * hgi);
  const int sp = blockIdx.z;
  const int NKV = p.NH / p.gqa;
  const DecRange rg = dec_range(p, b, tk, sp, append);

  // ---- q rows of this head group -> LDS (fp32): one 16-byte load per thread and chunk,
  // head index clamped (rows past the group are zeroed after the load)
  // A head dim HDr = p.HD below the kernel width HD (a multiple of 8) runs with zero columns
  // HDr..HD-1 in q, K and V (rows in memory are HDr long); only HDr output columns are kept.
  const int HDr = p.HD;
  const T* qg = (const T*)p.q + ((long long)(b * p.nq + tk) * p.NH + h0) * HDr;
  for (int i = tid; i < 16 * RCH; i += 256) {
    const int g = i / RCH, c = i % RCH;
    const bool cok = 8 * c < HDr;
    const u32x4 raw = *(const u32x4*)(qg + (long long)min(g, hg - 1) * HDr + (cok ? 8 * c : 0));
    const V8 v = bitcast<V8>(raw);
#pragma unroll
    for (int e = 0; e < 8; e++) qsh[g][8 * c + e] = g < hg && cok ? (float)v[e] : 0.0f;
  }
  __syncthreads();
  if (p.rotary) {
    const int rdim = p.rotary_dim > 0 ? p.rotary_dim : HDr, half = rdim / 2;
    const int rp = (p.rotary_pos ? p.rotary_pos[b] : p.ctx_len[b]) + tk;
    for (int i = tid; i < hg * half; i += 256) {
      const int g = i / half, j = i % half;
      const float c = p.cos[(long long)rp * half + j], s = p.sin[(long long)rp * half + j];
      const int ia = p.rotary == 1 ? j : 2 * j, ib = p.rotary == 1 ? j + half : 2 * j + 1;
      const float x = qsh[g][ia], y = qsh[g][ib];
      qsh[g][ia] = x * c - y * s;
      qsh[g][ib] = y * c + x * s;
    }
    __syncthreads();
  }
  // Q^T as the B operand: lane holds head lh, head-dim 32*ds + 8*lg + e. A rotated q is not
  // representable in T; it is carried as hi + lo (two MFMAs per step) so rotation costs no
  // precision beyond fp32.
  const bool qsplit = p.rotary != 0;
  V8 qb[NDS], ql[NDS];
#pragma unroll
  for (int ds = 0; ds < NDS; ds++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float x = qsh[lh][32 * ds + 8 * lg + e];
      const T hi = (T)x;
      qb[ds][e] = hi;
      ql[ds][e] = (T)(x - (float)hi);
    }
  __syncthreads();  // q staging is dead from here on: the region becomes the V chunk buffers

  f32x4 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; db++) oacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  const float c_log2 = p.scale * kLog2e;
  const float slope = (FEAT && p.alibi && lh < hg) ? p.alibi[h0 + lh] : 0.0f;
  const T* Kc = (const T*)p.Kc;
  const T* Vc = (const T*)p.Vc;
  const int* bt = p.block_table + (long long)b * p.max_blocks;
  const int pmask = p.page - 1;
  T* vb = (T*)vraw + wave * kDecKeys * HD;
  T* kbuf = (T*)kraw + wave * kDecKeys * HD;

  // Keys of a chunk are clamped into [start, end-1] (masked in the softmax), so every load is
  // unconditional. Block-table entries are fetched ahead of the row loads that use them, so the
  // K/V row loads of a chunk issue back to back instead of behind their table lookups.
  constexpr int NVI = kDecKeys * RCH / 64;  // K (and V) row loads per lane per chunk
  const int last = rg.end - 1;
  auto vkey = [&](int kc0, int i) { return min(kc0 + (64 * i + lane) / RCH, last); };
  int vblk[SPT ? 1 : NVI], sblk[2];
  auto table = [&](int kc0) {
    if constexpr (SPT) {
      const int b0 = kc0 >> page_shift, bl = last >> page_shift;  // wave-uniform
#pragma unroll
      for (int j = 0; j < 2; j++) sblk[j] = bt[min(b0 + j, bl)];
    } else {
#pragma unroll
      for (int i = 0; i < NVI; i++) vblk[i] = bt[vkey(kc0, i) >> page_shift];
    }
  };
  // entry of load i's row: page (key >> page_shift) - (kc0 >> page_shift) of the chunk's two
  // (a key clamped to `last` lies in the chunk's last page, whose index the table clamped too)
  auto blk_of = [&](int kc0, int i) {
    if constexpr (SPT) {
      const int j = (vkey(kc0, i) >> page_shift) - (kc0 >> page_shift);
      return j <= 0 ? sblk[0] : sblk[1];
    } else {
      return vblk[i];
    }
  };
  auto row_off = [&](int blk, int key) -> long long {
    return (((long long)blk * p.page + (key & pmask)) * NKV + kvh) * HDr;
  };
  // 16-byte chunks in the zero columns load the row's first chunk and are replaced by zeros
  const bool padded = HDr < HD;
  bool vok[NVI];
#pragma unroll
  for (int i = 0; i < NVI; i++) vok[i] = 8 * ((64 * i + lane) % RCH) < HDr;
  // K/V rows of the chunk at kc0: load i covers row (64i + lane) / RCH, 16-byte chunk
  // (64i + lane) % RCH of both caches, so consecutive lanes read whole rows. Loading K straight
  // into the MFMA A layout instead (16 keys x 64 bytes per load) read the cache ~12% slower.
  // The cache rows are read once per step: non-temporal loads keep them from displacing the
  // block table and q in the caches (C4: 368.6 -> 360.3 us for the partial kernel).
  auto load = [&](int kc0, u32x4 (&kr)[NVI], u32x4 (&vr)[NVI]) {
#pragma unroll
    for (int i = 0; i < NVI; i++) {
      const int ch = (64 * i + lane) % RCH;
      const long long off = row_off(blk_of(kc0, i), vkey(kc0, i)) + (vok[i] ? 8 * ch : 0);
      kr[i] = __builtin_nontemporal_load((const u32x4*)(Kc + off));
      vr[i] = __builtin_nontemporal_load((const u32x4*)(Vc + off));
    }
  };
  // zero columns of a padded head dim, put in where the rows are used (which waits for the
  // loads anyway; a select right after the loads would make the compiler wait there)
  auto zero_pad = [&](u32x4 (&kr)[NVI], u32x4 (&vr)[NVI]) {
    if (padded) {
#pragma unroll
      for (int i = 0; i < NVI; i++) {
        kr[i] = vok[i] ? kr[i] : u32x4{0, 0, 0, 0};
        vr[i] = vok[i] ? vr[i] : u32x4{0, 0, 0, 0};
      }
    }
  };
  // K slice: row r holds logical 16-byte chunk c at physical chunk c ^ kswz(r). The rows of
  // one 256-byte bank line share a pattern and consecutive lines differ, so the 16 lanes of an
  // A-operand read (16 rows, one chunk) and of a row write hit 16 different bank groups.
  // (A width whose chunk count is not a power of two XORs within aligned groups of the largest
  // power of two that divides it, so a chunk never leaves its row: 12 chunks at width 96 swizzle
  // in groups of 4.)
  constexpr int kRowsPerLine = HD >= 128 ? 1 : 128 / HD;
  constexpr int kSwzGroup = (RCH & -RCH) < 16 ? (RCH & -RCH) : 16;
  constexpr int kSwzMask = kSwzGroup - 1;
  auto kswz = [](int r) { return (r / kRowsPerLine) & kSwzMask; };
  // V slice: chunk c of row r at c ^ vswz(r), pairs of chunks for the transposing reads
  auto vswz = [](int r) { return kSwzGroup >= 8 ? 2 * (r & 3) : 2 * (r & 1); };
  // Each wave walks 16-key chunks with one register set: a chunk's rows go to LDS, the next
  // chunk's loads are issued, and the chunk is computed from LDS meanwhile. Table entries run
  // one chunk ahead. Keys past the end clamp to the last one. Read probes over the C4 cache
  // streamed fastest with about 8 KiB of rows in flight per wave (16 keys of K and V at
  // D=128); 32-key chunks with a second register set in flight read ~6% slower there.
  constexpr int kStep = kDecKeys * kDecWaves;
  const int kfirst = rg.start + kDecKeys * wave;
  u32x4 kreg[NVI], vreg[NVI];
  if (kfirst < rg.end) {
    table(kfirst);
    load(kfirst, kreg, vreg);
    table(kfirst + kStep);
  }
  for (int kc0 = kfirst; kc0 < rg.end; kc0 += kStep) {
    zero_pad(kreg, vreg);
    // K and V -> this wave's LDS slices; the slices are the wave's own, and LDS operations of
    // one wave complete in order, so no barrier orders these writes against the reads below or
    // against the previous chunk's reads
#pragma unroll
    for (int i = 0; i < NVI; i++) {
      const int row = (64 * i + lane) / RCH, ch = (64 * i + lane) % RCH;
      *(u32x4*)(kbuf + row * HD + 8 * (ch ^ kswz(row))) = kreg[i];
      *(u32x4*)(vb + row * HD + 8 * (ch ^ vswz(row))) = vreg[i];
    }
    // the next chunk's rows are in flight during this chunk's products
    if (kc0 + kStep < rg.end) {
      load(kc0 + kStep, kreg, vreg);
      table(kc0 + 2 * kStep);
    }
    // S^T = K . Q^T, A operand: lane (lg, lh) reads key row lh, head-dim chunk 4*ds + lg
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
    {
      V8 ka[NDS];
#pragma unroll
      for (int ds = 0; ds < NDS; ds++) ka[ds] = bitcast<V8>(*(const u32x4*)(kbuf + lh * HD + 8 * ((4 * ds + lg) ^ kswz(lh))));
#pragma unroll
      for (int ds = 0; ds < NDS; ds++) s = Dt<T>::mma16(ka[ds], qb[ds], s);
      if (qsplit) {
#pragma unroll
        for (int ds = 0; ds < NDS; ds++) s = Dt<T>::mma16(ka[ds], ql[ds], s);
      }
    }
    // logits (log2 domain) and masking: s[r] is key kc0 + 4*lg + r, head lh
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int key = kc0 + 4 * lg + r;
      float t;
      if (FEAT) {
        float x = s[r] * p.scale;
        if (p.softcap > 0.0f) x = p.softcap * tanh_exp(x / p.softcap);
        x += slope * (float)(key - rg.qpos);
        t = x * kLog2e;
      } else {
        t = s[r] * c_log2;
      }
      t = key < rg.end ? t : -INFINITY;
      s[r] = t;
      mx = fmaxf(mx, t);
    }
    mx = half_max(xor16_max(mx));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float corr = exp2_fast(m_run - m_use);
    float rs = 0.0f;
    typename Dt<T>::V4 pb;  // P^T, the B operand of the k=16 product: keys 4*lg + r, head lh
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float e = exp2_fast(s[r] - m_use);
      rs += e;
      pb[r] = (T)e;
    }
    l_run = l_run * corr + rs;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < NDB; db++) oacc[db] *= corr;
    // O^T += V^T . P^T, A operand by transposing LDS reads: lane lh of group lg addresses row
    // 4*lg + lh/4, head-dim 16*db + 4*(lh%4); it receives V[4*lg + r][16*db + lh]
#pragma unroll
    for (int db = 0; db < NDB; db++) {
      const int row = 4 * lg + (lh >> 2);
      const int col = 16 * db + 4 * (lh & 3);
      const int off = row * HD + 8 * ((col >> 3) ^ vswz(row)) + (col & 7);
      typedef short s4 __attribute__((ext_vector_type(4)));
      const s4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s4*)((__attribute__((address_space(3))) T*)vb + off));
      oacc[db] = Dt<T>::mma16k16(bitcast<typename Dt<T>::V4>(t), pb, oacc[db]);
    }
  }

  // ---- merge the four waves: per head max, sum and O^T accumulators through LDS
  const float l_grp = half_sum(xor16_sum(l_run));
  __syncthreads();  // every wave is done with its V slice: reuse it for the accumulators
  float* red_o = (float*)vraw;  // [wave][16 heads][HD]
  if (lg == 0) {
    red_m[wave][lh] = m_run;
    red_l[wave][lh] = l_grp;
  }
#pragma unroll
  for (int db = 0; db < NDB; db++)
#pragma unroll
    for (int r = 0; r < 4; r++) red_o[(wave * 16 + lh) * HD + 16 * db + 4 * lg + r] = oacc[db][r];
  __syncthreads();
  const bool final_out = (flags & kDecFinal) != 0;
  for (int i = tid; i < hg * HDr; i += 256) {
    const int g = i / HDr, d = i % HDr;
    float gm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecWaves; w++) gm = fmaxf(gm, red_m[w][g]);
    float l = 0.0f, acc = 0.0f;
    if (gm != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kDecWaves; w++) {
        const float f = exp2_fast(red_m[w][g] - gm);
        l += f * red_l[w][g];
        acc += f * red_o[(w * 16 + g) * HD + d];
      }
    }
    if (final_out) {
      // what the combine kernel computes from one split (its weight exp2(0) is exactly 1)
      const long long row = (long long)(b * p.nq + tk) * p.NH + h0 + g;
      const bool ok = gm != -INFINITY && l > 0.0f;
      ((T*)p.o)[row * HDr + d] = (T)(ok ? acc / l : 0.0f);
      if (p.lse_out && d == 0) p.lse_out[row] = ok ? gm * kLn2 + __logf(l) : -INFINITY;
      continue;
    }
    float* out = p.scratch + (((long long)(b * p.nq + tk) * p.NH + h0 + g) * p.nsplit + sp) * (HDr + 2);
    if (d == 0) {
      out[0] = gm;
      out[1] = l;
    }
    out[2 + d] = acc;
  }
}

// fp32 caches (the reference's decode serves fp16/bf16/fp32, fa_decode.hip:4,360): the same
// workgroup and wave split, on v_mfma_f32_16x16x4_f32. Lane (head lh, group lg) holds q dims
// lg*HD/4 + t as the B operand of S^T = K . Q^T, whose A operand is loaded straight from the
// paged cache (16 bytes of one key row per lane); P^T is the B operand of O^T = V^T . P^T,
// whose A operand is one float per lane (V[key 16kb + 4lg + j][16db + lh]), read from the cache
// as well (four 64-byte row segments per load). Rotation of q stays exact in fp32. Kernel
// widths HD = 64, 128, 256 serve every head dim p.HD that is a multiple of 8: rows are p.HD
// floats apart and the partial record holds the p.HD real columns. Columns past p.HD are read
// at a clamped column of the same row (always in bounds, no branch): for K the product meets
// q columns that are zero there, and for V it only fills O^T rows past p.HD, which are never
// stored. (Per-load branches here raised the kernel's scalar registers past the file and the
// 256-wide alibi variant then computed wrong logits; the clamped form keeps the register use
// of the full-width kernel.)
template <int HD, bool FEAT>
__global__ __launch_bounds__(256) void dec_partial_f32_kernel(FableDecParams p, int page_shift, int ngrp, int append) {
  constexpr int NQ = HD / 4;    // S^T contraction steps (q floats per lane)
  constexpr int NDB = HD / 16;  // 16-row blocks of O^T
  constexpr int QSTR = HD + 4;
  constexpr int QBYTES = 16 * QSTR * 4, OBYTES = kDecWaves * 16 * HD * 4;
  __shared__ __attribute__((aligned(16))) char raw[QBYTES > OBYTES ? QBYTES : OBYTES];
  __shared__ float red_m[kDecWaves][16], red_l[kDecWaves][16];
  float (*qsh)[QSTR] = (float (*)[QSTR])raw;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lg = lane >> 4, lh = lane & 15;
  const int b = blockIdx.y / p.nq, tk = blockIdx.y % p.nq;
  const int kvh = blockIdx.x / ngrp, hgi = blockIdx.x % ngrp;
  const int h0 = kvh * p.gqa + 16 * hgi, hg = min(16, p.gqa - 16 * hgi);
  const int sp = blockIdx.z;
  const int NKV = p.NH / p.gqa, HDr = p.HD;
  const DecRange rg = dec_range(p, b, tk, sp, append);

  const float* qg = (const float*)p.q + ((long long)(b * p.nq + tk) * p.NH + h0) * HDr;
  for (int i = tid; i < 16 * NQ; i += 256) {
    const int g = i / NQ, c = i % NQ;
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    if (g < hg && 4 * c < HDr) v = *(const f32x4*)(qg + (long long)g * HDr + 4 * c);
#pragma unroll
    for (int e = 0; e < 4; e++) qsh[g][4 * c + e] = v[e];
  }
  __syncthreads();
  if (p.rotary) {
    const int rdim = p.rotary_dim > 0 ? p.rotary_dim : HDr, half = rdim / 2;
    const int rp = (p.rotary_pos ? p.rotary_pos[b] : p.ctx_len[b]) + tk;
    for (int i = tid; i < hg * half; i += 256) {
      const int g = i / half, j = i % half;
      const float c = p.cos[(long long)rp * half + j], s = p.sin[(long long)rp * half + j];
      const int ia = p.rotary == 1 ? j : 2 * j, ib = p.rotary == 1 ? j + half : 2 * j + 1;
      const float x = qsh[g][ia], y = qsh[g][ib];
      qsh[g][ia] = x * c - y * s;
      qsh[g][ib] = y * c + x * s;
    }
    __syncthreads();
  }
  float qreg[NQ];
#pragma unroll
  for (int t = 0; t < NQ; t++) qreg[t] = qsh[lh][lg * NQ + t];

  f32x4 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; db++) oacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  const float c_log2 = p.scale * kLog2e;
  const float slope = (FEAT && p.alibi && lh < hg) ? p.alibi[h0 + lh] : 0.0f;
  const float inv_cap = p.softcap > 0.0f ? 1.0f / p.softcap : 0.0f;
  const float* Kc = (const float*)p.Kc;
  const float* Vc = (const float*)p.Vc;
  const int* bt = p.block_table + (long long)b * p.max_blocks;
  const int pmask = p.page - 1;
  const int last = rg.end - 1;
  auto row_off = [&](int key) -> long long {
    return (((long long)bt[key >> page_shift] * p.page + (key & pmask)) * NKV + kvh) * HDr;
  };
  constexpr int kStep = kDecChunk * kDecWaves;
  for (int kc0 = rg.start + kDecChunk * wave; kc0 < rg.end; kc0 += kStep) {
    // keys past the end clamp to the last one (masked below), so every load is unconditional
    f32x4 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
      const float* kr = Kc + row_off(min(kc0 + 16 * kb + lh, last));
      s[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < NQ / 4; u++) {
        const f32x4 a = *(const f32x4*)(kr + min(lg * NQ + 4 * u, HDr - 4));
#pragma unroll
        for (int e = 0; e < 4; e++) s[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], qreg[4 * u + e], s[kb], 0, 0, 0);
      }
    }
    // s[kb][r] is key kc0 + 16*kb + 4*lg + r, head lh
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int key = kc0 + 16 * kb + 4 * lg + r;
        float t;
        if (FEAT) {
          float x = s[kb][r] * p.scale;
          if (p.softcap > 0.0f) x = p.softcap * tanhf(x * inv_cap);
          x += slope * (float)(key - rg.qpos);
          t = x * kLog2e;
        } else {
          t = s[kb][r] * c_log2;
        }
        t = key < rg.end ? t : -INFINITY;
        s[kb][r] = t;
        mx = fmaxf(mx, t);
      }
    mx = half_max(xor16_max(mx));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float corr = exp2_fast(m_run - m_use);
    float rs = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float e = exp2_fast(s[kb][r] - m_use);
        rs += e;
        s[kb][r] = e;
      }
    l_run = l_run * corr + rs;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < NDB; db++) oacc[db] *= corr;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float* vr = Vc + row_off(min(kc0 + 16 * kb + 4 * lg + r, last));
#pragma unroll
        for (int db = 0; db < NDB; db++)
          oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[min(16 * db + lh, HDr - 1)], s[kb][r], oacc[db], 0, 0, 0);
      }
  }

  // ---- merge the four waves (as the fp16/bf16 kernel)
  const float l_grp = half_sum(xor16_sum(l_run));
  __syncthreads();  // q staging is dead: the region holds the accumulators
  float* red_o = (float*)raw;  // [wave][16 heads][HD]
  if (lg == 0) {
    red_m[wave][lh] = m_run;
    red_l[wave][lh] = l_grp;
  }
#pragma unroll
  for (int db = 0; db < NDB; db++)
#pragma unroll
    for (int r = 0; r < 4; r++) red_o[(wave * 16 + lh) * HD + 16 * db + 4 * lg + r] = oacc[db][r];
  __syncthreads();
  for (int i = tid; i < hg * HDr; i += 256) {
    const int g = i / HDr, d = i % HDr;
    float gm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecWaves; w++) gm = fmaxf(gm, red_m[w][g]);
    float l = 0.0f, acc = 0.0f;
    if (gm != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kDecWaves; w++) {
        const float f = exp2_fast(red_m[w][g] - gm);
        l += f * red_l[w][g];
        acc += f * red_o[(w * 16 + g) * HD + d];
      }
    }
    float* out = p.scratch + (((long long)(b * p.nq + tk) * p.NH + h0 + g) * p.nsplit + sp) * (HDr + 2);
    if (d == 0) {
      out[0] = gm;
      out[1] = l;
    }
    out[2 + d] = acc;
  }
}

// merge nsplit partials of one (token, head): grid (batch*nq, NH), block HD
template <typename T, int HD, int NC>
__global__ __launch_bounds__(256) void dec_combine_kernel(FableDecParams p) {
  // one thread per column of the kernel width HD; the head dim p.HD <= HD sets the strides
  const int row = blockIdx.x, h = blockIdx.y, d = threadIdx.x, HDr = p.HD;
  const int dc = min(d, HDr - 1);  // threads past the head dim read a valid column, store nothing
  const float* base = p.scratch + ((long long)row * p.NH + h) * p.nsplit * (HDr + 2);
  // the splits in chunks of NC (2, 4 or 8, at least the split count up to 8) whose loads are all
  // issued before any is used (indices past the last split repeat it and are not used): a few
  // memory latencies instead of one per split (a batch-1 decode of 21 splits took 12 us here
  // with one load per step); sums in split order
  constexpr int kC = NC;
  const int ns = p.nsplit;
  auto rec = [&](int s) { return base + (long long)min(s, ns - 1) * (HDr + 2); };
  float gm = -INFINITY;
  for (int s0 = 0; s0 < ns; s0 += kC) {
    float m[kC];
#pragma unroll
    for (int u = 0; u < kC; u++) m[u] = rec(s0 + u)[0];
#pragma unroll
    for (int u = 0; u < kC; u++)
      if (s0 + u < ns) gm = fmaxf(gm, m[u]);
  }
  float l = 0.0f, acc = 0.0f;
  if (gm != -INFINITY) {
    for (int s0 = 0; s0 < ns; s0 += kC) {
      float m[kC], ls[kC], a[kC];
#pragma unroll
      for (int u = 0; u < kC; u++) {
        const float* ps = rec(s0 + u);
        m[u] = ps[0];
        ls[u] = ps[1];
        a[u] = ps[2 + dc];
      }
#pragma unroll
      for (int u = 0; u < kC; u++) {
        if (s0 + u < ns) {
          const float w = exp2_fast(m[u] - gm);
          l += w * ls[u];
          acc += w * a[u];
        }
      }
    }
  }
  const bool ok = gm != -INFINITY && l > 0.0f;
  if (d < HDr) ((T*)p.o)[((long long)row * p.NH + h) * HDr + d] = (T)(ok ? acc / l : 0.0f);
  if (p.lse_out && d == 0) p.lse_out[(long long)row * p.NH + h] = ok ? gm * kLn2 + __logf(l) : -INFINITY;
}

// write new_k (rotary applied) / new_v at positions ctx_len[b]+tk: grid (batch*nq, NKV), block HD
template <typename T, int HD>
__global__ __launch_bounds__(256) void dec_append_kernel(FableDecParams p, const T* nk, const T* nv, int page_shift) {
  __shared__ float ks[HD];
  // one thread per column of the kernel width HD; rows are p.HD <= HD long
  const int b = blockIdx.x / p.nq, tk = blockIdx.x % p.nq, kvh = blockIdx.y, d = threadIdx.x;
  const int NKV = p.NH / p.gqa, HDr = p.HD;
  const int pos = p.ctx_len[b] + tk;
  const bool ok = pos >= 0 && (pos >> page_shift) < p.max_blocks && d < HDr;
  const long long src = ((long long)(b * p.nq + tk) * NKV + kvh) * HDr;
  ks[d] = d < HDr ? (float)nk[src + d] : 0.0f;
  __syncthreads();
  if (p.rotary) {
    const int rdim = p.rotary_dim > 0 ? p.rotary_dim : HDr, half = rdim / 2;
    const int rp = (p.rotary_pos ? p.rotary_pos[b] : p.ctx_len[b]) + tk;
    const bool act = d < half;
    const int ia = p.rotary == 1 ? d : 2 * d, ib = p.rotary == 1 ? d + half : 2 * d + 1;
    float x = 0.0f, y = 0.0f, c = 0.0f, s = 0.0f;
    if (act) {
      c = p.cos[(long long)rp * half + d];
      s = p.sin[(long long)rp * half + d];
      x = ks[ia];
      y = ks[ib];
    }
    __syncthreads();
    if (act) {
      ks[ia] = x * c - y * s;
      ks[ib] = y * c + x * s;
    }
    __syncthreads();
  }
  if (!ok) return;
  const int blk = p.block_table[(long long)b * p.max_blocks + (pos >> page_shift)];
  const long long dst = (((long long)blk * p.page + (pos & (p.page - 1))) * NKV + kvh) * HDr + d;
  ((T*)p.Kc)[dst] = (T)ks[d];
  ((T*)p.Vc)[dst] = nv[src + d];
}

template <typename T, int HD>
static int launch_dec(const FableDecParams& p, hipStream_t st, const void* nk, const void* nv) {
  const int page_shift = __builtin_ctz((unsigned)p.page);
  const int NKV = p.NH / p.gqa;
  const int ngrp = (p.gqa + 15) / 16;
  if (nk) {
    hipLaunchKernelGGL((dec_append_kernel<T, HD>), dim3(p.batch * p.nq, NKV), dim3(HD), 0, st, p,
                       (const T*)nk, (const T*)nv, page_shift);
    if (int rc = launch_status("fable_attn_dec (append)")) return rc;
  }
  const bool feat = p.softcap > 0.0f || p.alibi != nullptr;
  dim3 grid(NKV * ngrp, p.batch * p.nq, p.nsplit);
  if constexpr (std::is_same<T, float>::value) {
    if (feat)
      hipLaunchKernelGGL((dec_partial_f32_kernel<HD, true>), grid, dim3(256), 0, st, p, page_shift, ngrp, nk ? 1 : 0);
    else
      hipLaunchKernelGGL((dec_partial_f32_kernel<HD, false>), grid, dim3(256), 0, st, p, page_shift, ngrp, nk ? 1 : 0);
  } else {
    const bool spt = p.page >= 16;
    // one split: the partial kernel writes the output and LSE, and no combine is launched
    const int flags = (nk ? kDecAppend : 0) | (p.nsplit == 1 ? kDecFinal : 0);
    if (feat && spt)
      hipLaunchKernelGGL((dec_partial_kernel<T, HD, true, true>), grid, dim3(256), 0, st, p, page_shift, ngrp, flags);
    else if (feat)
      hipLaunchKernelGGL((dec_partial_kernel<T, HD, true, false>), grid, dim3(256), 0, st, p, page_shift, ngrp, flags);
    else if (spt)
      hipLaunchKernelGGL((dec_partial_kernel<T, HD, false, true>), grid, dim3(256), 0, st, p, page_shift, ngrp, flags);
    else
      hipLaunchKernelGGL((dec_partial_kernel<T, HD, false, false>), grid, dim3(256), 0, st, p, page_shift, ngrp, flags);
    if (int rc = launch_status("fable_attn_dec (partial)")) return rc;
    if (p.nsplit == 1) return FA_OK;
  }
  if (int rc = launch_status("fable_attn_dec (partial)")) return rc;
  const dim3 cg(p.batch * p.nq, p.NH);
  if (p.nsplit <= 2)
    hipLaunchKernelGGL((dec_combine_kernel<T, HD, 2>), cg, dim3(HD), 0, st, p);
  else if (p.nsplit <= 4)
    hipLaunchKernelGGL((dec_combine_kernel<T, HD, 4>), cg, dim3(HD), 0, st, p);
  else
    hipLaunchKernelGGL((dec_combine_kernel<T, HD, 8>), cg, dim3(HD), 0, st, p);
  return launch_status("fable_attn_dec (combine)");
}

// fp16/bf16: every head dim that is a multiple of 8 up to 256 runs in the kernel of the next
// multiple of 32 (64 at least: the K slice swizzle needs 8 chunks per row) with zero columns
// past it. The loads skip those columns' bytes, so HBM traffic is that of the real head dim.
// fp32 runs in kernels of width 64, 128 and 256, the same way.
template <typename T>
static int dec_dispatch(const FableDecParams& p, hipStream_t st, const void* nk, const void* nv) {
  constexpr bool f32 = std::is_same<T, float>::value;
  if (p.HD <= 0 || p.HD > 256 || p.HD % 8)
    return fail(FA_ERR_HEADDIM, "fable_attn_dec: head_dim=%d has no kernel (multiples of 8 up to 256)", p.HD);
  if constexpr (f32) {
    if (p.HD <= 64) return launch_dec<T, 64>(p, st, nk, nv);
    if (p.HD <= 128) return launch_dec<T, 128>(p, st, nk, nv);
    return launch_dec<T, 256>(p, st, nk, nv);
  } else {
    switch (p.HD <= 64 ? 2 : (p.HD + 31) / 32) {
      case 2: return launch_dec<T, 64>(p, st, nk, nv);
      case 3: return launch_dec<T, 96>(p, st, nk, nv);
      case 4: return launch_dec<T, 128>(p, st, nk, nv);
      case 5: return launch_dec<T, 160>(p, st, nk, nv);
      case 6: return launch_dec<T, 192>(p, st, nk, nv);
      case 7: return launch_dec<T, 224>(p, st, nk, nv);
      default: return launch_dec<T, 256>(p, st, nk, nv);
    }
  }
}

}  // namespace fa

// Split count from a model of the partial kernel as a stream of workgroup rounds: one
// workgroup per CU is resident (256 CUs), the cache read saturates HBM once ~168 workgroups
// stream together, and each split pays a fixed cost of about 64 keys (prologue, partial
// write, combine). Time of a round of t workgroups ~ t * (keys per split + 64) / min(t, 168);
// the smallest n within the minimum wins. At least 256 keys per split, n in [1, 512].
// On the C4 shape (128 groups, 32768 keys) the model ranks n = 1, 2, 3, 4 as measured on
// MI355X (474, 371, 414, 375 us). Reference heuristic (72 CUs): package/csrc/dispatch.cpp:182-200.
extern "C" int fa_decode_num_splits(int batch, int nq, int NH, int gqa, int64_t ctx_bound, int hint) {
  if (hint > 0) return hint > 512 ? 512 : hint;
  constexpr long long kSlots = 256, kSat = 168, kSplitCost = 64;
  const int g = gqa > 0 ? gqa : 1;
  long long groups = (long long)batch * (nq > 0 ? nq : 1) * (NH / g > 0 ? NH / g : 1) * ((g + 15) / 16);
  if (groups < 1) groups = 1;
  const long long ctx = ctx_bound > 1 ? ctx_bound : 1;
  long long maxn = (ctx + 255) / 256;
  maxn = maxn < 1 ? 1 : (maxn > 512 ? 512 : maxn);
  int best = 1;
  double best_cost = 0.0;
  for (long long n = 1; n <= maxn; n++) {
    const double per = (double)((ctx + n - 1) / n + kSplitCost);
    const long long wgs = groups * n, full = wgs / kSlots, tail = wgs % kSlots;
    double cost = (double)full * kSlots * per / kSat;
    if (tail) cost += (double)tail * per / (double)(tail < kSat ? tail : kSat);
    if (n == 1 || cost < best_cost * 0.995) {
      best = (int)n;
      best_cost = cost;
    }
  }
  // A choice that leaves CUs idle in its one round: with few groups each workgroup streams a
  // long span alone, below the rate the model's saturation point assumes, so fill the round
  // while every split keeps at least kFillKeys keys (batch 1, 8 kv heads, 32768 keys: 21 -> 32
  // splits, partial kernel 30.0 -> 24.5 us)
  constexpr long long kFillKeys = 512;
  const long long fill = kSlots / groups;
  if ((long long)best * groups < kSlots && fill > best && fill <= maxn && (ctx + fill - 1) / fill >= kFillKeys)
    best = (int)fill;
  return best;
}

// Whether a call reads or writes p.scratch: with one split the fp16/bf16 partial kernel writes the
// output and LSE itself and no combine runs; fp32 always combines through the scratch.
static bool dec_uses_scratch(const FableDecParams& p, int dtype) { return p.nsplit != 1 || dtype == FA_F32; }

extern "C" int fable_attn_dec(FableDecParams p, int dtype, void* stream, const void* new_k, const void* new_v) {
  using namespace fa;
  if (!p.q || !p.Kc || !p.Vc || !p.block_table || !p.o || !p.ctx_len)
    return fail(FA_ERR_ARG, "fable_attn_dec: null pointer");
  if (!p.scratch && dec_uses_scratch(p, dtype))
    return fail(FA_ERR_ARG, "fable_attn_dec: null scratch (needed unless nsplit == 1 with fp16/bf16)");
  return dec_checked(p, dtype, stream, new_k, new_v);
}

// ------------------------------------------------------------------ decode without allocation
// The split partials live in a device array of fixed size that the library owns (one copy per
// GPU, held until the process ends), for callers that cannot allocate: code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc. In host code `dec_scratch`
// names a host-side stand-in, not device memory: its device address on the current GPU comes
// from hipGetSymbolAddress, once per device, and only that address is ever passed to a kernel.
// Every partial slot is written before the combine reads it, so nothing needs clearing between
// calls; calls that overlap on one GPU (two streams, or a graph replay beside an eager call)
// race on the array and must be serialised by the caller.
namespace {

constexpr long long kDecScratchFloats = 4ll << 20;  // 16 MiB
static __device__ __align__(256) float dec_scratch[kDecScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_dec_scratch_mu;
float* g_dec_scratch_ptr[kMaxDevices] = {};

// device address of dec_scratch on the GPU of `stream` (which must be the current device)
int dec_scratch_ptr(void* stream, float** out) {
  using fa::fail;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur < 0 || cur >= kMaxDevices)
    return fail(FA_ERR_LAUNCH, "fable_attn_dec_noalloc: no current device (%d)", cur);
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice((hipStream_t)stream, &sdev) != hipSuccess)
      return fail(FA_ERR_ARG, "fable_attn_dec_noalloc: the stream's device is unknown");
    if (sdev != cur)
      return fail(FA_ERR_ARG, "fable_attn_dec_noalloc: the stream belongs to device %d, the current "
                              "device is %d (make the stream's device current)", (int)sdev, cur);
  }
  std::lock_guard<std::mutex> lock(g_dec_scratch_mu);
  if (!g_dec_scratch_ptr[cur]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(dec_scratch));
    if (e != hipSuccess || !ptr)
      return fail(FA_ERR_LAUNCH, "fable_attn_dec_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
    g_dec_scratch_ptr[cur] = (float*)ptr;
  }
  *out = g_dec_scratch_ptr[cur];
  return FA_OK;
}

}  // namespace

extern "C" int64_t fable_attn_dec_noalloc_max_floats(void) { return kDecScratchFloats; }

extern "C" int fable_attn_dec_noalloc(FableDecParams p, int dtype, void* stream, const void* new_k,
                                      const void* new_v) {
  using namespace fa;
  if (!p.q || !p.Kc || !p.Vc || !p.block_table || !p.o || !p.ctx_len)
    return fail(FA_ERR_ARG, "fable_attn_dec_noalloc: null pointer");
  if (p.batch <= 0) return FA_OK;
  if (p.NH <= 0) return fail(FA_ERR_ARG, "fable_attn_dec_noalloc: NH=%d", p.NH);
  if (p.nsplit < 1 || p.nsplit > 512) return fail(FA_ERR_ARG, "fable_attn_dec_noalloc: nsplit=%d", p.nsplit);
  if (p.HD <= 0) return fail(FA_ERR_HEADDIM, "fable_attn_dec_noalloc: head_dim=%d", p.HD);
  // one fp16/bf16 split never touches the array: no size limit then
  const long long need = (long long)p.batch * (p.nq < 1 ? 1 : p.nq) * p.NH * p.nsplit * (p.HD + 2);
  if (dec_uses_scratch(p, dtype) && need > kDecScratchFloats)
    return fail(FA_ERR_ARG, "fable_attn_dec_noalloc: batch*nq*NH*nsplit*(HD+2) = %lld floats of split "
                            "partials exceed the fixed %lld (lower nsplit, or use fable_attn_dec with a "
                            "caller-allocated scratch)", need, kDecScratchFloats);
  if (int rc = dec_scratch_ptr(stream, &p.scratch)) return rc;
  return dec_checked(p, dtype, stream, new_k, new_v);
}

namespace fa {

// the checks and dispatch shared by fable_attn_dec and fable_attn_dec_noalloc
static int dec_checked(FableDecParams p, int dtype, void* stream, const void* new_k, const void* new_v) {
  if (p.page <= 0 || (p.page & (p.page - 1))) return fail(FA_ERR_ARG, "fable_attn_dec: page=%d is not a power of two", p.page);
  if (p.NH <= 0 || p.gqa <= 0 || p.NH % p.gqa) return fail(FA_ERR_ARG, "fable_attn_dec: NH=%d gqa=%d", p.NH, p.gqa);
  if (p.nsplit < 1 || p.nsplit > 512) return fail(FA_ERR_ARG, "fable_attn_dec: nsplit=%d", p.nsplit);
  if (p.nq < 1) p.nq = 1;
  if ((new_k == nullptr) != (new_v == nullptr)) return fail(FA_ERR_ARG, "fable_attn_dec: new_k and new_v go together");
  if (p.rotary && (!p.cos || !p.sin)) return fail(FA_ERR_ARG, "fable_attn_dec: rotary needs cos and sin");
  if (p.rotary && (p.rotary_dim < 0 || p.rotary_dim > p.HD || p.rotary_dim % 2)) return fail(FA_ERR_ARG, "fable_attn_dec: rotary_dim=%d", p.rotary_dim);
  if (p.batch <= 0) return FA_OK;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case FA_F16: return dec_dispatch<_Float16>(p, st, new_k, new_v);
    case FA_BF16: return dec_dispatch<__bf16>(p, st, new_k, new_v);
    case FA_F32: return dec_dispatch<float>(p, st, new_k, new_v);
    default: return fail(FA_ERR_DTYPE, "fable_attn_dec: dtype %d not implemented (fp16/bf16/fp32)", dtype);
  }
}

}  // namespace fa
