// attn_device.hpp — gfx950 (CDNA4) device helpers shared by the attention kernels.
//
// Vector types for the MFMA operands, the two MFMA shapes the kernels use, dtype traits for
// fp16/bf16 storage, and a few math helpers. Everything here is written for wave64 CDNA4 only.
//
// MFMA lane layouts relied on (v_mfma_f32_32x32x16_{f16,bf16}, wave64):
//   A (32 x 16):  lane l holds A[l % 32][8*(l/32) + e], e = 0..7 (one 16-byte register quad)
//   B (16 x 32):  lane l holds B[8*(l/32) + e][l % 32]
//   C (32 x 32):  lane l, accumulator r = 0..15 holds C[8*(r/4) + 4*(l/32) + (r%4)][l % 32]
// The contraction index mapping (e -> k) only has to agree between A and B, which it does by
// construction, so the kernels are free to permute the contraction order; the C layout is the
// one that fixes where each output element lives.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fable_attn_abi.h"

namespace fa {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// storage dtype traits
template <typename T>
struct Dt;

template <>
struct Dt<_Float16> {
  using V8 = f16x8;
  using V4 = f16x4;
  static __device__ __forceinline__ f32x16 mma32(V8 a, V8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(V8 a, V8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  // 16x16x16: lane (g, l) holds A[l][4g..4g+3] and B[4g..4g+3][l]
  static __device__ __forceinline__ f32x4 mma16k16(V4 a, V4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }
  // c + a.x + a.y with the pair's exact products by one (v_dot2c_f32_f16, fp32 accumulate)
  static __device__ __forceinline__ float sum2(f16x2 a, float c) {
    return __builtin_amdgcn_fdot2(a, f16x2{(_Float16)1.0f, (_Float16)1.0f}, c, false);
  }
  using V2 = f16x2;
};

template <>
struct Dt<__bf16> {
  using V8 = bf16x8;
  using V4 = bf16x4;
  static __device__ __forceinline__ f32x16 mma32(V8 a, V8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(V8 a, V8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16k16(V4 a, V4 b, f32x4 c) {
    typedef short s4 __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4, a), __builtin_bit_cast(s4, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f32(__bf16 x) { return (float)x; }
  static __device__ __forceinline__ float sum2(bf16x2 a, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, bf16x2{(__bf16)1.0f, (__bf16)1.0f}, c, false);
  }
  using V2 = bf16x2;
};

template <typename V, typename U>
__device__ __forceinline__ V bitcast(U u) {
  static_assert(sizeof(V) == sizeof(U), "bitcast size");
  return __builtin_bit_cast(V, u);
}

// Store of one 32-column block of a row held in the v_mfma_f32_32x32 accumulator layout: lane
// (r, hh) holds columns 8rq + 4hh + 0..3 of row r (rq = 0..3), scaled and rounded to T here.
// A v_permlane32_swap per dword pair (lane l <-> l + 32, i.e. the other half of the same row)
// trades the rq = 2j+1 run of lane hh = 0 for the rq = 2j run of lane hh = 1, leaving columns
// 16j + 0..7 in lane hh = 0 and 16j + 8..15 in lane hh = 1: each row goes out in 16-byte stores,
// 32 contiguous bytes per row and instruction, instead of 8-byte ones. Every lane executes the
// swaps; `ok` (the same for both lanes of a row) only guards the stores.
// `ncols` (default: all 32) stores only the block's columns below it: a head dim that is not a
// multiple of 32 (a multiple of 8) ends inside a block.
template <typename T>
__device__ __forceinline__ void store_cblock(T* dst, const f32x16& acc, float scale, int hh, bool ok,
                                             int ncols = 32) {
  using V4 = typename Dt<T>::V4;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    V4 x, y;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      x[c] = (T)(acc[8 * j + c] * scale);
      y[c] = (T)(acc[8 * j + 4 + c] * scale);
    }
    const u32x2 xd = __builtin_bit_cast(u32x2, x), yd = __builtin_bit_cast(u32x2, y);
    const auto r0 = __builtin_amdgcn_permlane32_swap(xd[0], yd[0], false, false);
    const auto r1 = __builtin_amdgcn_permlane32_swap(xd[1], yd[1], false, false);
    const u32x4 o = {r0[0], r1[0], r0[1], r1[1]};
    if (ok && 16 * j + 8 * hh < ncols) *(u32x4*)(dst + 16 * j + 8 * hh) = o;
  }
}

// The same C block in fp32, without the exchange: the lane's 16 values are head dims
// 16j + 8u + 4hh + 0..3 (j, u in {0, 1}) of its query, four 16-byte stores.
__device__ __forceinline__ void store_cblock_f32(float* dst, const f32x16& acc, float scale, int hh, bool ok,
                                                 int ncols = 32) {
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int d = 16 * j + 8 * u + 4 * hh;
      const f32x4 v = {acc[8 * j + 4 * u] * scale, acc[8 * j + 4 * u + 1] * scale,
                       acc[8 * j + 4 * u + 2] * scale, acc[8 * j + 4 * u + 3] * scale};
      if (ok && d < ncols) *(f32x4*)(dst + d) = v;
    }
}

// 2^x on the transcendental unit (v_exp_f32): exp2(-inf) = 0.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// tanh from the identity tanh(y) = 1 - 2 / (exp(2y) + 1); saturates to +-1 for large |y|.
__device__ __forceinline__ float tanh_exp(float y) {
  const float e = exp2_fast(2.0f * kLog2e * y);
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3",
// SC 2011): word 0 after ten rounds on the counter (idx, 0, 0) under the key `seed`. The
// reference draws its dropout stream this way (kernels/fa_common.hpp:71-82).
__device__ __forceinline__ uint32_t philox_w0(uint64_t seed, uint64_t idx) {
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  uint32_t c0 = (uint32_t)idx, c1 = (uint32_t)(idx >> 32), c2 = 0u, c3 = 0u;
#pragma unroll
  for (int r = 0; r < 10; r++) {
    const uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c0;
}

// Dropout multiplier of one score: keep_scale (= 1/(1-p)) when (word0 >> 8) * 2^-24 >= p,
// otherwise 0; idx = (h*SQ + q)*SK + key with no batch term (fa_common.hpp:84-88,
// fa_forward.hip:255-259).
__device__ __forceinline__ float dropout_z(uint64_t seed, uint64_t idx, float p, float keep_scale) {
  const float u = (float)(philox_w0(seed, idx) >> 8) * (1.0f / 16777216.0f);
  return u >= p ? keep_scale : 0.0f;
}

// Reductions across lanes l and l^32 (the two halves of one MFMA 32x32 C column) with
// v_permlane32_swap. Swapping a register with itself leaves, in every lane, the pair
// {x[l], x[l^32]} spread over the two results, so a symmetric op over both results is the
// cross-half reduction whichever result holds which value.
__device__ __forceinline__ float half_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ds_read_b64_tr_b16 on LDS: within each group of 16 lanes, lane i receives element i%4 of
// the 4-element (8-byte) runs addressed by lanes i/4, i/4+4, i/4+8, i/4+12. If lane j of a
// group addresses row R0 + j/4, column C0 + 4*(j%4) of a row-major 16-bit matrix, lane i gets
// column C0 + i of rows R0..R0+3: a transposed read.
template <typename T>
__device__ __forceinline__ typename Dt<T>::V4 lds_read_tr(const T* p) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  s4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s4*)((__attribute__((address_space(3))) T*)p));
  return __builtin_bit_cast(typename Dt<T>::V4, t);
}

// Offset (in elements) of row r, 16-byte chunk c of a row-major LDS tile with HD columns;
// chunks are XOR-swizzled by the row so that 8 consecutive rows read at one column hit
// different banks.
__device__ __forceinline__ int kofs(int r, int c, int HD, int KSW) {
  return r * HD + 8 * (c ^ (r % KSW));
}

// Raw buffer resource over [base, base + nbytes): 16-byte loads at offsets >= nbytes return
// zeros, so tile loads need no per-lane condition. nbytes is clamped to [0, kBufMax]; the third
// descriptor word selects 32-bit raw (untyped) access on gfx9-family parts. kBufMax stays below
// kBufZero, so a load at offset kBufZero always reads zeros: the zero columns of a padded head
// dim load from there (no select, no branch).
// (The clamp tests the high word with 32-bit compares, which stay on the scalar unit; a 64-bit
// ordered compare has no scalar form and goes to the VALU. The empty asm makes the high word
// opaque: without it the compiler folds `hi < 0` back into the 64-bit `nbytes < 0`. Its "s"
// constraint also states that the byte count is uniform, as every descriptor field must be.)
constexpr unsigned kBufMax = 0xFFFFFF00u;
constexpr int kBufZero = (int)0xFFFFFFF0u;  // as a byte offset: past every descriptor's range
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, long long nbytes) {
  int hi = (int)(nbytes >> 32);
  asm("" : "+s"(hi));
  unsigned n = hi < 0 ? 0u : (hi > 0 ? kBufMax : (unsigned)nbytes);
  n = n > kBufMax ? kBufMax : n;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, int voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
}
// the same with the non-temporal cache policy (cache-policy bit 1 is `nt` on gfx950), for data
// read once
__device__ __forceinline__ u32x4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, int voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 2);
}

// blockIdx.x -> work index so that consecutive work items land on the same XCD (one L2).
// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X.
__device__ __forceinline__ int xcd_remap(int L, int N) {
  constexpr int kXcd = 8;
  const int x = L % kXcd, idx = L / kXcd;
  const int per = N / kXcd, rem = N % kXcd;
  return x * per + (x < rem ? x : rem) + idx;
}

// blockIdx.x -> work index for a grid of N = (K/V groups) x gqa x U work items: work index
// w = (group * gqa + sibling) * U + u, where a K/V group is one K/V head of one sequence, its
// gqa query heads (siblings) read the same K/V, and u runs over the U items of one query head
// (q tiles, heaviest first under a causal mask).
//  * Whole K/V groups are dealt round-robin to the XCDs (group g to XCD g % 8), so a group's
//    K/V stays in one L2 and every XCD gets every eighth group. (Cutting the grid into 8
//    contiguous ranges instead gave XCD x the x-th eighth of the groups: with packed sequences
//    of unequal lengths that is one XCD per sequence, and the XCD holding the longest one set
//    the run time, 1.6x the balanced one at 8 causal sequences of 1.2k..6.9k rows.)
//  * An XCD with at most `umajor_max` items (a few per workgroup slot) runs them u-major (u,
//    then group, then sibling): the heaviest tiles of all its heads start first and the light
//    ones fill the end. That balanced causal S=4096 H=32 (two workgroups per slot) 1.24x better
//    than group after group, S=8192 1.04x, the C3 backward 1.07x. A larger share runs group
//    after group, its concurrent workgroups mostly on one head, whose K/V they then share in
//    L2: u-major over 16 packed sequence-heads per XCD cost 17% (C5-like windows) to 32%
//    (causal, head dim 256), and over the 4 heads per XCD of causal S=16384 H=32 it read 1.6x
//    the HBM bytes (1.80 vs 1.12 GB per launch) for the same time.
//  * Groups past the last full round of 8 are cut into 8 contiguous ranges.
// u-major limits (items per XCD): the forward kernels keep the 4 heads per XCD of long causal
// sequences group after group; the backward kernels gain from u-major up to 512. Dense plain
// causal forward grids up to head dim 128 run u-major up to kFwdUMajorCausal (their q tiles
// range from one key tile to the whole row, and group after group left the light tiles of the
// last heads to the end): B8 S2048 H32 D128 1.20-1.22x, D96 1.31x, D32 1.27x, B4 S4096 D96
// 1.18x, D64 1.13-1.17x, C2 1.00-1.015x. Non-causal tiles are all alike, and u-major only
// spread a CU's concurrent workgroups over more heads (B4 S4096 non-causal 0.92x).
constexpr int kFwdUMajor = 128, kBwdUMajor = 512, kFwdUMajorCausal = 512;
__device__ __forceinline__ int xcd_group_remap(int L, int N, int U, int gqa, int umajor_max) {
  constexpr int kXcd = 8;
  const int G = U * gqa;                   // items per K/V group
  const int R = N / G / kXcd;              // groups per XCD in the full rounds
  const int M = R * kXcd * G;
  if (L >= M) return M + xcd_remap(L - M, N - M);
  const int x = L % kXcd, k = L / kXcd;    // k < R * G
  if (R * G > umajor_max) return (x + kXcd * (k / G)) * G + k % G;
  const int u = k / (R * gqa), v = k % (R * gqa);
  const int group = x + kXcd * (v / gqa), sib = v % gqa;
  return (group * gqa + sib) * U + u;
}

}  // namespace fa
