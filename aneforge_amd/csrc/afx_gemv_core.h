// Per-format weight-chunk dot products shared by the GEMV and the MoE grouped kernels.
// See afx_gemv.hip for the formats and the work decomposition.
#pragma once
#include "afx_common.h"

namespace afx {

enum { FMT_I8 = 0, FMT_Q4 = 1, FMT_F16 = 2, FMT_BW = 3 };

// ---- x sources: global memory or the LDS copy written by the norm prologue ----
template <int N8>
__device__ __forceinline__ void load_x(const half_t* p, h2 (&out)[N8 * 4]) {
#pragma unroll
  for (int i = 0; i < N8; ++i) {
    u4 v = *(const u4*)(p + 8 * i);
    out[4 * i + 0] = as_h2(v.x); out[4 * i + 1] = as_h2(v.y);
    out[4 * i + 2] = as_h2(v.z); out[4 * i + 3] = as_h2(v.w);
  }
}

// ---- per-format chunk geometry and math ----
// A "chunk" is the 16 weight bytes one lane loads per row: 16 int8 codes, 32 Q4 codes, or 8
// fp16 weights.  load_x fetches the matching activations once per chunk (kXH2 fp16 pairs) so
// they are reused across all rows a wavefront owns.
template <int FMT> struct Fmt;

template <> struct Fmt<FMT_I8> {
  static constexpr int kWeightsPerChunk = 16;
  static constexpr int kXH2 = 8;
  __device__ static size_t row_bytes(int K) { return (size_t)K; }
  __device__ static void load_x(const half_t* xrow, int c, h2 (&x)[kXH2]) { afx::load_x<2>(xrow + 16 * c, x); }
  __device__ static float dot(const u4& w, const h2 (&x)[kXH2], const u2&, float acc) {
    h2 q[8];
    i8x4_to_h2(w.x, q[0], q[1]); i8x4_to_h2(w.y, q[2], q[3]);
    i8x4_to_h2(w.z, q[4], q[5]); i8x4_to_h2(w.w, q[6], q[7]);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = dot2(q[i], x[i], acc);
    return acc;
  }
};

template <> struct Fmt<FMT_Q4> {
  static constexpr int kWeightsPerChunk = 32;
  static constexpr int kXH2 = 16;
  __device__ static size_t row_bytes(int K) { return (size_t)(K >> 1); }
  // chunk c = superblock sb*4 + word-group g; dword j of the chunk = elements 8g..8g+7 of
  // block 4sb+j; d = the 4 block scales of the superblock.
  __device__ static void load_x(const half_t* xrow, int c, h2 (&x)[kXH2]) {
    const int sb = c >> 2, g = c & 3;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h2 t[4];
      afx::load_x<1>(xrow + 32 * (4 * sb + j) + 8 * g, t);
      x[4 * j + 0] = t[0]; x[4 * j + 1] = t[1]; x[4 * j + 2] = t[2]; x[4 * j + 3] = t[3];
    }
  }
  __device__ static float dot(const u4& w, const h2 (&x)[kXH2], const u2& d, float acc) {
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    const h2 d01 = as_h2(d.x), d23 = as_h2(d.y);
    const float ds[4] = {(float)d01.x, (float)d01.y, (float)d23.x, (float)d23.y};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h2 q[4];
      q4_word_to_h2(wd[j], q);
      float s = dot2(q[0], x[4 * j + 0], 0.0f);
      s = dot2(q[1], x[4 * j + 1], s);
      s = dot2(q[2], x[4 * j + 2], s);
      s = dot2(q[3], x[4 * j + 3], s);
      acc = __builtin_fmaf(ds[j], s, acc);
    }
    return acc;
  }
};

// compress="blockwise": int8 codes [N][K] with one fp16 scale per 32 consecutive weights of a row,
// scale[N][K/32] (aneforge/_blob.py:46-56 with block_size 32).  The weight is the reference's
// reconstruction fp16(q * s) (one v_pk_mul_f16 per pair, exact product rounded once); a 16-code
// chunk lies in one block.  d.x = the scales of chunks 4i..4i+3 (two fp16), d.y = which half.
template <> struct Fmt<FMT_BW> {
  static constexpr int kWeightsPerChunk = 16;
  static constexpr int kXH2 = 8;
  __device__ static size_t row_bytes(int K) { return (size_t)K; }
  __device__ static void load_x(const half_t* xrow, int c, h2 (&x)[kXH2]) { afx::load_x<2>(xrow + 16 * c, x); }
  __device__ static float dot(const u4& w, const h2 (&x)[kXH2], const u2& d, float acc) {
    const h2 sp = as_h2(d.x);
    const half_t s = d.y ? sp.y : sp.x;
    const h2 s2 = {s, s};
    h2 q[8];
    i8x4_to_h2(w.x, q[0], q[1]); i8x4_to_h2(w.y, q[2], q[3]);
    i8x4_to_h2(w.z, q[4], q[5]); i8x4_to_h2(w.w, q[6], q[7]);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = dot2(q[i] * s2, x[i], acc);
    return acc;
  }
};

template <> struct Fmt<FMT_F16> {
  static constexpr int kWeightsPerChunk = 8;
  static constexpr int kXH2 = 4;
  __device__ static size_t row_bytes(int K) { return (size_t)K * 2; }
  __device__ static void load_x(const half_t* xrow, int c, h2 (&x)[kXH2]) { afx::load_x<1>(xrow + 8 * c, x); }
  __device__ static float dot(const u4& w, const h2 (&x)[kXH2], const u2&, float acc) {
    acc = dot2(as_h2(w.x), x[0], acc);
    acc = dot2(as_h2(w.y), x[1], acc);
    acc = dot2(as_h2(w.z), x[2], acc);
    acc = dot2(as_h2(w.w), x[3], acc);
    return acc;
  }
};

// Block scales for a chunk: Q4, the 4 fp16 of its superblock; blockwise, the 2 fp16 of chunks
// 4i..4i+3 and the half that is the chunk's; other formats have none.
template <int FMT>
__device__ __forceinline__ u2 load_scales(const half_t* drow, int c) {
  if constexpr (FMT == FMT_Q4) return *(const u2*)(drow + 4 * (c >> 2));
  else if constexpr (FMT == FMT_BW) return (u2){*(const uint32_t*)(drow + 2 * (c >> 2)), (uint32_t)((c >> 1) & 1)};
  else return (u2){0u, 0u};
}
// Whether the format carries per-block scales in a [N][K/32] array.
template <int FMT> constexpr bool has_block_scales() { return FMT == FMT_Q4 || FMT == FMT_BW; }

}  // namespace afx
