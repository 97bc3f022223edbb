// Per-format weight-chunk dot products shared by the GEMV and the MoE grouped kernels.
// See afx_gemv.hip for the formats and the work decomposition.
#pragma once
#include "afx_common.h"

namespace afx {

enum { FMT_I8 = 0, FMT_Q4 = 1, FMT_F16 = 2 };

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
template <int FMT> struct Fmt;

template <> struct Fmt<FMT_I8> {
  static constexpr int kWeightsPerChunk = 16;
  __device__ static size_t row_bytes(int K) { return (size_t)K; }
  // dot of one 16-code chunk with the 16 x values at k = 16c
  template <int M>
  __device__ static void dot(const u4& w, const half_t* const (&xp)[M], int c, int, const u2&,
                             float (&acc)[M]) {
    h2 q[8];
    i8x4_to_h2(w.x, q[0], q[1]); i8x4_to_h2(w.y, q[2], q[3]);
    i8x4_to_h2(w.z, q[4], q[5]); i8x4_to_h2(w.w, q[6], q[7]);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      h2 xv[8];
      load_x<2>(xp[m] + 16 * c, xv);
      float s = acc[m];
#pragma unroll
      for (int i = 0; i < 8; ++i) s = dot2(q[i], xv[i], s);
      acc[m] = s;
    }
  }
};

template <> struct Fmt<FMT_Q4> {
  static constexpr int kWeightsPerChunk = 32;
  __device__ static size_t row_bytes(int K) { return (size_t)(K >> 1); }
  // chunk c = superblock sb*4 + word-group g; dword j of the chunk = elements 8g..8g+7 of
  // block 4sb+j; d = the 4 block scales of the superblock.
  template <int M>
  __device__ static void dot(const u4& w, const half_t* const (&xp)[M], int c, int, const u2& d,
                             float (&acc)[M]) {
    const int sb = c >> 2, g = c & 3;
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    const h2 d01 = as_h2(d.x), d23 = as_h2(d.y);
    const float ds[4] = {(float)d01.x, (float)d01.y, (float)d23.x, (float)d23.y};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h2 q[4];
      q4_word_to_h2(wd[j], q);
      const int k0 = 32 * (4 * sb + j) + 8 * g;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        h2 xv[4];
        load_x<1>(xp[m] + k0, xv);
        float s = dot2(q[0], xv[0], 0.0f);
        s = dot2(q[1], xv[1], s);
        s = dot2(q[2], xv[2], s);
        s = dot2(q[3], xv[3], s);
        acc[m] = __builtin_fmaf(ds[j], s, acc[m]);
      }
    }
  }
};

template <> struct Fmt<FMT_F16> {
  static constexpr int kWeightsPerChunk = 8;
  __device__ static size_t row_bytes(int K) { return (size_t)K * 2; }
  template <int M>
  __device__ static void dot(const u4& w, const half_t* const (&xp)[M], int c, int, const u2&,
                             float (&acc)[M]) {
    const h2 q[4] = {as_h2(w.x), as_h2(w.y), as_h2(w.z), as_h2(w.w)};
#pragma unroll
    for (int m = 0; m < M; ++m) {
      h2 xv[4];
      load_x<1>(xp[m] + 8 * c, xv);
      float s = acc[m];
#pragma unroll
      for (int i = 0; i < 4; ++i) s = dot2(q[i], xv[i], s);
      acc[m] = s;
    }
  }
};


}  // namespace afx
