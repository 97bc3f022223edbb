// Per-format weight-chunk dot products shared by the GEMV and the MoE grouped kernels.
// See afx_gemv.hip for the formats and the work decomposition.
#pragma once
#include "afx_common.h"

namespace afx {

enum { FMT_I8 = 0, FMT_Q4 = 1, FMT_F16 = 2, FMT_BW = 3, FMT_L4 = 4, FMT_Q4K = 5, FMT_Q6K = 6 };

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
// Ctx: per-row state a format's dot product needs beyond the chunk (the LUT4 codebook's byte
// tables), built once per row a wavefront owns from the scale pointer; empty for the others.
// S: the per-chunk side word loaded with each chunk (block scales; Q6_K's high bits and scales).
struct NoCtx {
  __device__ static NoCtx make(const half_t*, int) { return {}; }
};
// A "chunk" is the 16 weight bytes one lane loads per row: 16 int8 codes, 32 Q4 codes, or 8
// fp16 weights.  load_x fetches the matching activations once per chunk (kXH2 fp16 pairs) so
// they are reused across all rows a wavefront owns.
template <int FMT> struct Fmt;

template <> struct Fmt<FMT_I8> {
  using Ctx = NoCtx;
  using S = u2;
  static constexpr int kWeightsPerChunk = 16;
  static constexpr int kXH2 = 8;
  __device__ static size_t row_bytes(int K) { return (size_t)K; }
  __device__ static void load_x(const half_t* xrow, int c, h2 (&x)[kXH2]) { afx::load_x<2>(xrow + 16 * c, x); }
  __device__ static float dot(const u4& w, const h2 (&x)[kXH2], const u2&, const Ctx&, float acc) {
    h2 q[8];
    i8x4_to_h2(w.x, q[0], q[1]); i8x4_to_h2(w.y, q[2], q[3]);
    i8x4_to_h2(w.z, q[4], q[5]); i8x4_to_h2(w.w, q[6], q[7]);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = dot2(q[i], x[i], acc);
    return acc;
  }
  // The same chunk with every code offset by +1152 (the conversion's magic value left in place):
  // sum (q + 1152) x; the caller subtracts 1152 * sum(x) once per row.
  __device__ static float dot_biased(const u4& w, const h2 (&x)[kXH2], float acc) {
    const uint32_t wd[4] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u, w.z ^ 0x80808080u, w.w ^ 0x80808080u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc = dot2(as_h2(__builtin_amdgcn_perm(0x64646464u, wd[i], 0x04010400u)), x[2 * i], acc);
      acc = dot2(as_h2(__builtin_amdgcn_perm(0x64646464u, wd[i], 0x04030402u)), x[2 * i + 1], acc);
    }
    return acc;
  }
};

template <> struct Fmt<FMT_Q4> {
  using Ctx = NoCtx;
  using S = u2;
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
  // The weight is fp16((code - 8) * d), one v_pk_mul_f16 per pair (the exact product rounded
  // once): the value GGUFView.get hands the reference's matmul (aneforge/_gguf.py:34-39), and the
  // one the MFMA and prefill kernels multiply with.
  __device__ static float dot(const u4& w, const h2 (&x)[kXH2], const u2& d, const Ctx&, float acc) {
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    const h2 d01 = as_h2(d.x), d23 = as_h2(d.y);
    const half_t dh[4] = {d01.x, d01.y, d23.x, d23.y};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h2 q[4];
      q4_word_to_h2(wd[j], q);
      const h2 d2 = {dh[j], dh[j]};
      acc = dot2(q[0] * d2, x[4 * j + 0], acc);
      acc = dot2(q[1] * d2, x[4 * j + 1], acc);
      acc = dot2(q[2] * d2, x[4 * j + 2], acc);
      acc = dot2(q[3] * d2, x[4 * j + 3], acc);
    }
    return acc;
  }
};

// compress="blockwise": int8 codes [N][K] with one fp16 scale per 32 consecutive weights of a row,
// scale[N][K/32] (aneforge/_blob.py:46-56 with block_size 32).  The weight is the reference's
// reconstruction fp16(q * s) (one v_pk_mul_f16 per pair, exact product rounded once); a 16-code
// chunk lies in one block.  d.x = the scales of chunks 4i..4i+3 (two fp16), d.y = which half.
template <> struct Fmt<FMT_BW> {
  using Ctx = NoCtx;
  using S = u2;
  static constexpr int kWeightsPerChunk = 16;
  static constexpr int kXH2 = 8;
  __device__ static size_t row_bytes(int K) { return (size_t)K; }
  __device__ static void load_x(const half_t* xrow, int c, h2 (&x)[kXH2]) { afx::load_x<2>(xrow + 16 * c, x); }
  __device__ static float dot(const u4& w, const h2 (&x)[kXH2], const u2& d, const Ctx&, float acc) {
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
  using Ctx = NoCtx;
  using S = u2;
  static constexpr int kWeightsPerChunk = 8;
  static constexpr int kXH2 = 4;
  __device__ static size_t row_bytes(int K) { return (size_t)K * 2; }
  __device__ static void load_x(const half_t* xrow, int c, h2 (&x)[kXH2]) { afx::load_x<1>(xrow + 8 * c, x); }
  __device__ static float dot(const u4& w, const h2 (&x)[kXH2], const u2&, const Ctx&, float acc) {
    acc = dot2(as_h2(w.x), x[0], acc);
    acc = dot2(as_h2(w.y), x[1], acc);
    acc = dot2(as_h2(w.z), x[2], acc);
    acc = dot2(as_h2(w.w), x[3], acc);
    return acc;
  }
};

// compress="int4" (the reference's palettize_lut4, aneforge/_blob.py:28-43): a 16-entry fp16
// codebook per row, scale[N][16] (the codebook of the tensor the row came from, so fused q|k|v
// and gate|up matrices keep each tensor's own), 4-bit indices [N][K/2], byte j of a row =
// index of column 2j (low nibble) | index of column 2j + 1 (high nibble).  The weight is the
// codebook entry itself.  A chunk is 16 bytes = 32 columns; the lookup is pure VALU: the
// codebook's low and high bytes sit in 8 registers and v_perm_b32 picks four entries of an
// 8-entry half per instruction, v_bfi chooses the half by bit 3 of each index.  Columns come
// out as (c0, c2), (c4, c6), (c1, c3), (c5, c7) pairs, so load_x delivers x in that order.
struct L4Ctx {
  uint32_t lo[4], hi[4];   // lo[i] = low bytes of entries 4i .. 4i + 3; hi[i] = their high bytes
  __device__ static L4Ctx make(const half_t* scale, int row) {
    const half_t* cb = scale + 16 * (size_t)row;
    const u4 a = *(const u4*)cb, b = *(const u4*)(cb + 8);      // entries 0..7 and 8..15
    const uint32_t e[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};   // dword k = entries 2k, 2k + 1
    L4Ctx c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c.lo[i] = __builtin_amdgcn_perm(e[2 * i + 1], e[2 * i], 0x06040200u);
      c.hi[i] = __builtin_amdgcn_perm(e[2 * i + 1], e[2 * i], 0x07050301u);
    }
    return c;
  }
};
// Four entries at once.  sel: the low 3 bits of four indices, one per byte (upper bits zero);
// m: 0xFF in the bytes whose index is >= 8.
__device__ __forceinline__ void l4_lookup(const L4Ctx& t, uint32_t sel, uint32_t m, uint32_t& lb, uint32_t& hb) {
  const uint32_t l0 = __builtin_amdgcn_perm(t.lo[1], t.lo[0], sel), l1 = __builtin_amdgcn_perm(t.lo[3], t.lo[2], sel);
  const uint32_t h0 = __builtin_amdgcn_perm(t.hi[1], t.hi[0], sel), h1 = __builtin_amdgcn_perm(t.hi[3], t.hi[2], sel);
  lb = (m & l1) | (~m & l0);
  hb = (m & h1) | (~m & h0);
}
// Byte masks from bit 7 of each byte of s: v_perm selectors 8..11 replicate the sign bit of bytes
// 1, 3, 5, 7 of the 64-bit source {a, b}; with a = s and b = s << 8 those are bits 7, 23, 15, 31 of s.
__device__ __forceinline__ uint32_t l4_bit7_mask(uint32_t s) {
  return __builtin_amdgcn_perm(s, s << 8, 0x0B090A08u);
}
template <> struct Fmt<FMT_L4> {
  using Ctx = L4Ctx;
  using S = u2;
  static constexpr int kWeightsPerChunk = 32;
  static constexpr int kXH2 = 16;
  __device__ static size_t row_bytes(int K) { return (size_t)(K >> 1); }
  // x of the chunk's 32 columns as (x0, x2), (x4, x6), (x1, x3), (x5, x7) per group of 8
  __device__ static void load_x(const half_t* xrow, int c, h2 (&x)[kXH2]) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const u4 v = *(const u4*)(xrow + 32 * c + 8 * g);          // natural pairs (x0,x1) .. (x6,x7)
      x[4 * g + 0] = as_h2(__builtin_amdgcn_perm(v.y, v.x, 0x05040100u));
      x[4 * g + 1] = as_h2(__builtin_amdgcn_perm(v.w, v.z, 0x05040100u));
      x[4 * g + 2] = as_h2(__builtin_amdgcn_perm(v.y, v.x, 0x07060302u));
      x[4 * g + 3] = as_h2(__builtin_amdgcn_perm(v.w, v.z, 0x07060302u));
    }
  }
  __device__ static float dot(const u4& w, const h2 (&x)[kXH2], const u2&, const Ctx& t, float acc) {
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint32_t la, ha, lb, hb;
      // low nibbles: columns 0, 2, 4, 6 of the group (bit 3 of each byte -> bit 7 via << 4);
      // high nibbles: columns 1, 3, 5, 7 (bit 7 of each byte as it is)
      l4_lookup(t, wd[g] & 0x07070707u, l4_bit7_mask(wd[g] << 4), la, ha);
      l4_lookup(t, (wd[g] >> 4) & 0x07070707u, l4_bit7_mask(wd[g]), lb, hb);
      acc = dot2(as_h2(__builtin_amdgcn_perm(ha, la, 0x05010400u)), x[4 * g + 0], acc);   // (c0, c2)
      acc = dot2(as_h2(__builtin_amdgcn_perm(ha, la, 0x07030602u)), x[4 * g + 1], acc);   // (c4, c6)
      acc = dot2(as_h2(__builtin_amdgcn_perm(hb, lb, 0x05010400u)), x[4 * g + 2], acc);   // (c1, c3)
      acc = dot2(as_h2(__builtin_amdgcn_perm(hb, lb, 0x07030602u)), x[4 * g + 3], acc);   // (c5, c7)
    }
    return acc;
  }
};

// GGUF Q4_K (ggml block_q4_K: 256-weight super-blocks of 8 sub-blocks of 32 with 6-bit scales and
// mins; the reference dequantises it with gguf-py through GGUFView.get, aneforge/_gguf.py:34-39),
// repacked by afx_q4_k_repack: codes [N][K/2] keep each super-block's 128 code bytes in ggml order
// (byte 32p + l: element 64p + l in the low nibble, 64p + 32 + l in the high nibble), and the scale
// array holds 5 dwords per super-block: {fp16 d | fp16 dmin << 16}, then for each sub-block pair p
// the bytes {sc(2p), sc(2p + 1), m(2p), m(2p + 1)} (the 6-bit fields, unpacked).  The weight is the
// reference's fp16(d*sc*q - dmin*m) with gguf-py's float32 steps: d*sc and dmin*m are exact in
// fp32, and so is d*sc*q (17 + 4 bits), so one fma rounds exactly where gguf-py's subtraction does.
// Chunk c of a row: super-block c / 8, pair p = (c / 2) % 4, half h = c % 2; its low nibbles are
// elements 256(c / 8) + 64p + 16h + 0..15 (sub-block 2p), its high nibbles those + 32 (2p + 1).
__device__ __forceinline__ float ubyte_f32(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xFFu); }
template <> struct Fmt<FMT_Q4K> {
  using Ctx = NoCtx;
  using S = u2;
  static constexpr int kWeightsPerChunk = 32;
  static constexpr int kXH2 = 16;
  __device__ static size_t row_bytes(int K) { return (size_t)(K >> 1); }
  // x of the two 16-element runs: x[0..7] the low-nibble run, x[8..15] the high-nibble run
  __device__ static void load_x(const half_t* xrow, int c, h2 (&x)[kXH2]) {
    const half_t* p = xrow + 256 * (c >> 3) + 64 * ((c >> 1) & 3) + 16 * (c & 1);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const u4 v = *(const u4*)(p + 32 * r + 8 * i);
        x[8 * r + 4 * i + 0] = as_h2(v.x); x[8 * r + 4 * i + 1] = as_h2(v.y);
        x[8 * r + 4 * i + 2] = as_h2(v.z); x[8 * r + 4 * i + 3] = as_h2(v.w);
      }
  }
  // d.x = {d, dmin} of the super-block, d.y = the pair's scale and min bytes
  __device__ static float dot(const u4& w, const h2 (&x)[kXH2], const u2& d, const Ctx&, float acc) {
    const h2 dd = as_h2(d.x);
    const float dsup = (float)dd.x, dmin = (float)dd.y;
    const float dsa = dsup * ubyte_f32(d.y, 0), dsb = dsup * ubyte_f32(d.y, 1);
    const float dma = dmin * ubyte_f32(d.y, 2), dmb = dmin * ubyte_f32(d.y, 3);
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {                  // dword k: elements 4k..4k+3 of both runs
      uint32_t lo = wd[k] & 0x0F0F0F0Fu, hi = (wd[k] >> 4) & 0x0F0F0F0Fu;
      // opaque to the optimiser, so each byte converts with one v_cvt_f32_ubyte<n> (it would
      // otherwise re-extract every nibble from wd with a v_bfe first)
      asm("" : "+v"(lo), "+v"(hi));
      h2 a0, a1, b0, b1;
      a0.x = (half_t)__builtin_fmaf(dsa, ubyte_f32(lo, 0), -dma);
      a0.y = (half_t)__builtin_fmaf(dsa, ubyte_f32(lo, 1), -dma);
      a1.x = (half_t)__builtin_fmaf(dsa, ubyte_f32(lo, 2), -dma);
      a1.y = (half_t)__builtin_fmaf(dsa, ubyte_f32(lo, 3), -dma);
      b0.x = (half_t)__builtin_fmaf(dsb, ubyte_f32(hi, 0), -dmb);
      b0.y = (half_t)__builtin_fmaf(dsb, ubyte_f32(hi, 1), -dmb);
      b1.x = (half_t)__builtin_fmaf(dsb, ubyte_f32(hi, 2), -dmb);
      b1.y = (half_t)__builtin_fmaf(dsb, ubyte_f32(hi, 3), -dmb);
      acc = dot2(a0, x[2 * k], acc);
      acc = dot2(a1, x[2 * k + 1], acc);
      acc = dot2(b0, x[8 + 2 * k], acc);
      acc = dot2(b1, x[8 + 2 * k + 1], acc);
    }
    return acc;
  }
};

// GGUF Q6_K (ggml block_q6_K: 256 weights as 4-bit low parts ql, 2-bit high parts qh, int8 scales
// per 16 weights and an fp16 d; the reference dequantises it with gguf-py through GGUFView.get,
// aneforge/_gguf.py:34-39), repacked by afx_q6_k_repack into chunks of 32 consecutive weights:
// code dword k (k = 0..3) holds elements 8k + j in the low nibble and 8k + 4 + j in the high
// nibble of byte j; the side word is {H0, H1, sc_a | sc_b << 8 | d << 16} with H0 the high 2-bit
// parts of elements 0..15 and H1 of 16..31 (byte j of H_p: bits 0-1 element 16p + j, 2-3 element
// 16p + 4 + j, 4-5 element 16p + 8 + j, 6-7 element 16p + 12 + j), sc_a / sc_b the int8 scales of
// elements 0..15 / 16..31.  The weight is the reference's fp16(d*sc * (q - 32)): d*sc is exact in
// fp32 (11 + 8 bits) and so is its product with q - 32, so fma(d*sc, q, -32*d*sc) is that value
// (as +0 where gguf-py's product is -0, which adds nothing different to a dot product).
template <> struct Fmt<FMT_Q6K> {
  using Ctx = NoCtx;
  using S = u4;
  static constexpr int kWeightsPerChunk = 32;
  static constexpr int kXH2 = 16;
  __device__ static size_t row_bytes(int K) { return (size_t)(K >> 1); }
  __device__ static void load_x(const half_t* xrow, int c, h2 (&x)[kXH2]) { afx::load_x<4>(xrow + 32 * c, x); }
  __device__ static float dot(const u4& w, const h2 (&x)[kXH2], const u4& d, const Ctx&, float acc) {
    const float dsup = (float)as_h2(d.z).y;
    const float dsa = dsup * (float)(int8_t)(d.z & 0xFFu), dsb = dsup * (float)(int8_t)((d.z >> 8) & 0xFFu);
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    const uint32_t hh[2] = {d.x, d.y};
#pragma unroll
    for (int k = 0; k < 4; ++k) {                  // dword k: elements 8k..8k+3 (low) and 8k+4..8k+7 (high)
      const uint32_t H = hh[k >> 1];
      uint32_t lo = (wd[k] & 0x0F0F0F0Fu) | ((k & 1 ? H : H << 4) & 0x30303030u);
      uint32_t hi = ((wd[k] >> 4) & 0x0F0F0F0Fu) | ((k & 1 ? H >> 2 : H << 2) & 0x30303030u);
      asm("" : "+v"(lo), "+v"(hi));                // one v_cvt_f32_ubyte<n> per byte below
      const float ds = k < 2 ? dsa : dsb, off = -32.0f * ds;
      h2 a0, a1, b0, b1;
      a0.x = (half_t)__builtin_fmaf(ds, ubyte_f32(lo, 0), off);
      a0.y = (half_t)__builtin_fmaf(ds, ubyte_f32(lo, 1), off);
      a1.x = (half_t)__builtin_fmaf(ds, ubyte_f32(lo, 2), off);
      a1.y = (half_t)__builtin_fmaf(ds, ubyte_f32(lo, 3), off);
      b0.x = (half_t)__builtin_fmaf(ds, ubyte_f32(hi, 0), off);
      b0.y = (half_t)__builtin_fmaf(ds, ubyte_f32(hi, 1), off);
      b1.x = (half_t)__builtin_fmaf(ds, ubyte_f32(hi, 2), off);
      b1.y = (half_t)__builtin_fmaf(ds, ubyte_f32(hi, 3), off);
      acc = dot2(a0, x[4 * k], acc);
      acc = dot2(a1, x[4 * k + 1], acc);
      acc = dot2(b0, x[4 * k + 2], acc);
      acc = dot2(b1, x[4 * k + 3], acc);
    }
    return acc;
  }
};

// Per-chunk side words: Q4, the 4 fp16 of its superblock; blockwise, the 2 fp16 of chunks
// 4i..4i+3 and the half that is the chunk's; Q4_K, {d, dmin} and the pair's scale/min bytes;
// Q6_K, the chunk's 3 dwords; other formats have none.
template <int FMT>
__device__ __forceinline__ typename Fmt<FMT>::S load_scales(const half_t* drow, int c) {
  if constexpr (FMT == FMT_Q4) return *(const u2*)(drow + 4 * (c >> 2));
  else if constexpr (FMT == FMT_BW) return (u2){*(const uint32_t*)(drow + 2 * (c >> 2)), (uint32_t)((c >> 1) & 1)};
  else if constexpr (FMT == FMT_Q4K) {
    const uint32_t* q = (const uint32_t*)drow + 5 * (c >> 3);
    return (u2){q[0], q[1 + ((c >> 1) & 3)]};
  } else if constexpr (FMT == FMT_Q6K) {
    const uint32_t* q = (const uint32_t*)drow + 3 * c;
    return (u4){q[0], q[1], q[2], 0u};
  } else return typename Fmt<FMT>::S{};
}
// Whether the format carries per-chunk side words in a per-row array, and that row's length in halves.
template <int FMT> constexpr bool has_block_scales() {
  return FMT == FMT_Q4 || FMT == FMT_BW || FMT == FMT_Q4K || FMT == FMT_Q6K;
}
template <int FMT> __host__ __device__ constexpr long long scale_row_halves(int K) {
  return FMT == FMT_Q4K ? (long long)(K >> 8) * 10 : FMT == FMT_Q6K ? (long long)(K >> 5) * 6 : (long long)(K >> 5);
}

}  // namespace afx
