// Batched prefill around the MFMA GEMM (afx_gemm.hip): the fused projection's split into
// q / cache rows with RoPE, and causal GQA flash attention over the resident cache.
//
// afx_qkv_split_rope: the prompt's [q | k | v] projection rows (q and k rows in RoPE-pair
// order, as the decode path packs them) -> RoPE'd q [M][Hq*dh] and K/V cache rows at positions
// pos0 .. pos0 + M - 1.  Same arithmetic as the decode epilogue: the fp16 projection value,
// then (x0 c0 - x1 s0, x1 c1 + x0 s1) in fp32 with the fp16 tables (aneforge/llm.py:96-105,
// rows written as in the reference's cache update, aneforge/llm.py:149-168).
//
// afx_prefill_attn: o = softmax(q K^T * scale + causal) V for query m at position pos0 + m over
// cache rows [0, pos0 + m] (aneforge/llm.py:149-168: the prompt attends the cache and itself;
// GQA head h reads kv head h / G, llm.py:205-211), fp32 scores and softmax, fp16 output.
// A 256-thread workgroup takes 64 queries of one head; each wavefront 16 of them as MFMA rows.
// Key blocks of 64 go through LDS: K row-major (the B operand of S = Q K^T reads 16 contiguous
// bytes of a key row), V transposed while staged (the B operand of O += P V needs 8
// consecutive keys of one dim).  S stays in registers for an online softmax (row max and sum
// by DPP rotations inside the 16-lane rows that hold one query row's scores); P goes through a
// wavefront-private LDS tile to change from the MFMA result layout to the operand layout.
#include <stdlib.h>
#include "afx_common.h"

namespace afx {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

__global__ void qkv_split_rope_kernel(const half_t* __restrict__ qkv, int ldqkv, int M, int nq, int nk, int dh,
                                      const half_t* __restrict__ cos_t, const half_t* __restrict__ sin_t,
                                      int pos0, int rope, half_t* __restrict__ q, int ldq,
                                      half_t* __restrict__ kc, half_t* __restrict__ vc, long long kv_hs) {
  const int pairs = (nq + 2 * nk) >> 1;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * pairs) return;
  const int m = (int)(i / pairs), pr = (int)(i - (long long)m * pairs);
  const int row0 = 2 * pr, p = pos0 + m;
  const half_t* src = qkv + (size_t)m * ldqkv + row0;
  const float v0 = (float)src[0], v1 = (float)src[1];
  if (row0 < nq + nk) {
    const bool isk = row0 >= nq;
    const int rl = isk ? row0 - nq : row0;
    const int head = rl / dh, d = (rl - head * dh) >> 1, half = dh >> 1;
    float o0 = v0, o1 = v1;                      // row0 holds dim d, row0 + 1 dim d + dh / 2
    if (rope) {
      const float c0 = (float)cos_t[(size_t)p * dh + d], s0 = (float)sin_t[(size_t)p * dh + d];
      const float c1 = (float)cos_t[(size_t)p * dh + d + half], s1 = (float)sin_t[(size_t)p * dh + d + half];
      o0 = __builtin_fmaf(v0, c0, -(v1 * s0));   // the contraction spelled out: both kernels round alike
      o1 = __builtin_fmaf(v1, c1, v0 * s1);
    }
    half_t* dst = isk ? kc + (size_t)head * kv_hs + (size_t)p * dh : q + (size_t)m * ldq + (size_t)head * dh;
    dst[d] = (half_t)o0;
    dst[d + half] = (half_t)o1;
  } else {
    const int rl = row0 - nq - nk;
    const int head = rl / dh, d = rl - head * dh;
    half_t* dst = vc + (size_t)head * kv_hs + (size_t)p * dh + d;
    dst[0] = (half_t)v0;
    dst[1] = (half_t)v1;
  }
}

// The same split with 8 packed rows (4 RoPE pairs, or 8 V dims) per thread: one 16-byte load, two
// 8-byte stores (dims d .. d + 3 and d + dh/2 .. + 3) or one 16-byte store, and 8-byte table loads;
// the per-element arithmetic is the scalar kernel's.  Needs dh % 8 == 0 and 16 / 8-byte aligned rows.
__global__ void qkv_split_rope_kernel8(const half_t* __restrict__ qkv, int ldqkv, int M, int nq, int nk, int dh,
                                       const half_t* __restrict__ cos_t, const half_t* __restrict__ sin_t,
                                       int pos0, int rope, half_t* __restrict__ q, int ldq,
                                       half_t* __restrict__ kc, half_t* __restrict__ vc, long long kv_hs) {
  const int chunks = (nq + 2 * nk) >> 3;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * chunks) return;
  const int m = (int)(i / chunks), c = (int)(i - (long long)m * chunks);
  const int col0 = 8 * c, p = pos0 + m;
  const u4 raw = *(const u4*)(qkv + (size_t)m * ldqkv + col0);
  if (col0 < nq + nk) {
    const bool isk = col0 >= nq;
    const int rl = isk ? col0 - nq : col0;
    const int head = rl / dh, d = (rl - head * dh) >> 1, half = dh >> 1;   // pairs d .. d + 3
    const h2 pr[4] = {as_h2(raw.x), as_h2(raw.y), as_h2(raw.z), as_h2(raw.w)};
    half_t r0[4], r1[4];                         // dims d + j and d + dh/2 + j
#pragma unroll
    for (int j = 0; j < 4; ++j) { r0[j] = pr[j].x; r1[j] = pr[j].y; }
    if (rope) {
      const u2 c0 = *(const u2*)(cos_t + (size_t)p * dh + d), c1 = *(const u2*)(cos_t + (size_t)p * dh + d + half);
      const u2 s0 = *(const u2*)(sin_t + (size_t)p * dh + d), s1 = *(const u2*)(sin_t + (size_t)p * dh + d + half);
      const h2 cc0[2] = {as_h2(c0.x), as_h2(c0.y)}, cc1[2] = {as_h2(c1.x), as_h2(c1.y)};
      const h2 ss0[2] = {as_h2(s0.x), as_h2(s0.y)}, ss1[2] = {as_h2(s1.x), as_h2(s1.y)};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float v0 = (float)r0[j], v1 = (float)r1[j];
        const float a0 = (float)(j & 1 ? cc0[j >> 1].y : cc0[j >> 1].x), b0 = (float)(j & 1 ? ss0[j >> 1].y : ss0[j >> 1].x);
        const float a1 = (float)(j & 1 ? cc1[j >> 1].y : cc1[j >> 1].x), b1 = (float)(j & 1 ? ss1[j >> 1].y : ss1[j >> 1].x);
        // each result rounded straight from the fma to fp16, as in the one-pair kernel and the decode
        // epilogue (the fp16 conversion fused into the fma: not the fp32 result rounded again)
        r0[j] = (half_t)__builtin_fmaf(v0, a0, -(v1 * b0));
        r1[j] = (half_t)__builtin_fmaf(v1, a1, v0 * b1);
      }
    }
    half_t* dst = isk ? kc + (size_t)head * kv_hs + (size_t)p * dh : q + (size_t)m * ldq + (size_t)head * dh;
    const h2 l0 = {r0[0], r0[1]}, l1 = {r0[2], r0[3]}, u0 = {r1[0], r1[1]}, u1 = {r1[2], r1[3]};
    *(u2*)(dst + d) = (u2){as_u32(l0), as_u32(l1)};
    *(u2*)(dst + d + half) = (u2){as_u32(u0), as_u32(u1)};
  } else {
    const int rl = col0 - nq - nk;
    const int head = rl / dh, d = rl - head * dh;
    *(u4*)(vc + (size_t)head * kv_hs + (size_t)p * dh + d) = raw;
  }
}

constexpr int kPD = 128;                 // head dim
constexpr int kPQ = 64, kPK = 64;        // queries per workgroup, keys per block
constexpr int kKStride = kPD * 2 + 16;   // bytes per staged K row
constexpr int kVStride = kPK * 2 + 16;   // bytes per staged V^T row (one dim, 64 keys)
constexpr int kPStride = kPK * 2 + 16;   // bytes per staged P row

struct PrefillAttnArgs {
  const half_t* q; const half_t* k; const half_t* v; half_t* o;
  long long kv_hs;
  int ldq, ldo, M, pos0, Hq, Hkv, Mmax;
  float scale_log2;
  int tiles;              // query tiles (the pipelined form's grid is tiles * Hq workgroups)
  int xcd_map;            // pipelined form: kv head k on XCD k % 8 (Hkv % 8 == 0)
  int order;              // form 3 tile order: 1 paired heavy / light, 0 heaviest first
};

// max / sum over the 16 lanes of each DPP row (every lane receives the result)
template <bool MAX>
__device__ __forceinline__ float row16(float v) {
  auto f = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  v = f(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x121, 0xf, 0xf, false)));
  v = f(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x122, 0xf, 0xf, false)));
  v = f(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false)));
  v = f(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false)));
  return v;
}

// One 64-key block of a wavefront's 16 queries: S = Q K^T from the staged K, the online softmax
// update (log2 domain), P through the wavefront's LDS tile, O += P V from the staged V^T.
__device__ __forceinline__ void attn_block(const PrefillAttnArgs& a, const unsigned char* Ks, const unsigned char* Vt,
                                           unsigned char* pw, const h8 (&qf)[4], const int (&qpos)[4], int key0,
                                           int mwave, int fr, int fg, f4 (&acc)[8], float (&mrow)[4],
                                           float (&lrow)[4]) {
  // S = Q K^T for 16 queries x 64 keys (four 16-key tiles)
  f4 s[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    s[j] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const h8 kf = __builtin_bit_cast(h8, *(const u4*)(Ks + (j * 16 + fr) * kKStride + (ks * 32 + 8 * fg) * 2));
      s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qf[ks], kf, s[j], 0, 0, 0);
    }
  }
  // online softmax (log2 domain); lane holds rows 4 * fg + i, key j * 16 + fr.  Only a block with a key
  // past the wavefront's first query position needs the causal mask (wavefront-uniform); the scale
  // (positive) is applied to the block maximum and inside the exponent's FMA.
  if (key0 + kPK - 1 > mwave) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) s[j][i] = key0 + j * 16 + fr <= qpos[i] ? s[j][i] : -INFINITY;
  }
  float alpha[4];
  bool grew = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float bm = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) bm = fmaxf(bm, s[j][i]);
    bm = row16<true>(bm) * a.scale_log2;
    const float mn = fmaxf(mrow[i], bm);         // finite: every row sees key 0 in block 0
    grew = grew || mn > mrow[i];
    alpha[i] = __builtin_amdgcn_exp2f(mrow[i] - mn);
    mrow[i] = mn;
    float rs = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j][i], a.scale_log2, -mn));
      s[j][i] = p;
      rs += p;
    }
    lrow[i] = lrow[i] * alpha[i] + row16<false>(rs);
  }
  // rescale only when some row's maximum grew (otherwise every alpha is exactly 1)
  if (__builtin_amdgcn_ballot_w64(grew)) {
#pragma unroll
    for (int d = 0; d < 8; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[d][i] *= alpha[i];
  }
  // P (fp16) through the wavefront's LDS tile into the A-operand layout
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *(half_t*)(pw + (4 * fg + i) * kPStride + (j * 16 + fr) * 2) = (half_t)s[j][i];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  h8 pf[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) pf[ks] = __builtin_bit_cast(h8, *(const u4*)(pw + fr * kPStride + (ks * 32 + 8 * fg) * 2));
  // O += P V over eight 16-dim tiles
#pragma unroll
  for (int d = 0; d < 8; ++d)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const h8 vf = __builtin_bit_cast(h8, *(const u4*)(Vt + (d * 16 + fr) * kVStride + (ks * 32 + 8 * fg) * 2));
      acc[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf[ks], vf, acc[d], 0, 0, 0);
    }
}

// K (row-major, 4 x 16 B per thread) and V (transposed while staged: one key per lane, four
// 16-byte dim groups per wavefront) of the 64-key block at key0 into LDS.
struct KvRegs { u4 k[4], v[4]; };
__device__ __forceinline__ void kv_load(const PrefillAttnArgs& a, const half_t* kbase, const half_t* vbase, int key0,
                                        int tid, int lane, int wave, KvRegs& r) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 256 * i, row = c >> 4, ch = c & 15;
    const int key = key0 + row < a.Mmax ? key0 + row : a.Mmax - 1;   // past the cache: masked in attn_block
    r.k[i] = *(const u4*)(kbase + (size_t)key * kPD + ch * 8);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ch = wave * 4 + i;                 // dims ch * 8 .. + 7 of key `lane`
    const int key = key0 + lane < a.Mmax ? key0 + lane : a.Mmax - 1;
    r.v[i] = *(const u4*)(vbase + (size_t)key * kPD + ch * 8);
  }
}
__device__ __forceinline__ void kv_stage(const KvRegs& r, unsigned char* Ks, unsigned char* Vt, int tid, int lane,
                                         int wave) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 256 * i, row = c >> 4, ch = c & 15;
    *(u4*)(Ks + row * kKStride + ch * 16) = r.k[i];
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ch = wave * 4 + i;
    const uint32_t w4[4] = {r.v[i].x, r.v[i].y, r.v[i].z, r.v[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      *(uint16_t*)(Vt + (ch * 8 + 2 * j) * kVStride + lane * 2) = (uint16_t)(w4[j] & 0xffffu);
      *(uint16_t*)(Vt + (ch * 8 + 2 * j + 1) * kVStride + lane * 2) = (uint16_t)(w4[j] >> 16);
    }
  }
}

// The workgroup's query tile and head, and the lane's query fragments / positions.
struct AttnTile { int h, kvh, m0, nkb; };
__device__ __forceinline__ void attn_prologue(const PrefillAttnArgs& a, const AttnTile& tl, int wave, int fr, int fg,
                                              h8 (&qf)[4], int (&qpos)[4]) {
  const int mq = tl.m0 + wave * 16 + fr;
  const half_t* qrow = a.q + (size_t)(mq < a.M ? mq : a.M - 1) * a.ldq + (size_t)tl.h * kPD;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) qf[ks] = __builtin_bit_cast(h8, *(const u4*)(qrow + ks * 32 + 8 * fg));
#pragma unroll
  for (int i = 0; i < 4; ++i) qpos[i] = a.pos0 + tl.m0 + wave * 16 + 4 * fg + i;
}
// o = acc / l: lane holds rows 4 * fg + i of dim d * 16 + fr
__device__ __forceinline__ void attn_store(const PrefillAttnArgs& a, const AttnTile& tl, int wave, int fr, int fg,
                                           const f4 (&acc)[8], const float (&lrow)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = tl.m0 + wave * 16 + 4 * fg + i;
    if (m >= a.M) continue;
    const float inv = 1.0f / lrow[i];
    half_t* orow = a.o + (size_t)m * a.ldo + (size_t)tl.h * kPD;
#pragma unroll
    for (int d = 0; d < 8; ++d) orow[d * 16 + fr] = (half_t)(acc[d][i] * inv);
  }
}
__device__ __forceinline__ AttnTile attn_tile(const PrefillAttnArgs& a, int h, int m0) {
  AttnTile t;
  t.h = h;
  t.kvh = h / (a.Hq / a.Hkv);
  t.m0 = m0;
  const int mlast = m0 + kPQ - 1 < a.M - 1 ? m0 + kPQ - 1 : a.M - 1;
  t.nkb = (a.pos0 + mlast) / kPK + 1;            // through the last key any query of the tile sees
  return t;
}

// Single-buffered form: grid (query tiles, heads), K/V of each block loaded, staged, then used.
__global__ __launch_bounds__(256) void prefill_attn_kernel(PrefillAttnArgs a) {
  __shared__ __align__(16) unsigned char Ks[kPK * kKStride];
  __shared__ __align__(16) unsigned char Vt[kPD * kVStride];
  __shared__ __align__(16) unsigned char Ps[4][16 * kPStride];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, fg = lane >> 4;
  const AttnTile tl = attn_tile(a, blockIdx.y, blockIdx.x * kPQ);
  const half_t* kbase = a.k + (size_t)tl.kvh * a.kv_hs;
  const half_t* vbase = a.v + (size_t)tl.kvh * a.kv_hs;
  h8 qf[4];
  int qpos[4];
  attn_prologue(a, tl, wave, fr, fg, qf, qpos);
  f4 acc[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) acc[d] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
  float mrow[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY}, lrow[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int kb = 0; kb < tl.nkb; ++kb) {
    KvRegs r;
    kv_load(a, kbase, vbase, kb * kPK, tid, lane, wave, r);
    kv_stage(r, Ks, Vt, tid, lane, wave);
    __syncthreads();
    attn_block(a, Ks, Vt, Ps[wave], qf, qpos, kb * kPK, a.pos0 + tl.m0 + wave * 16, fr, fg, acc, mrow, lrow);
    __syncthreads();                               // Ks, Vt and this wavefront's P are reused next block
  }
  attn_store(a, tl, wave, fr, fg, acc, lrow);
}

// Pipelined form (the default): the same per-block math, with
//  * the next block's K/V loaded into registers while the current block's MFMAs run, and staged into
//    the other of two LDS buffers afterwards (one barrier per block);
//  * the heaviest query tiles (the most causal key blocks) dispatched first, so the launch does not
//    end on a few long tiles;
//  * with Hkv % 8 == 0, every tile of kv head k on XCD k % 8 (workgroup b runs on XCD b % 8), so a
//    head's K/V rows are fetched into one L2 and reused there by its G query heads.
// Outputs are bit-identical to the single-buffered form.
__global__ __launch_bounds__(256) void prefill_attn_kernel2(PrefillAttnArgs a) {
  __shared__ __align__(16) unsigned char Ks[2][kPK * kKStride];
  __shared__ __align__(16) unsigned char Vt[2][kPD * kVStride];
  __shared__ __align__(16) unsigned char Ps[4][16 * kPStride];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, fg = lane >> 4;
  const int id = blockIdx.x, G = a.Hq / a.Hkv;
  int t, h;
  if (a.xcd_map) {
    const int x = id & 7, l = id >> 3, per_t = (a.Hkv >> 3) * G;
    t = a.tiles - 1 - l / per_t;
    const int r = l - (l / per_t) * per_t;
    h = (x + 8 * (r / G)) * G + r % G;
  } else {
    t = a.tiles - 1 - id / a.Hq;
    h = id % a.Hq;
  }
  const AttnTile tl = attn_tile(a, h, t * kPQ);
  const half_t* kbase = a.k + (size_t)tl.kvh * a.kv_hs;
  const half_t* vbase = a.v + (size_t)tl.kvh * a.kv_hs;
  KvRegs r;
  kv_load(a, kbase, vbase, 0, tid, lane, wave, r);
  h8 qf[4];
  int qpos[4];
  attn_prologue(a, tl, wave, fr, fg, qf, qpos);
  f4 acc[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) acc[d] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
  float mrow[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY}, lrow[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  kv_stage(r, Ks[0], Vt[0], tid, lane, wave);
  __syncthreads();
  const int mwave = a.pos0 + tl.m0 + wave * 16;
  for (int kb = 0; kb < tl.nkb; ++kb) {
    const int s = kb & 1;
    if (kb + 1 < tl.nkb) kv_load(a, kbase, vbase, (kb + 1) * kPK, tid, lane, wave, r);
    attn_block(a, Ks[s], Vt[s], Ps[wave], qf, qpos, kb * kPK, mwave, fr, fg, acc, mrow, lrow);
    if (kb + 1 < tl.nkb) kv_stage(r, Ks[s ^ 1], Vt[s ^ 1], tid, lane, wave);   // last read before the previous barrier
    __syncthreads();
  }
  attn_store(a, tl, wave, fr, fg, acc, lrow);
}

// ---- transposed-score form: S^T = K Q^T, 32 queries per wavefront, P never leaves the registers ----
// With K as the A operand and Q^T as B, a lane's MFMA result holds keys 4 * fg .. + 3 (of a 16-key
// tile) for query fr, so every score of one query sits in the four lanes fr, fr + 16, fr + 32, fr + 48:
//  * row maxima and sums are a lane-local reduction over 16 values plus two cross-lane exchanges;
//  * the fp16 probabilities of key tiles 2ks and 2ks + 1 are exactly the B operand P^T of the
//    32-key slot ks of O^T = V^T P^T, under the k order (4 fg .. + 3, 16 + 4 fg .. + 3), which V^T
//    is staged in (vt_pos), so a lane's 8 keys of one dim are one 16-byte LDS read;
//  * O^T's result holds dims 4 * fg .. + 3 of query fr: the softmax rescale is lane-local.
// Two query tiles per wavefront share every K and V fragment read (half the LDS reads per MFMA of
// the forms above).  Summation orders differ from them: results agree to fp16 rounding.
constexpr int kPQ3 = 128;                // queries per workgroup (4 wavefronts x 32)

__device__ __forceinline__ int vt_pos(int key) {   // staged position of key (0..63) in a V^T row
  const int k = key & 31;
  return (key & 32) + 8 * ((k & 15) >> 2) + 4 * (k >> 4) + (k & 3);
}
// over the lanes l, l ^ 16, l ^ 32, l ^ 48 (one query's four lanes), through the permlane swaps rather
// than LDS permutes: (v_l op v_l^16) op (v_l^32 op v_l^48) in every lane
__device__ __forceinline__ float xor_max(float v) { return swap32_max(swap16_max(v)); }
__device__ __forceinline__ float xor_sum(float v) { return swap32_sum(swap16_sum(v)); }
__device__ __forceinline__ void kv_stage3(const KvRegs& r, unsigned char* Ks, unsigned char* Vt, int tid, int lane,
                                          int wave) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 256 * i, row = c >> 4, ch = c & 15;
    *(u4*)(Ks + row * kKStride + ch * 16) = r.k[i];
  }
  const int vp = vt_pos(lane) * 2;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ch = wave * 4 + i;
    const uint32_t w4[4] = {r.v[i].x, r.v[i].y, r.v[i].z, r.v[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      *(uint16_t*)(Vt + (ch * 8 + 2 * j) * kVStride + vp) = (uint16_t)(w4[j] & 0xffffu);
      *(uint16_t*)(Vt + (ch * 8 + 2 * j + 1) * kVStride + vp) = (uint16_t)(w4[j] >> 16);
    }
  }
}

// Row-major V stages for the transposing LDS reads (ds_read_b64_tr_b16): V rows of 256 bytes,
// unpadded, their 16-byte chunks permuted by an even XOR of the row (chunk c of row r at
// c ^ 2 (r & 7)).  One operand read takes 32 bytes from each of 16 rows; the XOR puts rows with
// r & 7 = 0..7 on 8 distinct 32-byte bank ranges, and spreads the 16-byte staging stores of 8
// consecutive rows at one logical chunk over 8 distinct chunks.
constexpr int kVRow = kPD * 2;
__device__ __forceinline__ int vsw(int row, int ch) { return row * kVRow + ((ch ^ ((row & 7) << 1)) << 4); }

// K and V rows alike: 16 lanes per key row, consecutive 16-byte chunks; K first, so the scores
// can start while V is in flight.
__device__ __forceinline__ void kv_load_rm(const PrefillAttnArgs& a, const half_t* kbase, const half_t* vbase,
                                           int key0, int tid, KvRegs& r) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 256 * i, row = c >> 4, ch = c & 15;
    const int key = key0 + row < a.Mmax ? key0 + row : a.Mmax - 1;   // past the cache: masked in attn_block3
    r.k[i] = *(const u4*)(kbase + (size_t)key * kPD + ch * 8);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 256 * i, row = c >> 4, ch = c & 15;
    const int key = key0 + row < a.Mmax ? key0 + row : a.Mmax - 1;
    r.v[i] = *(const u4*)(vbase + (size_t)key * kPD + ch * 8);
  }
}
__device__ __forceinline__ void kv_stage_rm(const KvRegs& r, unsigned char* Ks, unsigned char* Vs, int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 256 * i, row = c >> 4, ch = c & 15;
    *(u4*)(Ks + row * kKStride + ch * 16) = r.k[i];
    *(u4*)(Vs + vsw(row, ch)) = r.v[i];
  }
}

typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

// EMPTY: a query may have seen no key yet (a block range that starts past its position); its
// running maximum is then -inf and the exponents take 0 in its place, so its probabilities are 0.
// VTR: V staged row-major (kv_stage_rm) and read through ds_read_b64_tr_b16, else V^T (kv_stage3).
// The block in two phases: attn_s3 (S^T, mask, online softmax, the accumulators rescaled, P^T packed
// into pf) and attn_pv3 (O^T += V^T P^T); attn_block3 runs both.
template <bool EMPTY = false>
__device__ __forceinline__ void attn_s3(const PrefillAttnArgs& a, const unsigned char* Ks, const h8 (&qf)[2][4],
                                        const int (&qp)[2], int key0, int mwpos, int fr, int fg, f4 (&acc)[2][8],
                                        float (&mrow)[2], float (&lrow)[2], h8 (&pf)[2][2]) {
  f4 st[2][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h8 kf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      kf[ks] = __builtin_bit_cast(h8, *(const u4*)(Ks + (j * 16 + fr) * kKStride + (ks * 32 + 8 * fg) * 2));
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      st[u][j] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) st[u][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[ks], qf[u][ks], st[u][j], 0, 0, 0);
    }
  }
  // causal mask only in a block holding a key past the wavefront's first query position (uniform)
  if (key0 + kPK - 1 > mwpos) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) st[u][j][i] = key0 + j * 16 + 4 * fg + i <= qp[u] ? st[u][j][i] : -INFINITY;
  }
  float alpha[2];
  bool grew = false;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    float bm = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) bm = fmaxf(bm, st[u][j][i]);
    bm = xor_max(bm) * a.scale_log2;
    const float mn = fmaxf(mrow[u], bm);         // finite unless EMPTY: every query sees key 0 in block 0
    const float me = EMPTY && mn == -INFINITY ? 0.0f : mn;
    grew = grew || mn > mrow[u];
    alpha[u] = __builtin_amdgcn_exp2f(mrow[u] - me);
    mrow[u] = mn;
    float rs = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(st[u][j][i], a.scale_log2, -me));
        st[u][j][i] = p;
        rs += p;
      }
    lrow[u] = lrow[u] * alpha[u] + xor_sum(rs);
  }
  if (__builtin_amdgcn_ballot_w64(grew)) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int d = 0; d < 8; ++d)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[u][d][i] *= alpha[u];
  }
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const f4 lo = st[u][2 * ks], hi = st[u][2 * ks + 1];
      pf[u][ks] = (h8){(half_t)lo[0], (half_t)lo[1], (half_t)lo[2], (half_t)lo[3],
                       (half_t)hi[0], (half_t)hi[1], (half_t)hi[2], (half_t)hi[3]};
    }
}
template <bool VTR = false>
__device__ __forceinline__ void attn_pv3(const unsigned char* Vt, const h8 (&pf)[2][2], int fr, int fg,
                                         f4 (&acc)[2][8]) {
#pragma unroll
  for (int d = 0; d < 8; ++d)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      h8 vf;
      if constexpr (VTR) {
        // within each 16-lane group the read hands lane i element j of lane i / 4 + 4 j's 8 bytes:
        // lane (fr, fg) asks for dims 16 d + 4 (fr & 3) .. + 3 of key 32 ks + 4 fg + fr / 4 and
        // receives dim 16 d + fr of keys 32 ks + 4 fg + 0..3; the second read takes keys + 16
        const int row = ks * 32 + 4 * fg + (fr >> 2);
        unsigned char* const vp = (unsigned char*)Vt + vsw(row, 2 * d + ((fr >> 1) & 1)) + (fr & 1) * 8;
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)vp);
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vp + 16 * kVRow));
        vf = __builtin_bit_cast(h8, (v8s){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
      } else {
        vf = __builtin_bit_cast(h8, *(const u4*)(Vt + (d * 16 + fr) * kVStride + (ks * 32 + 8 * fg) * 2));
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) acc[u][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[u][ks], acc[u][d], 0, 0, 0);
    }
}
template <bool EMPTY = false, bool VTR = false>
__device__ __forceinline__ void attn_block3(const PrefillAttnArgs& a, const unsigned char* Ks, const unsigned char* Vt,
                                            const h8 (&qf)[2][4], const int (&qp)[2], int key0, int mwpos, int fr,
                                            int fg, f4 (&acc)[2][8], float (&mrow)[2], float (&lrow)[2]) {
  h8 pf[2][2];
  attn_s3<EMPTY>(a, Ks, qf, qp, key0, mwpos, fr, fg, acc, mrow, lrow, pf);
  attn_pv3<VTR>(Vt, pf, fr, fg, acc);
}

template <bool VTR>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_attn_kernel3(PrefillAttnArgs a) {
  constexpr int VB = VTR ? kPK * kVRow : kPD * kVStride;   // bytes of one V stage
  __shared__ __align__(16) unsigned char Ks[2][kPK * kKStride];
  __shared__ __align__(16) unsigned char Vt[2][VB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, fg = lane >> 4;
  const int id = blockIdx.x, G = a.Hq / a.Hkv;
  int k, h;                                      // k-th tile slot of the order below; kv head k on XCD k % 8
  if (a.xcd_map) {
    const int x = id & 7, l = id >> 3, per_t = (a.Hkv >> 3) * G;
    k = l / per_t;
    const int r = l - k * per_t;
    h = (x + 8 * (r / G)) * G + r % G;
  } else {
    k = id / a.Hq;
    h = id % a.Hq;
  }
  // Tile order: the first half of the slots heaviest first (the most causal key blocks), the second
  // half lightest first.  When the grid fits the CUs in two workgroups each, a CU's second
  // workgroup then pairs tile T - 1 - j with tile j: every CU gets about the same number of blocks.
  // a.order == 0: heaviest first throughout.
  const int half = (a.tiles + 1) >> 1;
  const int t = a.order == 0 || k < half ? a.tiles - 1 - k : k - half;
  const int m0 = t * kPQ3, kvh = h / G;
  const int mlast = m0 + kPQ3 - 1 < a.M - 1 ? m0 + kPQ3 - 1 : a.M - 1;
  const int nkb = (a.pos0 + mlast) / kPK + 1;
  const int mw = m0 + 32 * wave;                 // the wavefront's first query
  const int wlast = mw < a.M ? a.pos0 + (mw + 31 < a.M - 1 ? mw + 31 : a.M - 1) : -1;   // its last visible key
  const half_t* kbase = a.k + (size_t)kvh * a.kv_hs;
  const half_t* vbase = a.v + (size_t)kvh * a.kv_hs;
  KvRegs r;
  auto load = [&](int key0) {
    if constexpr (VTR) kv_load_rm(a, kbase, vbase, key0, tid, r);
    else kv_load(a, kbase, vbase, key0, tid, lane, wave, r);
  };
  auto stage = [&](unsigned char* K, unsigned char* V) {
    if constexpr (VTR) kv_stage_rm(r, K, V, tid);
    else kv_stage3(r, K, V, tid, lane, wave);
  };
  load(0);
  h8 qf[2][4];
  int qp[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int mq = mw + 16 * u + fr;
    const half_t* qrow = a.q + (size_t)(mq < a.M ? mq : a.M - 1) * a.ldq + (size_t)h * kPD;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[u][ks] = __builtin_bit_cast(h8, *(const u4*)(qrow + ks * 32 + 8 * fg));
    qp[u] = a.pos0 + mq;
  }
  f4 acc[2][8];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[u][d] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
  float mrow[2] = {-INFINITY, -INFINITY}, lrow[2] = {0.0f, 0.0f};
  stage(Ks[0], Vt[0]);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int s = kb & 1;
    if (kb + 1 < nkb) load((kb + 1) * kPK);
    if (kb * kPK <= wlast)                       // blocks wholly past the wavefront's queries are skipped
      attn_block3<false, VTR>(a, Ks[s], Vt[s], qf, qp, kb * kPK, a.pos0 + mw, fr, fg, acc, mrow, lrow);
    if (kb + 1 < nkb) stage(Ks[s ^ 1], Vt[s ^ 1]);
    __syncthreads();
  }
  // o = O^T / l: lane holds dims 16 d + 4 fg .. + 3 of query mw + 16 u + fr
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int m = mw + 16 * u + fr;
    if (m >= a.M) continue;
    const float inv = 1.0f / lrow[u];
    half_t* orow = a.o + (size_t)m * a.ldo + (size_t)h * kPD + 4 * fg;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const h2 lo = {(half_t)(acc[u][d][0] * inv), (half_t)(acc[u][d][1] * inv)};
      const h2 hi = {(half_t)(acc[u][d][2] * inv), (half_t)(acc[u][d][3] * inv)};
      *(u2*)(orow + d * 16) = (u2){as_u32(lo), as_u32(hi)};
    }
  }
}

// ---- form 3 with each tile's key range split over two halves of one workgroup ----
// A causal prompt's query tiles differ in work by up to the tile count (tile t has 2t + 2 key
// blocks), and one 4-wavefront workgroup per tile leaves a CU with a heavy tile running alone long
// after its light neighbour is done.  Here an 8-wavefront workgroup takes one 128-query tile: waves
// 0-3 run form 3 over the first half of its key blocks, waves 4-7 over the second half, each half
// with its own double-buffered K and V stages (132 KB of LDS with row-major V, 140 KB with V^T: one
// workgroup per CU, two wavefronts per SIMD as in form 3), and the second half's running maxima, sums
// and accumulators are merged
// into the first's through LDS.  No tile costs more than half the longest key range, and with the
// tiles dispatched heaviest first over two rounds of workgroups the CUs finish together.
constexpr int kKB4 = kPK * kKStride;     // bytes of one K stage
constexpr int kX4 = 68;                  // floats per lane handed over: 2 x 8 accumulator f4s + 2 maxima + 2 sums

template <bool VTR>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_attn_kernel4(PrefillAttnArgs a) {
  constexpr int kVB4 = VTR ? kPK * kVRow : kPD * kVStride;   // bytes of one V stage
  __shared__ __align__(16) unsigned char lds[4 * kKB4 + 4 * kVB4];   // K stages [half][2], then V stages [half][2]
  static_assert(4 * 64 * kX4 * 4 <= 4 * kKB4, "the handover fits in the K stages");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hf = wave >> 2, w4 = wave & 3, htid = tid & 255;   // half, wavefront and thread within it
  const int fr = lane & 15, fg = lane >> 4;
  unsigned char* const Kh = lds + hf * 2 * kKB4;
  unsigned char* const Vh = lds + 4 * kKB4 + hf * 2 * kVB4;
  const int id = blockIdx.x, G = a.Hq / a.Hkv;
  int k, h;                                      // k-th tile slot, heaviest first; kv head k on XCD k % 8
  if (a.xcd_map) {
    const int x = id & 7, l = id >> 3, per_t = (a.Hkv >> 3) * G;
    k = l / per_t;
    const int r = l - k * per_t;
    h = (x + 8 * (r / G)) * G + r % G;
  } else {
    k = id / a.Hq;
    h = id % a.Hq;
  }
  const int t = a.tiles - 1 - k;
  const int m0 = t * kPQ3, kvh = h / G;
  const int mlast = m0 + kPQ3 - 1 < a.M - 1 ? m0 + kPQ3 - 1 : a.M - 1;
  const int nkb = (a.pos0 + mlast) / kPK + 1;
  const int nb0 = nkb >> 1;                      // the first half takes blocks [0, nb0), the second [nb0, nkb)
  const int kb0 = hf ? nb0 : 0, kb1 = hf ? nkb : nb0;
  const int trips = nkb - nb0;                   // the longer half's count: both halves meet every barrier
  const int mw = m0 + 32 * w4;                   // the wavefront's first query
  const int wlast = mw < a.M ? a.pos0 + (mw + 31 < a.M - 1 ? mw + 31 : a.M - 1) : -1;   // its last visible key
  const half_t* kbase = a.k + (size_t)kvh * a.kv_hs;
  const half_t* vbase = a.v + (size_t)kvh * a.kv_hs;
  KvRegs r;
  auto load = [&](int key0) {
    if constexpr (VTR) kv_load_rm(a, kbase, vbase, key0, htid, r);
    else kv_load(a, kbase, vbase, key0, htid, lane, w4, r);
  };
  auto stage = [&](unsigned char* K, unsigned char* V) {
    if constexpr (VTR) kv_stage_rm(r, K, V, htid);
    else kv_stage3(r, K, V, htid, lane, w4);
  };
  if (kb0 < kb1) load(kb0 * kPK);
  h8 qf[2][4];
  int qp[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int mq = mw + 16 * u + fr;
    const half_t* qrow = a.q + (size_t)(mq < a.M ? mq : a.M - 1) * a.ldq + (size_t)h * kPD;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[u][ks] = __builtin_bit_cast(h8, *(const u4*)(qrow + ks * 32 + 8 * fg));
    qp[u] = a.pos0 + mq;
  }
  f4 acc[2][8];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[u][d] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
  float mrow[2] = {-INFINITY, -INFINITY}, lrow[2] = {0.0f, 0.0f};
  if (kb0 < kb1) stage(Kh, Vh);
  __syncthreads();
  for (int i = 0; i < trips; ++i) {
    const int kb = kb0 + i, s = i & 1;
    const bool more = kb + 1 < kb1;              // uniform over the half
    if (more) load((kb + 1) * kPK);
    if (kb < kb1 && kb * kPK <= wlast)           // blocks wholly past the wavefront's queries are skipped
      attn_block3<true, VTR>(a, Kh + s * kKB4, Vh + s * kVB4, qf, qp, kb * kPK, a.pos0 + mw, fr, fg, acc, mrow, lrow);
    if (more) stage(Kh + (s ^ 1) * kKB4, Vh + (s ^ 1) * kVB4);
    __syncthreads();
  }
  // the second half hands over through the (now idle) K stages: lane-major, so the accesses are
  // consecutive words; wavefront w4 of each half holds the same queries in the same lanes
  float* const xw = (float*)lds + w4 * kX4 * 64 + lane;
  if (hf) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int d = 0; d < 8; ++d)
#pragma unroll
        for (int i = 0; i < 4; ++i) xw[((u * 8 + d) * 4 + i) * 64] = acc[u][d][i];
      xw[(64 + u) * 64] = mrow[u];
      xw[(66 + u) * 64] = lrow[u];
    }
  }
  __syncthreads();
  if (hf) return;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const float mb = xw[(64 + u) * 64], lb = xw[(66 + u) * 64];
    const float mn = fmaxf(mrow[u], mb);         // finite for every stored query: the half holding block 0 saw key 0
    const float sa = __builtin_amdgcn_exp2f(mrow[u] - mn);
    const float sb = mb == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mb - mn);
    lrow[u] = lrow[u] * sa + lb * sb;
#pragma unroll
    for (int d = 0; d < 8; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[u][d][i] = acc[u][d][i] * sa + xw[((u * 8 + d) * 4 + i) * 64] * sb;
  }
  // o = O^T / l: lane holds dims 16 d + 4 fg .. + 3 of query mw + 16 u + fr
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int m = mw + 16 * u + fr;
    if (m >= a.M) continue;
    const float inv = 1.0f / lrow[u];
    half_t* orow = a.o + (size_t)m * a.ldo + (size_t)h * kPD + 4 * fg;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const h2 lo = {(half_t)(acc[u][d][0] * inv), (half_t)(acc[u][d][1] * inv)};
      const h2 hi = {(half_t)(acc[u][d][2] * inv), (half_t)(acc[u][d][3] * inv)};
      *(u2*)(orow + d * 16) = (u2){as_u32(lo), as_u32(hi)};
    }
  }
}

// ---- form 4 with the second half one phase behind ----
// In form 4 both halves pass the block barrier together and run the same code, so the two wavefronts
// of a SIMD (one per half) issue their S^T products, then their softmax, then their P.V products at the
// same time.  Here the second half runs block i - 1's P.V before block i's S^T and softmax, so across a
// SIMD one wavefront's softmax (VALU) meets the other's products (MFMA).  The second half then reads
// block i - 1's V during block i, while block i + 1 is staged: its V takes three stages (the K stages
// stay two).  LDS: 148 KB with row-major V.  The arithmetic of every block is form 4's.
template <bool VTR>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_attn_kernel5(PrefillAttnArgs a) {
  constexpr int kVB5 = VTR ? kPK * kVRow : kPD * kVStride;   // bytes of one V stage
  // K stages [half][2], then V stages: the first half's two, the second half's three
  __shared__ __align__(16) unsigned char lds[4 * kKB4 + 5 * kVB5];
  static_assert(4 * 64 * kX4 * 4 <= 4 * kKB4, "the handover fits in the K stages");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hf = wave >> 2, w4 = wave & 3, htid = tid & 255;
  const int fr = lane & 15, fg = lane >> 4;
  unsigned char* const Kh = lds + hf * 2 * kKB4;
  unsigned char* const Vh = lds + 4 * kKB4 + hf * 2 * kVB5;
  const int id = blockIdx.x, G = a.Hq / a.Hkv;
  int k, h;                                      // k-th tile slot, heaviest first; kv head k on XCD k % 8
  if (a.xcd_map) {
    const int x = id & 7, l = id >> 3, per_t = (a.Hkv >> 3) * G;
    k = l / per_t;
    const int r = l - k * per_t;
    h = (x + 8 * (r / G)) * G + r % G;
  } else {
    k = id / a.Hq;
    h = id % a.Hq;
  }
  const int t = a.tiles - 1 - k;
  const int m0 = t * kPQ3, kvh = h / G;
  const int mlast = m0 + kPQ3 - 1 < a.M - 1 ? m0 + kPQ3 - 1 : a.M - 1;
  const int nkb = (a.pos0 + mlast) / kPK + 1;
  const int nb0 = nkb >> 1;
  const int kb0 = hf ? nb0 : 0, kb1 = hf ? nkb : nb0;
  const int trips = nkb - nb0;
  const int mw = m0 + 32 * w4;
  const int wlast = mw < a.M ? a.pos0 + (mw + 31 < a.M - 1 ? mw + 31 : a.M - 1) : -1;
  const half_t* kbase = a.k + (size_t)kvh * a.kv_hs;
  const half_t* vbase = a.v + (size_t)kvh * a.kv_hs;
  KvRegs r;
  auto load = [&](int key0) {
    if constexpr (VTR) kv_load_rm(a, kbase, vbase, key0, htid, r);
    else kv_load(a, kbase, vbase, key0, htid, lane, w4, r);
  };
  auto stage = [&](unsigned char* K, unsigned char* V) {
    if constexpr (VTR) kv_stage_rm(r, K, V, htid);
    else kv_stage3(r, K, V, htid, lane, w4);
  };
  // the half's V stage of its i-th block: two alternating for the first half, three for the second
  auto vstage = [&](int i) { return Vh + (hf ? i % 3 : i & 1) * kVB5; };
  if (kb0 < kb1) load(kb0 * kPK);
  h8 qf[2][4];
  int qp[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int mq = mw + 16 * u + fr;
    const half_t* qrow = a.q + (size_t)(mq < a.M ? mq : a.M - 1) * a.ldq + (size_t)h * kPD;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[u][ks] = __builtin_bit_cast(h8, *(const u4*)(qrow + ks * 32 + 8 * fg));
    qp[u] = a.pos0 + mq;
  }
  f4 acc[2][8];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[u][d] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
  float mrow[2] = {-INFINITY, -INFINITY}, lrow[2] = {0.0f, 0.0f};
  h8 pf[2][2];                                   // the second half: the previous block's P^T
  if (kb0 < kb1) stage(Kh, vstage(0));
  __syncthreads();
  for (int i = 0; i < trips; ++i) {
    const int kb = kb0 + i;
    const bool mine = kb < kb1, more = kb + 1 < kb1;   // uniform over the half
    if (more) load((kb + 1) * kPK);
    if (hf == 0) {
      if (mine && kb * kPK <= wlast) {
        h8 p0[2][2];
        attn_s3<false>(a, Kh + (i & 1) * kKB4, qf, qp, kb * kPK, a.pos0 + mw, fr, fg, acc, mrow, lrow, p0);
        attn_pv3<VTR>(vstage(i), p0, fr, fg, acc);
      }
    } else {
      // block i - 1's P.V (its V stays in its stage until block i + 2 is staged), then block i's S^T
      if (i > 0 && (kb - 1) * kPK <= wlast) attn_pv3<VTR>(vstage(i - 1), pf, fr, fg, acc);
      if (kb * kPK <= wlast)
        attn_s3<true>(a, Kh + (i & 1) * kKB4, qf, qp, kb * kPK, a.pos0 + mw, fr, fg, acc, mrow, lrow, pf);
    }
    if (more) stage(Kh + ((i + 1) & 1) * kKB4, vstage(i + 1));
    __syncthreads();
  }
  // the second half's last P.V: its V was staged before the last barrier and is not written again
  if (hf && trips > 0 && (kb1 - 1) * kPK <= wlast) attn_pv3<VTR>(vstage(trips - 1), pf, fr, fg, acc);
  float* const xw = (float*)lds + w4 * kX4 * 64 + lane;
  if (hf) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int d = 0; d < 8; ++d)
#pragma unroll
        for (int i = 0; i < 4; ++i) xw[((u * 8 + d) * 4 + i) * 64] = acc[u][d][i];
      xw[(64 + u) * 64] = mrow[u];
      xw[(66 + u) * 64] = lrow[u];
    }
  }
  __syncthreads();
  if (hf) return;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const float mb = xw[(64 + u) * 64], lb = xw[(66 + u) * 64];
    const float mn = fmaxf(mrow[u], mb);         // finite for every stored query: the half holding block 0 saw key 0
    const float sa = __builtin_amdgcn_exp2f(mrow[u] - mn);
    const float sb = mb == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mb - mn);
    lrow[u] = lrow[u] * sa + lb * sb;
#pragma unroll
    for (int d = 0; d < 8; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[u][d][i] = acc[u][d][i] * sa + xw[((u * 8 + d) * 4 + i) * 64] * sb;
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int m = mw + 16 * u + fr;
    if (m >= a.M) continue;
    const float inv = 1.0f / lrow[u];
    half_t* orow = a.o + (size_t)m * a.ldo + (size_t)h * kPD + 4 * fg;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const h2 lo = {(half_t)(acc[u][d][0] * inv), (half_t)(acc[u][d][1] * inv)};
      const h2 hi = {(half_t)(acc[u][d][2] * inv), (half_t)(acc[u][d][3] * inv)};
      *(u2*)(orow + d * 16) = (u2){as_u32(lo), as_u32(hi)};
    }
  }
}

}  // namespace afx

using namespace afx;

extern "C" {

// qkv [M][ldqkv] = [q (nq) | k (nk) | v (nk)] projection rows, q and k in RoPE-pair order
// (row 2i = dim i, 2i + 1 = dim i + dh/2 of a head).  Writes q [M][ldq] (natural order) and cache
// rows kc/vc[head][pos0 + m][dh] (head stride kv_hs elements, cache length kv_len).
int afx_qkv_split_rope(const void* qkv, int ldqkv, int M, int nq, int nk, int dh, const void* cos_tab,
                       const void* sin_tab, int pos0, int rope, void* q, int ldq, void* kcache, void* vcache,
                       long long kv_hs, int kv_len, void* stream) {
  AFX_REQUIRE(qkv && q && kcache && vcache && (!rope || (cos_tab && sin_tab)), "afx_qkv_split_rope: null pointer");
  AFX_REQUIRE(M >= 1 && dh >= 2 && dh % 2 == 0 && nq % dh == 0 && nk % dh == 0 && ldqkv >= nq + 2 * nk && ldq >= nq,
              "afx_qkv_split_rope: bad sizes");
  AFX_REQUIRE(pos0 >= 0 && pos0 + M <= kv_len && kv_hs >= (long long)kv_len * dh,
              "afx_qkv_split_rope: positions %d..%d outside the %d-row cache", pos0, pos0 + M - 1, kv_len);
  // 8 packed rows per thread where every row, table and cache row is 16-byte aligned (AFX_QKV_SPLIT_VEC=0
  // forces one pair per thread; the outputs are the same bits)
  const char* ve = getenv("AFX_QKV_SPLIT_VEC");
  const bool vec = (ve ? atoi(ve) != 0 : true) && dh % 8 == 0 && ldqkv % 8 == 0 && ldq % 8 == 0 && kv_hs % 8 == 0 &&
                   (((uintptr_t)qkv | (uintptr_t)q | (uintptr_t)kcache | (uintptr_t)vcache) & 15) == 0 &&
                   (!rope || (((uintptr_t)cos_tab | (uintptr_t)sin_tab) & 7) == 0);
  const long long n = (long long)M * ((nq + 2 * nk) / (vec ? 8 : 2));
  hipLaunchKernelGGL(vec ? qkv_split_rope_kernel8 : qkv_split_rope_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256),
                     0, (hipStream_t)stream, (const half_t*)qkv, ldqkv, M, nq, nk, dh, (const half_t*)cos_tab,
                     (const half_t*)sin_tab, pos0, rope, (half_t*)q, ldq, (half_t*)kcache, (half_t*)vcache, kv_hs);
  return check_launch("afx_qkv_split_rope");
}

// Causal GQA attention of M prompt queries (query m at position pos0 + m) over cache rows
// [0, pos0 + m] (head dim 128).  q [M][ldq] and o [M][ldo] hold head h at h * 128; the cache is
// k/v[kvh][Mmax][128] with head stride kv_hs elements.
int afx_prefill_attn(const void* q, int ldq, const void* kcache, const void* vcache, long long kv_hs, int Mmax,
                     void* o, int ldo, int M, int pos0, int Hq, int Hkv, int D, float scale, void* stream) {
  AFX_REQUIRE(q && kcache && vcache && o, "afx_prefill_attn: null pointer");
  AFX_REQUIRE(D == kPD, "afx_prefill_attn: head dim %d not supported (128)", D);
  AFX_REQUIRE(scale > 0.0f, "afx_prefill_attn: scale %g must be positive", (double)scale);
  AFX_REQUIRE(Hkv >= 1 && Hq % Hkv == 0, "afx_prefill_attn: bad heads Hq=%d Hkv=%d", Hq, Hkv);
  AFX_REQUIRE(M >= 1 && pos0 >= 0 && pos0 + M <= Mmax && kv_hs >= (long long)Mmax * D,
              "afx_prefill_attn: positions %d..%d outside the %d-row cache", pos0, pos0 + M - 1, Mmax);
  AFX_REQUIRE(ldq % 8 == 0 && ldq >= Hq * D && ldo >= Hq * D && kv_hs % 8 == 0 &&
              (((uintptr_t)q | (uintptr_t)kcache | (uintptr_t)vcache) & 15) == 0,
              "afx_prefill_attn: q / cache must be 16-byte aligned rows");
  PrefillAttnArgs a = {};
  a.q = (const half_t*)q; a.k = (const half_t*)kcache; a.v = (const half_t*)vcache; a.o = (half_t*)o;
  a.kv_hs = kv_hs; a.ldq = ldq; a.ldo = ldo; a.M = M; a.pos0 = pos0; a.Hq = Hq; a.Hkv = Hkv; a.Mmax = Mmax;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.tiles = (M + kPQ - 1) / kPQ;
  a.xcd_map = Hkv % 8 == 0;
  // Default: form 5 (form 4's arithmetic, bit for bit) while the causal part dominates (pos0 < M: tile
  // work grows with the tile index, and splitting each tile's keys evens the CUs out), form 3 once the
  // cached prefix does (a later chunk, whose tiles differ little and which the split forms' single
  // barrier domain per CU slows by 3-6%).
  const char* fe = getenv("AFX_PREFILL_ATTN_FORM");   // read per call: tests compare the forms in one process
  const int form_env = fe ? atoi(fe) : (pos0 < M ? 5 : 3);
  if (form_env == 1) {                             // single-buffered
    hipLaunchKernelGGL(prefill_attn_kernel, dim3(a.tiles, Hq), dim3(256), 0, (hipStream_t)stream, a);
  } else if (form_env == 2 || ldo % 4 != 0 || ((uintptr_t)o & 7) != 0) {   // pipelined, bit-identical to form 1
    hipLaunchKernelGGL(prefill_attn_kernel2, dim3(a.tiles * Hq), dim3(256), 0, (hipStream_t)stream, a);
  } else {
    a.tiles = (M + kPQ3 - 1) / kPQ3;
    const char* ve = getenv("AFX_PREFILL_ATTN_VTR");   // V staged row-major + transposing reads (1) or V^T (0)
    const bool vtr = ve ? atoi(ve) != 0 : true;
    if (form_env == 4) {                           // form 3 with each tile's keys split over two halves
      auto kfn = vtr ? prefill_attn_kernel4<true> : prefill_attn_kernel4<false>;
      hipLaunchKernelGGL(kfn, dim3(a.tiles * Hq), dim3(512), 0, (hipStream_t)stream, a);
    } else if (form_env == 5) {                    // form 4 with the second half one phase behind
      auto kfn = vtr ? prefill_attn_kernel5<true> : prefill_attn_kernel5<false>;
      hipLaunchKernelGGL(kfn, dim3(a.tiles * Hq), dim3(512), 0, (hipStream_t)stream, a);
    } else {                                       // transposed scores, 128 queries per workgroup (8-byte stores)
      const char* oe = getenv("AFX_PREFILL_ATTN_ORDER");
      a.order = oe ? atoi(oe) : 1;
      auto kfn = vtr ? prefill_attn_kernel3<true> : prefill_attn_kernel3<false>;
      hipLaunchKernelGGL(kfn, dim3(a.tiles * Hq), dim3(256), 0, (hipStream_t)stream, a);
    }
  }
  return check_launch("afx_prefill_attn");
}

}  // extern "C"
