// Decode attention over a resident fp16 KV cache (flash-decoding / split-KV).
//
//   o[b, h, :] = softmax(q[b, h, :] . K[b, h/G, :L, :]^T * scale) @ V[b, h/G, :L, :]
//
// Semantics follow the reference's decode attention (aneforge/llm.py:214-237: GQA head h
// reads kv head h // G as in _repeat_kv3, llm.py:205-211; positions > pos masked) and the
// af.sdpa oracle (aneforge/_bridges/ane_sdpa_fused.py:57-68: fp32 scores with max
// subtraction, fp32 softmax, fp16 output).  Optional additive mask [B][Skv] and causal
// alignment for the af.sdpa entry (aneforge/graph.py:993-1040).
//
// Partial kernel: grid (splits, KVH, B); one workgroup of kAttnWaves wavefronts handles
// `chunk` positions of one kv head for all G query heads that share it, so each K/V byte is
// read from HBM once per GQA group.  D/8 lanes cover one 16-byte row slice each; every lane
// issues all its K and V loads first.  The loads do not wait for the context length: row
// indices are clamped to the cache bound (max_len), and positions at or past the length are
// masked afterwards (scores to -inf, V to 0), so the device-side position load overlaps the
// KV stream.  Scores stay in registers (two-pass softmax inside the chunk), P@V accumulates
// in fp32, and the per-position-group partial sums meet in LDS (one pass per head block)
// before the split partials (m, l, o[D]) go to a caller-provided fp32 workspace.
// Combine kernel: one thread per (head, dim) merges that dim's split partials in one memory
// round trip.  (A single-launch variant, in which the last workgroup to arrive merges the
// splits, needs an agent-scope release per workgroup; on this part that writes back the
// XCD's L2 and costs more than the second launch, so the merge is a launch of its own.)
#include <stdlib.h>
#include <mutex>
#include "afx_common.h"

namespace afx {

constexpr int kMaxSplits = 128;   // partials per (b, head); the chunk grows so ctx/chunk <= this

// Split partials of afx_decode_attn_noalloc: a file-scope device array instead of a caller
// workspace.  Every device the library runs on holds its own copy until the process ends.  In
// host code `scratch` only names the symbol; its device address comes from hipGetSymbolAddress,
// once per device (scratch_ptr below).  32 MiB holds B * Hq * splits * (D + 2) fp32 partials for
// every decode-attention shape of the 7B models at the default split size (B = 16, 32 heads,
// ctx 8192: 17 MB; B = 1: at most 1.1 MB).
constexpr long long kScratchBytes = 32ll << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct AttnArgs {
  const half_t* q;   // [B][Hq][D] via strides
  const half_t* k;   // cache: b*kv_bs + kvh*kv_hs + pos*D
  const half_t* v;
  half_t* o;         // same strides as q
  const half_t* mask;  // optional additive mask [B][mask_bs] over positions
  const int* pos;      // optional: ctx length of sequence b = pos[b] + 1 (device)
  float* ws_o;         // [B][Hq][nsp][D] split partial outputs (a split's head row is contiguous)
  float* ws_ml;        // [B][Hq][2][nsp] split max (log2 domain) and row sum
  long long q_bs, q_hs, kv_bs, kv_hs;
  long long mask_bs;
  int B, Hq, Hkv, L, Mmax, chunk, nsplit, nsp, causal_off;  // causal_off < 0: no causal masking
  float scale_log2;    // scale * log2(e)
  int xcd;             // 1: one-dimensional grids placed by XCD (see partial_coords)
};

// Workgroup b of a launch runs on XCD b % 8.  With a.xcd set (Hkv * B a multiple of 8), both
// launches use one-dimensional grids in which every workgroup of one (kv head, sequence) group g =
// kvh + Hkv * b runs on XCD g % 8: the partial workgroups of all its splits, and the combine
// workgroups of its query heads, which then read the partials from that XCD's L2 instead of HBM.
__device__ __forceinline__ void partial_coords(const AttnArgs& a, int& split, int& kvh, int& b) {
  if (!a.xcd) {
    split = blockIdx.x; kvh = blockIdx.y; b = blockIdx.z;
    return;
  }
  const int x = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int g = x + 8 * (slot / a.nsplit);
  split = slot % a.nsplit;
  kvh = g % a.Hkv;
  b = g / a.Hkv;
}
__device__ __forceinline__ void combine_coords(const AttnArgs& a, int& h, int& b) {
  if (!a.xcd) {
    h = blockIdx.x; b = blockIdx.y;
    return;
  }
  const int gq = a.Hq / a.Hkv;
  const int x = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int g = x + 8 * (slot / gq);
  h = (g % a.Hkv) * gq + slot % gq;
  b = g / a.Hkv;
}

__device__ __forceinline__ int seq_len(const AttnArgs& a, int b) {
  int L = a.pos ? a.pos[b] + 1 : a.L;
  if (L > a.Mmax) L = a.Mmax;
  if (a.causal_off >= 0) {
    const int lc = a.causal_off + b + 1;   // query b attends keys [0, causal_off + b]
    L = lc < L ? lc : L;
  }
  return L < 1 ? 1 : L;
}

// Cross-lane reductions without LDS (DPP row permutations and the gfx950 permlane swaps).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// swap16 / swap32 and their sums and maxima: afx_common.h.
// Sum over each aligned group of LPP consecutive lanes (quad_perm xor 1 / xor 2, then the half
// and full row mirrors, which pair the two halves of an 8 / 16 lane group); all lanes of the
// group receive the sum.
template <int LPP>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (LPP >= 2) v += dpp<0xB1>(v);    // quad_perm [1,0,3,2]
  if constexpr (LPP >= 4) v += dpp<0x4E>(v);    // quad_perm [2,3,0,1]
  if constexpr (LPP >= 8) v += dpp<0x141>(v);   // row_half_mirror
  if constexpr (LPP >= 16) v += dpp<0x140>(v);  // row_mirror
  if constexpr (LPP >= 32) v = swap16_sum(v);
  return v;
}
// Reduce over the lanes that hold the same slot of different groups (lane % LPP equal):
// rotations within a 16-lane row, then the cross-row swaps.
template <int LPP>
__device__ __forceinline__ float across_sum(float v) {
  if constexpr (LPP <= 1) v += dpp<0x121>(v);   // row_ror:1
  if constexpr (LPP <= 2) v += dpp<0x122>(v);   // row_ror:2
  if constexpr (LPP <= 4) v += dpp<0x124>(v);   // row_ror:4
  if constexpr (LPP <= 8) v += dpp<0x128>(v);   // row_ror:8
  if constexpr (LPP <= 16) v = swap16_sum(v);
  return swap32_sum(v);
}
template <int LPP>
__device__ __forceinline__ float across_max(float v) {
  if constexpr (LPP <= 1) v = fmaxf(v, dpp<0x121>(v));
  if constexpr (LPP <= 2) v = fmaxf(v, dpp<0x122>(v));
  if constexpr (LPP <= 4) v = fmaxf(v, dpp<0x124>(v));
  if constexpr (LPP <= 8) v = fmaxf(v, dpp<0x128>(v));
  if constexpr (LPP <= 16) v = swap16_max(v);
  return swap32_max(v);
}

// Full-wavefront reductions through DPP (row shifts, then the row broadcasts into lane 63,
// read back as a uniform scalar).  Lanes a step does not write keep `old`: 0 for a sum,
// their own value for a max.
template <int CTRL, int RMASK, bool MAX>
__device__ __forceinline__ float dpp_combine(float v) {
  const int iv = __builtin_bit_cast(int, v);
  const float o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(MAX ? iv : 0, iv, CTRL, RMASK, 0xf, false));
  return MAX ? fmaxf(v, o) : v + o;
}
template <bool MAX>
__device__ __forceinline__ float wave_reduce_uniform(float v) {
  v = dpp_combine<0x111, 0xf, MAX>(v);   // row_shr:1
  v = dpp_combine<0x112, 0xf, MAX>(v);   // row_shr:2
  v = dpp_combine<0x114, 0xf, MAX>(v);   // row_shr:4
  v = dpp_combine<0x118, 0xf, MAX>(v);   // row_shr:8: lane 15 of each row holds the row's result
  v = dpp_combine<0x142, 0xa, MAX>(v);   // row_bcast:15 into rows 1 and 3
  v = dpp_combine<0x143, 0xc, MAX>(v);   // row_bcast:31 into rows 2 and 3: lane 63 holds the total
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
// Sum over the lanes of a 16-lane row that hold the same slot (lane % LPP), for LPP <= 8.
template <int LPP>
__device__ __forceinline__ float row_slot_sum(float v) {
  if constexpr (LPP <= 1) v += dpp<0x121>(v);   // row_ror:1
  if constexpr (LPP <= 2) v += dpp<0x122>(v);   // row_ror:2
  if constexpr (LPP <= 4) v += dpp<0x124>(v);   // row_ror:4
  if constexpr (LPP <= 8) v += dpp<0x128>(v);   // row_ror:8
  return v;
}

constexpr int kRedBytes = 32768;   // LDS for the cross-position partial sums of one pass

// Partial kernel: grid (splits, KVH, B), NW wavefronts.  D/8 lanes cover one position's
// 16-byte slices; a wavefront step covers 64/(D/8) positions, the workgroup NSTEP steps.
template <int D, int G, int NSTEP, int NW>
__global__ __launch_bounds__(NW * 64) void attn_partial_kernel(AttnArgs a) {
  constexpr int LPP = D / 8;                   // lanes per position
  constexpr int PPS = 64 / LPP;                // positions per wavefront step
  constexpr int C = NSTEP * NW * PPS;          // positions per workgroup (the split chunk)
  constexpr int RG = LPP >= 16 ? PPS : 4;      // partial groups per wavefront after the in-row sums
  constexpr int Q = NW * RG;                   // partial groups per workgroup
  constexpr int HB0 = kRedBytes / (Q * D * 4);
  constexpr int HB = HB0 >= G ? G : (HB0 >= 1 ? HB0 : 1);   // heads per LDS reduction pass
  static_assert(G % HB == 0, "heads per pass must divide the group");
  __shared__ float red_m[NW][G];
  __shared__ float red_l[Q][G];
  __shared__ float red_o[Q][HB][D];

  int split, kvh, b;
  partial_coords(a, split, kvh, b);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int p0 = split * C;
  const int dl = lane % LPP;       // which 8-dim slice
  const int pl = lane / LPP;       // which position within the step

  // Loads: K rows, then q and the mask entries, then V rows (K/V row indices clamped to the
  // cache bound, positions past the length masked later), so the scores start while V is
  // still in flight.
  int posn[NSTEP], pcl[NSTEP];
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    posn[s] = p0 + (wave + NW * s) * PPS + pl;
    pcl[s] = posn[s] < a.Mmax ? posn[s] : a.Mmax - 1;
  }
  const half_t* kb = a.k + (size_t)b * a.kv_bs + (size_t)kvh * a.kv_hs + dl * 8;
  const half_t* vb = a.v + (size_t)b * a.kv_bs + (size_t)kvh * a.kv_hs + dl * 8;
  u4 kv[NSTEP], vv[NSTEP];
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) kv[s] = __builtin_nontemporal_load((const u4*)(kb + (size_t)pcl[s] * D));
  h2 qh[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const half_t* qp = a.q + (size_t)b * a.q_bs + (size_t)(kvh * G + g) * a.q_hs + dl * 8;
    u4 t = *(const u4*)qp;
    qh[g][0] = as_h2(t.x); qh[g][1] = as_h2(t.y); qh[g][2] = as_h2(t.z); qh[g][3] = as_h2(t.w);
  }
  // additive mask entries (af.sdpa), loaded unconditionally from a valid address
  float mk[NSTEP];
  const half_t* mrow = a.mask ? a.mask + (size_t)b * a.mask_bs : a.q;
  const int mstride = a.mask ? 1 : 0;
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) mk[s] = (float)mrow[pcl[s] * mstride];
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) vv[s] = __builtin_nontemporal_load((const u4*)(vb + (size_t)pcl[s] * D));
  const int L = seq_len(a, b);
  const bool active = p0 < L;      // workgroup-uniform: a split past the length stores an empty partial

  // scores (log2 domain), identical in all LPP lanes of a position
  float sc[NSTEP][G];
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    const h2 k0 = as_h2(kv[s].x), k1 = as_h2(kv[s].y), k2 = as_h2(kv[s].z), k3 = as_h2(kv[s].w);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float t = dot2(qh[g][0], k0, 0.0f);
      t = dot2(qh[g][1], k1, t);
      t = dot2(qh[g][2], k2, t);
      t = dot2(qh[g][3], k3, t);
      t = group_sum<LPP>(t);
      float x = t * a.scale_log2;
      if (a.mask) x += mk[s] * 1.4426950408889634f;
      sc[s][g] = posn[s] < L ? x : -INFINITY;
    }
  }

  // chunk max per head
  float mx[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float m = -INFINITY;
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) m = fmaxf(m, sc[s][g]);
    mx[g] = across_max<LPP>(m);
  }
  if (lane == 0)
#pragma unroll
    for (int g = 0; g < G; ++g) red_m[wave][g] = mx[g];
  __syncthreads();
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float m = red_m[0][g];
#pragma unroll
    for (int w = 1; w < NW; ++w) m = fmaxf(m, red_m[w][g]);
    mx[g] = m;
  }

  // probabilities, row sums and P@V
  float o[G][8];
  float l[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[g][i] = 0.0f;
  }
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    const bool ok = posn[s] < L;
    const h2 v0 = as_h2(ok ? vv[s].x : 0u), v1 = as_h2(ok ? vv[s].y : 0u);
    const h2 v2 = as_h2(ok ? vv[s].z : 0u), v3 = as_h2(ok ? vv[s].w : 0u);
    const float vf[8] = {(float)v0.x, (float)v0.y, (float)v1.x, (float)v1.y,
                         (float)v2.x, (float)v2.y, (float)v3.x, (float)v3.y};
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float p = __builtin_amdgcn_exp2f(sc[s][g] - mx[g]);   // 0 for masked positions
      l[g] += p;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[g][i] = __builtin_fmaf(p, vf[i], o[g][i]);
    }
  }
  // narrow heads: sum the positions that share a 16-lane row first
  if constexpr (LPP <= 8) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      l[g] = row_slot_sum<LPP>(l[g]);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[g][i] = row_slot_sum<LPP>(o[g][i]);
    }
  }
  // the remaining Q partial groups meet in LDS
  const bool writer = LPP >= 16 || (lane & 15) < LPP;
  const int q = wave * RG + (LPP >= 16 ? lane / LPP : lane >> 4);
  if (writer && dl == 0)
#pragma unroll
    for (int g = 0; g < G; ++g) red_l[q][g] = l[g];
  const int NSP = a.nsp;
#pragma unroll
  for (int h0 = 0; h0 < G; h0 += HB) {
    if (h0) __syncthreads();                  // the previous pass has read red_o
    if (writer) {
#pragma unroll
      for (int g = 0; g < HB; ++g) {
        *(f4*)&red_o[q][g][dl * 8] = (f4){o[h0 + g][0], o[h0 + g][1], o[h0 + g][2], o[h0 + g][3]};
        *(f4*)&red_o[q][g][dl * 8 + 4] = (f4){o[h0 + g][4], o[h0 + g][5], o[h0 + g][6], o[h0 + g][7]};
      }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < HB * D; idx += NW * 64) {
      const int g = idx / D, d = idx - g * D;
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < Q; ++j) acc += red_o[j][g][d];
      const size_t bh = (size_t)b * a.Hq + kvh * G + h0 + g;
      float* ocol = a.ws_o + bh * NSP * D + d;     // split t at ocol[t * D]: rows stored whole
      ocol[(size_t)split * D] = active ? acc : 0.0f;
      for (int t = a.nsplit; split == a.nsplit - 1 && t < NSP; ++t) ocol[(size_t)t * D] = 0.0f;   // padding splits
      if (d == 0) {
        float lt = 0.0f;
#pragma unroll
        for (int j = 0; j < Q; ++j) lt += red_l[j][h0 + g];
        float* mrow = a.ws_ml + bh * 2 * NSP;
        mrow[split] = active ? mx[h0 + g] : -INFINITY;
        mrow[NSP + split] = active ? lt : 0.0f;
        for (int t = a.nsplit; split == a.nsplit - 1 && t < NSP; ++t) {
          mrow[t] = -INFINITY;
          mrow[NSP + t] = 0.0f;
        }
      }
    }
  }
}

// Combine launch: grid (Hq, B), max(D, 64) threads; thread d owns output dim d and issues
// all its loads at once (its dim's value in each of 4 * NV4 split rows, coalesced across the
// threads, and the maxima and sums of splits lane and lane + 64), so the kernel costs one
// memory round trip.  Every split slot
// below nsp holds a partial from the same call (splits past the length and the padding slots
// hold m = -inf, l = 0, o = 0), so the weights need no length:
// w_t = exp2(m_t - max) / sum_s exp2(m_s - max) * l_s.  Every wavefront derives the weights
// itself with DPP reductions, so there is no barrier.
template <int D, int NV4>
__global__ __launch_bounds__(D < 64 ? 64 : D) void attn_combine_kernel(AttnArgs a) {
  constexpr int NT = D < 64 ? 64 : D;
  static_assert(kMaxSplits == 128 && NV4 * 4 <= kMaxSplits, "two split statistics per lane");
  int h, b;
  combine_coords(a, h, b);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int NSP = a.nsp;                        // multiple of 4, <= kMaxSplits
  const size_t bh = (size_t)b * a.Hq + h;
  const int d = t < D ? t : D - 1;
  const float* col = a.ws_o + bh * NSP * D + d;  // split t's value at col[t * D]
  float ov[4 * NV4];
#pragma unroll
  for (int j = 0; j < 4 * NV4; ++j) {
    const int s = j < NSP ? j : NSP - 1;           // clamped repeats get weight 0 below
    ov[j] = __builtin_nontemporal_load(col + (size_t)s * D);
  }
  const float* mrow = a.ws_ml + bh * 2 * NSP;
  const bool va = lane < NSP, vb = lane + 64 < NSP;
  const int sa = va ? lane : 0, sb = vb ? lane + 64 : 0;
  const float ma = __builtin_nontemporal_load(mrow + sa), la = __builtin_nontemporal_load(mrow + NSP + sa);
  const float mb = __builtin_nontemporal_load(mrow + sb), lb = __builtin_nontemporal_load(mrow + NSP + sb);
  const float mx = wave_reduce_uniform<true>(fmaxf(va ? ma : -INFINITY, vb ? mb : -INFINITY));
  const float wa = va ? __builtin_amdgcn_exp2f(ma - mx) : 0.0f;   // exp2(-inf) = 0 for empty splits
  const float wb = vb ? __builtin_amdgcn_exp2f(mb - mx) : 0.0f;
  const float inv = 1.0f / wave_reduce_uniform<false>(wa * la + wb * lb);
  __shared__ float s_w[NT / 64][kMaxSplits];    // per-wavefront copy: written and read by one wavefront
  s_w[wave][lane] = wa * inv;
  s_w[wave][lane + 64] = wb * inv;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float num = 0.0f;
#pragma unroll
  for (int j = 0; j < NV4; ++j) {
    const f4 w = *(const f4*)&s_w[wave][4 * j];
    num = __builtin_fmaf(w.x, ov[4 * j + 0], num);
    num = __builtin_fmaf(w.y, ov[4 * j + 1], num);
    num = __builtin_fmaf(w.z, ov[4 * j + 2], num);
    num = __builtin_fmaf(w.w, ov[4 * j + 3], num);
  }
  if (t < D) a.o[(size_t)b * a.q_bs + (size_t)h * a.q_hs + d] = (half_t)num;
}

typedef void (*attn_fn)(AttnArgs);

// Split rows read by each combine thread: 4 * NV4, the smallest of 4, 8, 12, 16, 24, 32, 48,
// 64, 96, 128 covering nsp.
template <int D>
static attn_fn pick_combine(int nsp) {
  const int n4 = (nsp + 3) / 4;
  if (n4 <= 1) return attn_combine_kernel<D, 1>;
  if (n4 <= 2) return attn_combine_kernel<D, 2>;
  if (n4 <= 3) return attn_combine_kernel<D, 3>;
  if (n4 <= 4) return attn_combine_kernel<D, 4>;
  if (n4 <= 6) return attn_combine_kernel<D, 6>;
  if (n4 <= 8) return attn_combine_kernel<D, 8>;
  if (n4 <= 12) return attn_combine_kernel<D, 12>;
  if (n4 <= 16) return attn_combine_kernel<D, 16>;
  if (n4 <= 24) return attn_combine_kernel<D, 24>;
  return attn_combine_kernel<D, 32>;
}

constexpr int kAttnWaves = 4;   // wavefronts per partial workgroup

template <int D, int G>
static attn_fn pick_steps(int nstep) {
  switch (nstep) {
    case 1: return attn_partial_kernel<D, G, 1, kAttnWaves>;
    case 2: return attn_partial_kernel<D, G, 2, kAttnWaves>;
    case 3: return attn_partial_kernel<D, G, 3, kAttnWaves>;
    case 4: return attn_partial_kernel<D, G, 4, kAttnWaves>;
    case 5: return attn_partial_kernel<D, G, 5, kAttnWaves>;
    case 6: return attn_partial_kernel<D, G, 6, kAttnWaves>;
    case 8: return attn_partial_kernel<D, G, 8, kAttnWaves>;
    default: return attn_partial_kernel<D, G, 16, kAttnWaves>;
  }
}
template <int D>
static attn_fn pick_g(int G, int nstep) {
  switch (G) {
    case 1: return pick_steps<D, 1>(nstep);
    case 2: return pick_steps<D, 2>(nstep);
    case 4: return pick_steps<D, 4>(nstep);
    default: return pick_steps<D, 8>(nstep);
  }
}

static int attn_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    hipDeviceProp_t p;
    cus = hipGetDeviceProperties(&p, dev) == hipSuccess ? p.multiProcessorCount : 256;
  }
  return cus;
}

constexpr int kNsteps[] = {1, 2, 3, 4, 5, 6, 8, 16};   // instantiated steps per wavefront

// Steps per wavefront (chunk = nstep * kAttnWaves * (512 / D) positions).  Every partial
// workgroup streams its chunk at once and the launch ends with its slowest workgroup, so the cost
// of a split size is the number of dispatch rounds (workgroups / CUs, rounded up) times the chunk;
// the cheapest wins, on a tie the larger chunk (fewer partials to merge) up to 8 steps: 16 steps
// only when strictly cheaper (where the model ties them, 8 steps measured 4-8% faster than 16 on
// MI355X at ctx 2048 and 8192, B = 1..16).  A few workgroups past a
// whole round share CUs with others and set the launch's end: at the 7B cache bound of 2184 rows,
// 64-position chunks give 280 workgroups for 256 CUs and an 80-position chunk 224.  Never more
// than kMaxSplits splits; returns 0 if even the largest chunk leaves more.
static int choose_nstep(int D, int B, int Hkv, int L, int want) {
  const int pps = 512 / D;
  auto splits = [&](int ns) { const int c = ns * kAttnWaves * pps; return (L + c - 1) / c; };
  if (want == 0) {                              // tuning override: AFX_ATTN_NSTEP=1|2|3|4|5|6|8|16
    static int env = -1;
    if (env < 0) {
      const char* e = getenv("AFX_ATTN_NSTEP");
      env = e ? atoi(e) : 0;
    }
    want = env;
  }
  for (int ns : kNsteps)
    if (want == ns) return splits(want) <= kMaxSplits ? want : 0;
  const long long cus = attn_cus();
  int best = 0;
  long long best_cost = 0;
  for (int ns : kNsteps) {
    if (splits(ns) > kMaxSplits) continue;
    const long long wgs = (long long)B * Hkv * splits(ns);
    const long long cost = (wgs + cus - 1) / cus * ns;
    if (!best || cost < best_cost || (cost == best_cost && ns <= 8)) { best = ns; best_cost = cost; }
  }
  return best;
}

}  // namespace afx

using namespace afx;

extern "C" {

// Workspace bytes needed by afx_decode_attn for a given shape (max_len = the longest ctx).
long long afx_decode_attn_ws_bytes(int B, int Hq, int Hkv, int D, int max_len, int nstep_hint) {
  if (D != 8 && D != 16 && D != 32 && D != 64 && D != 128 && D != 256) return -1;
  const int ns = choose_nstep(D, B, Hkv, max_len, nstep_hint);
  if (ns == 0) return -2;
  const int chunk = ns * kAttnWaves * (512 / D);
  const long long nsplit = (max_len + chunk - 1) / chunk;
  const long long nsp = (nsplit + 3) / 4 * 4;
  return (long long)B * Hq * nsp * (D + 2) * 4;
}

// q/o: element (b, h, d) at b*q_bs + h*q_hs + d.  K/V: (b, kvh, p, d) at b*kv_bs + kvh*kv_hs + p*D + d.
// Context length: pos ? pos[b]+1 : ctx_len (clamped to max_len).  causal_off >= 0 additionally
// limits query b to keys [0, causal_off + b] (af.sdpa is_causal with Sq == Skv: causal_off = 0).
// mask: optional fp16 additive mask, element (b, p) at b*mask_bs + p.
int afx_decode_attn(const void* q, const void* k, const void* v, void* o, long long q_bs, long long q_hs,
                    long long kv_bs, long long kv_hs, int B, int Hq, int Hkv, int D, int ctx_len,
                    const int* pos, int max_len, const void* mask, long long mask_bs, int causal_off,
                    float scale, void* ws, long long ws_bytes, int nstep_hint, void* stream) {
  AFX_REQUIRE(q && k && v && o && ws, "afx_decode_attn: null pointer");
  AFX_REQUIRE(D == 8 || D == 16 || D == 32 || D == 64 || D == 128 || D == 256,
              "afx_decode_attn: head dim %d not supported (8, 16, 32, 64, 128, 256)", D);
  AFX_REQUIRE(B >= 1 && Hkv >= 1 && Hq % Hkv == 0, "afx_decode_attn: bad heads Hq=%d Hkv=%d", Hq, Hkv);
  const int G = Hq / Hkv;
  AFX_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "afx_decode_attn: GQA group %d not in {1,2,4,8}", G);
  AFX_REQUIRE(max_len >= 1 && (pos || (ctx_len >= 1 && ctx_len <= max_len)),
              "afx_decode_attn: ctx_len=%d outside [1, max_len=%d]", ctx_len, max_len);
  AFX_REQUIRE((q_hs % 8) == 0 && (q_bs % 8) == 0 && (kv_hs % 8) == 0 && (kv_bs % 8) == 0,
              "afx_decode_attn: strides must be multiples of 8 elements");
  const long long need = afx_decode_attn_ws_bytes(B, Hq, Hkv, D, max_len, nstep_hint);
  AFX_REQUIRE(need > 0, "afx_decode_attn: max_len=%d needs more than %d splits", max_len, kMaxSplits);
  AFX_REQUIRE(ws_bytes >= need, "afx_decode_attn: workspace %lld B < %lld B", ws_bytes, need);
  AttnArgs a = {};
  a.q = (const half_t*)q; a.k = (const half_t*)k; a.v = (const half_t*)v; a.o = (half_t*)o;
  a.mask = (const half_t*)mask; a.pos = pos;
  a.q_bs = q_bs; a.q_hs = q_hs; a.kv_bs = kv_bs; a.kv_hs = kv_hs; a.mask_bs = mask_bs;
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.L = ctx_len; a.Mmax = max_len; a.causal_off = causal_off;
  a.scale_log2 = scale * 1.4426950408889634f;
  const int ns = choose_nstep(D, B, Hkv, max_len, nstep_hint);
  a.chunk = ns * kAttnWaves * (512 / D);
  a.nsplit = (max_len + a.chunk - 1) / a.chunk;
  a.nsp = (a.nsplit + 3) / 4 * 4;
  a.ws_o = (float*)ws;
  a.ws_ml = a.ws_o + (size_t)B * Hq * D * a.nsp;
  const attn_fn fn = D == 8 ? pick_g<8>(G, ns) : D == 16 ? pick_g<16>(G, ns) : D == 32 ? pick_g<32>(G, ns)
                   : D == 64 ? pick_g<64>(G, ns) : D == 128 ? pick_g<128>(G, ns) : pick_g<256>(G, ns);
  static int xcd_env = -1;                         // tuning override: AFX_ATTN_XCD=0 keeps the 3-D grids
  if (xcd_env < 0) {
    const char* e = getenv("AFX_ATTN_XCD");
    xcd_env = e ? atoi(e) != 0 : 1;
  }
  a.xcd = xcd_env && (Hkv * B) % 8 == 0;
  if (a.xcd) hipLaunchKernelGGL(fn, dim3(a.nsplit * Hkv * B), dim3(kAttnWaves * 64), 0, (hipStream_t)stream, a);
  else hipLaunchKernelGGL(fn, dim3(a.nsplit, Hkv, B), dim3(kAttnWaves * 64), 0, (hipStream_t)stream, a);
  int rc = check_launch("afx_decode_attn");
  if (rc) return rc;
  const attn_fn cf = D == 8 ? pick_combine<8>(a.nsp) : D == 16 ? pick_combine<16>(a.nsp) : D == 32 ? pick_combine<32>(a.nsp)
                   : D == 64 ? pick_combine<64>(a.nsp) : D == 128 ? pick_combine<128>(a.nsp) : pick_combine<256>(a.nsp);
  if (a.xcd) hipLaunchKernelGGL(cf, dim3(Hq * B), dim3(D < 64 ? 64 : D), 0, (hipStream_t)stream, a);
  else hipLaunchKernelGGL(cf, dim3(Hq, B), dim3(D < 64 ? 64 : D), 0, (hipStream_t)stream, a);
  return check_launch("afx_decode_attn(combine)");
}

}  // extern "C"

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices];   // device address of `scratch` on each device, once resolved

// The calling thread's current device's copy of `scratch` (resolved on its first call there).
int scratch_ptr(void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error("afx_decode_attn_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error("afx_decode_attn_noalloc: device %d >= %d", dev, kMaxDevices);
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    if (e != hipSuccess) return set_error("afx_decode_attn_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
    if (sdev != dev)
      return set_error("afx_decode_attn_noalloc: stream is on device %d, current device is %d", (int)sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    // The first call on a device may come while the caller captures a graph: the symbol lookup is no
    // stream work, so this thread's capture mode is relaxed around it (and restored) so that a
    // capture in the global mode does not reject it.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const hipError_t em = hipThreadExchangeStreamCaptureMode(&mode);
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (em == hipSuccess) (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess || !p)
      return set_error("afx_decode_attn_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return 0;
}

}  // namespace

extern "C" {

// afx_decode_attn with its split partials in the device's `scratch` array: no allocation and
// no workspace argument.  Shapes whose partials exceed kScratchBytes are rejected.  Calls that
// overlap on one device share the array and race; every split slot is written by each call
// before the combine reads it, so nothing needs clearing between calls.
int afx_decode_attn_noalloc(const void* q, const void* k, const void* v, void* o, long long q_bs,
                            long long q_hs, long long kv_bs, long long kv_hs, int B, int Hq, int Hkv, int D,
                            int ctx_len, const int* pos, int max_len, const void* mask, long long mask_bs,
                            int causal_off, float scale, int nstep_hint, void* stream) {
  const long long need = afx_decode_attn_ws_bytes(B, Hq, Hkv, D, max_len, nstep_hint);
  AFX_REQUIRE(need != -1, "afx_decode_attn_noalloc: head dim %d not supported (8, 16, 32, 64, 128, 256)", D);
  AFX_REQUIRE(need > 0, "afx_decode_attn_noalloc: max_len=%d needs more than %d splits", max_len, kMaxSplits);
  AFX_REQUIRE(need <= kScratchBytes,
              "afx_decode_attn_noalloc: B=%d Hq=%d D=%d max_len=%d needs %lld B of split partials, more than "
              "the %lld B scratch array (use afx_decode_attn with a workspace)",
              B, Hq, D, max_len, need, kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_ptr(stream, &ws);
  if (rc) return rc;
  return afx_decode_attn(q, k, v, o, q_bs, q_hs, kv_bs, kv_hs, B, Hq, Hkv, D, ctx_len, pos, max_len, mask,
                         mask_bs, causal_off, scale, ws, kScratchBytes, nstep_hint, stream);
}

}  // extern "C"
