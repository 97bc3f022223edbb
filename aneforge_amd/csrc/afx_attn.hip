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
// Partial kernel: grid (splits, KVH, B); one 256-thread workgroup handles `chunk`
// positions of one kv head for all G query heads that share it, so each K/V byte is read
// from HBM once per GQA group.  D/8 lanes cover one 16-byte row slice each; every lane
// issues all its K and V loads first.  The loads do not wait for the context length: row
// indices are clamped to the cache bound (max_len), and positions at or past the length are
// masked afterwards (scores to -inf, V to 0), so the device-side position load overlaps the
// KV stream.  Scores stay in registers (two-pass softmax inside the chunk), P@V accumulates
// in fp32, and the split partials (m, l, o[D]) go to a caller-provided fp32 workspace.
// The last workgroup to arrive for a (b, kvh) group (agent-scope release/acquire fences and
// an arrival counter, which that workgroup resets, so graph replays need no memset) rescales
// and sums the group's split partials and writes the fp16 output.  The workspace's counter
// tail must be zero before the first call.  That variant is opt-in (AFX_ATTN_FUSED_COMBINE=1):
// each workgroup's agent-scope release writes back its XCD's L2, which costs more than a
// second launch, so by default a separate combine kernel merges the splits.
#include <stdlib.h>
#include "afx_common.h"

namespace afx {

constexpr int kMaxSplits = 128;   // partials per (b, head); the chunk grows so ctx/chunk <= this

struct AttnArgs {
  const half_t* q;   // [B][Hq][D] via strides
  const half_t* k;   // cache: b*kv_bs + kvh*kv_hs + pos*D
  const half_t* v;
  half_t* o;         // same strides as q
  const half_t* mask;  // optional additive mask [B][mask_bs] over positions
  const int* pos;      // optional: ctx length of sequence b = pos[b] + 1 (device)
  float* ws_o;         // [B][Hq][D][nsp] split partial outputs (a (head, dim) row is contiguous)
  float* ws_ml;        // [B][Hq][2][nsp] split max (log2 domain) and row sum
  int* counters;       // [B][Hkv] arrival counters (zero before first use; reset by the last arrival)
  long long q_bs, q_hs, kv_bs, kv_hs;
  long long mask_bs;
  int B, Hq, Hkv, L, Mmax, chunk, nsplit, nsp, causal_off;  // causal_off < 0: no causal masking
  float scale_log2;    // scale * log2(e)
};

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
// v_permlane16_swap(a, b) exchanges the odd 16-lane rows of a with the even rows of b, and
// v_permlane32_swap the upper 32 lanes of a with the lower 32 lanes of b.  With b a copy of a,
// afterwards a and b hold each row (half) and its partner row (half), so op(a, b) reduces over
// lane pairs 16 (32) apart in every lane.  Issued as inline assembly on two distinct registers
// (the s_nop covers the VALU-write-then-permlane hazard): this compiler's builtin returns the
// same half twice when its two results are combined.
__device__ __forceinline__ void swap16(float v, float& r0, float& r1) {
  unsigned a = __builtin_bit_cast(unsigned, v), b;
  asm volatile("v_mov_b32 %1, %0\n\ts_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "=&v"(b));
  r0 = __builtin_bit_cast(float, a);
  r1 = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ void swap32(float v, float& r0, float& r1) {
  unsigned a = __builtin_bit_cast(unsigned, v), b;
  asm volatile("v_mov_b32 %1, %0\n\ts_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "=&v"(b));
  r0 = __builtin_bit_cast(float, a);
  r1 = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float swap16_sum(float v) { float a, b; swap16(v, a, b); return a + b; }
__device__ __forceinline__ float swap32_sum(float v) { float a, b; swap32(v, a, b); return a + b; }
__device__ __forceinline__ float swap16_max(float v) { float a, b; swap16(v, a, b); return fmaxf(a, b); }
__device__ __forceinline__ float swap32_max(float v) { float a, b; swap32(v, a, b); return fmaxf(a, b); }
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

template <int D, int G>
__device__ void combine_group(const AttnArgs& a, int b, int kvh, int ns);

template <int D, int G, int NSTEP, bool FUSED>
__global__ __launch_bounds__(256) void attn_partial_kernel(AttnArgs a) {
  constexpr int LPP = D / 8;        // lanes per position (16 B each)
  constexpr int PPS = 64 / LPP;     // positions per wavefront step
  constexpr int C = NSTEP * 4 * PPS;
  __shared__ float red_m[4][G], red_l[4][G];
  __shared__ float red_o[4][G][D];

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int p0 = split * C;
  const int dl = lane % LPP;       // which 8-dim slice
  const int pl = lane / LPP;       // which position within the step

  // K and V rows first (clamped to the cache bound, masked later), then q and the length
  const half_t* kb = a.k + (size_t)b * a.kv_bs + (size_t)kvh * a.kv_hs + dl * 8;
  const half_t* vb = a.v + (size_t)b * a.kv_bs + (size_t)kvh * a.kv_hs + dl * 8;
  u4 kv[NSTEP], vv[NSTEP];
  int posn[NSTEP];
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    const int p = p0 + (wave + 4 * s) * PPS + pl;
    posn[s] = p;
    const int pc = p < a.Mmax ? p : a.Mmax - 1;
    kv[s] = __builtin_nontemporal_load((const u4*)(kb + (size_t)pc * D));
  }
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    const int pc = posn[s] < a.Mmax ? posn[s] : a.Mmax - 1;
    vv[s] = __builtin_nontemporal_load((const u4*)(vb + (size_t)pc * D));
  }
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
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    const int pc = posn[s] < a.Mmax ? posn[s] : a.Mmax - 1;
    mk[s] = (float)mrow[a.mask ? pc : 0];
  }
  const int L = seq_len(a, b);
  const bool active = p0 < L;      // workgroup-uniform: an empty split only arrives (fused mode)

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
  for (int g = 0; g < G; ++g)
    mx[g] = fmaxf(fmaxf(red_m[0][g], red_m[1][g]), fmaxf(red_m[2][g], red_m[3][g]));

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
      const float p = exp2f(sc[s][g] - mx[g]);   // 0 for masked positions
      l[g] += p;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[g][i] = __builtin_fmaf(p, vf[i], o[g][i]);
    }
  }
  // reduce across the position groups of the wavefront
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = across_sum<LPP>(l[g]);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[g][i] = across_sum<LPP>(o[g][i]);
  }
  if (lane < LPP) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int i = 0; i < 8; ++i) red_o[wave][g][dl * 8 + i] = o[g][i];
    }
  }
  if (lane == 0)
#pragma unroll
    for (int g = 0; g < G; ++g) red_l[wave][g] = l[g];
  __syncthreads();

  const int NSP = a.nsp;
  for (int idx = threadIdx.x; active && idx < G * D; idx += 256) {
    const int g = idx / D, d = idx - g * D;
    const float acc = red_o[0][g][d] + red_o[1][g][d] + red_o[2][g][d] + red_o[3][g][d];
    const size_t bh = (size_t)b * a.Hq + kvh * G + g;
    a.ws_o[(bh * D + d) * NSP + split] = acc;
    if (d == 0) {
      a.ws_ml[(bh * 2 + 0) * NSP + split] = mx[g];
      a.ws_ml[(bh * 2 + 1) * NSP + split] = red_l[0][g] + red_l[1][g] + red_l[2][g] + red_l[3][g];
    }
  }

  if constexpr (!FUSED) return;            // a separate combine launch merges the splits
  // ---- the last workgroup of this (b, kvh) to arrive merges the group's split partials ----
  const int ns = (L + C - 1) / C;            // splits that hold data for this sequence
  __shared__ int s_last;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");   // this workgroup's partials, agent-visible
  __syncthreads();
  if (threadIdx.x == 0) {
    int* ctr = a.counters + (size_t)b * a.Hkv + kvh;
    const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == (int)gridDim.x - 1;
    if (s_last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // ready for the next call
  }
  __syncthreads();
  if (!s_last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");   // see the other workgroups' partials
  combine_group<D, G>(a, b, kvh, ns);
}

// Merge the ns split partials of one (b, kvh) group: per head the global max and denominator,
// then every output (head, dim) sums its contiguous row of partials with float4 loads.
template <int D, int G>
__device__ void combine_group(const AttnArgs& a, int b, int kvh, int ns) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int NSP = a.nsp;
  __shared__ float s_w[G][kMaxSplits];       // exp2(m_s - M) / den per (head, split)
  __shared__ float s_l[G][kMaxSplits];
  for (int i = threadIdx.x; i < G * ns; i += 256) {
    const int g = i / ns, sp = i - g * ns;
    const size_t bh = (size_t)b * a.Hq + kvh * G + g;
    s_w[g][sp] = __builtin_nontemporal_load(a.ws_ml + (bh * 2 + 0) * NSP + sp);
    s_l[g][sp] = __builtin_nontemporal_load(a.ws_ml + (bh * 2 + 1) * NSP + sp);
  }
  __syncthreads();
  for (int g = wave; g < G; g += 4) {
    float m = -INFINITY;
    for (int sp = lane; sp < ns; sp += 64) m = fmaxf(m, s_w[g][sp]);
    m = wave_max(m);
    float den = 0.0f;
    for (int sp = lane; sp < ns; sp += 64) den += exp2f(s_w[g][sp] - m) * s_l[g][sp];
    den = wave_sum(den);
    const float inv = 1.0f / den;
    for (int sp = lane; sp < ns; sp += 64) s_w[g][sp] = exp2f(s_w[g][sp] - m) * inv;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * D; idx += 256) {
    const int g = idx / D, d = idx - g * D;
    const float* row = a.ws_o + (((size_t)b * a.Hq + kvh * G + g) * D + d) * NSP;
    float num = 0.0f;
    for (int s0 = 0; s0 < ns; s0 += 32) {
      f4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        v[j] = s0 + 4 * j < ns ? __builtin_nontemporal_load((const f4*)(row + s0 + 4 * j)) : (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int sp = s0 + 4 * j;
        if (sp + 0 < ns) num = __builtin_fmaf(s_w[g][sp + 0], v[j].x, num);
        if (sp + 1 < ns) num = __builtin_fmaf(s_w[g][sp + 1], v[j].y, num);
        if (sp + 2 < ns) num = __builtin_fmaf(s_w[g][sp + 2], v[j].z, num);
        if (sp + 3 < ns) num = __builtin_fmaf(s_w[g][sp + 3], v[j].w, num);
      }
    }
    a.o[(size_t)b * a.q_bs + (size_t)(kvh * G + g) * a.q_hs + d] = (half_t)num;
  }
}

// Separate combine launch: one workgroup per (head, sequence).  Thread (d, part) owns output
// dim d and a contiguous range of the head's splits; every global load (the partial rows,
// m and l of split t, the length) is issued at once, so the kernel costs one memory round
// trip.  Split t's weight is exp2(m_t - max) / sum_s exp2(m_s - max) * l_s; splits at or past
// ceil(L / chunk) hold no data for this sequence and get weight 0.
template <int D, int NV4>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  constexpr int P = 256 / D;                    // threads per output dim
  // NV4: float4 partial loads per thread, >= ceil(nsp / 4 / P) (chosen by the host)
  const int h = blockIdx.x, b = blockIdx.y;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int d = t % D, part = t / D;
  const int NSP = a.nsp;                        // multiple of 4, <= kMaxSplits
  const int per = ((NSP / 4 + P - 1) / P) * 4;  // splits per part
  const int s0 = part * per;
  const size_t bh = (size_t)b * a.Hq + h;
  const float* row = a.ws_o + (bh * D + d) * NSP;
  f4 ov[NV4];
#pragma unroll
  for (int j = 0; j < NV4; ++j) {
    int s = s0 + 4 * j;
    s = s < NSP - 4 ? s : NSP - 4;              // clamped reads are masked by weight 0 below
    ov[j] = __builtin_nontemporal_load((const f4*)(row + s));
  }
  const int sm = t < NSP ? t : NSP - 1;
  float mt = __builtin_nontemporal_load(a.ws_ml + (bh * 2 + 0) * NSP + sm);
  float lt = __builtin_nontemporal_load(a.ws_ml + (bh * 2 + 1) * NSP + sm);
  const int L = seq_len(a, b);
  const int ns = (L + a.chunk - 1) / a.chunk;
  const bool valid = t < ns;
  mt = valid ? mt : -INFINITY;
  lt = valid ? lt : 0.0f;

  __shared__ float red_m[4], red_l[4], s_w[kMaxSplits], s_num[256];
  float mx = wave_max(mt);
  if (lane == 0) red_m[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
  const float w = valid ? exp2f(mt - mx) : 0.0f;
  const float den = wave_sum(w * lt);
  if (lane == 0) red_l[wave] = den;
  if (t < kMaxSplits) s_w[t] = w;
  __syncthreads();
  const float inv = 1.0f / (red_l[0] + red_l[1] + red_l[2] + red_l[3]);
  float num = 0.0f;
#pragma unroll
  for (int j = 0; j < NV4; ++j) {
    const int s = s0 + 4 * j;
    const float e[4] = {ov[j].x, ov[j].y, ov[j].z, ov[j].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int sp = s + i;
      const bool use = 4 * j < per && sp < ns;
      num = __builtin_fmaf(use ? s_w[sp < kMaxSplits ? sp : 0] : 0.0f, e[i], num);
    }
  }
  s_num[t] = num;
  __syncthreads();
  if (part == 0) {
    float tot = 0.0f;
#pragma unroll
    for (int q = 0; q < P; ++q) tot += s_num[q * D + d];
    a.o[(size_t)b * a.q_bs + (size_t)h * a.q_hs + d] = (half_t)(tot * inv);
  }
}

typedef void (*attn_fn)(AttnArgs);

template <int D>
static attn_fn pick_combine(int per4) {
  constexpr int P = 256 / D, MAX4 = kMaxSplits / 4 / P;
  if (per4 <= 2 && 2 <= MAX4) return attn_combine_kernel<D, 2 <= MAX4 ? 2 : MAX4>;
  if (per4 <= 4 && 4 <= MAX4) return attn_combine_kernel<D, 4 <= MAX4 ? 4 : MAX4>;
  if (per4 <= 8 && 8 <= MAX4) return attn_combine_kernel<D, 8 <= MAX4 ? 8 : MAX4>;
  if (per4 <= 16 && 16 <= MAX4) return attn_combine_kernel<D, 16 <= MAX4 ? 16 : MAX4>;
  return attn_combine_kernel<D, MAX4>;
}

template <int D, int G, bool F>
static attn_fn pick_steps(int nstep) {
  switch (nstep) {
    case 1: return attn_partial_kernel<D, G, 1, F>;
    case 2: return attn_partial_kernel<D, G, 2, F>;
    case 4: return attn_partial_kernel<D, G, 4, F>;
    case 8: return attn_partial_kernel<D, G, 8, F>;
    default: return attn_partial_kernel<D, G, 16, F>;
  }
}
template <int D, bool F>
static attn_fn pick_g(int G, int nstep) {
  switch (G) {
    case 1: return pick_steps<D, 1, F>(nstep);
    case 2: return pick_steps<D, 2, F>(nstep);
    case 4: return pick_steps<D, 4, F>(nstep);
    default: return pick_steps<D, 8, F>(nstep);
  }
}
// 0 = two launches (default: partials, then the combine kernel), 1 = combine in the
// last-arriving workgroup (release/acquire fences + arrival counter; built for D = 128).
static int g_attn_mode = -1;
static int attn_mode() {
  if (g_attn_mode < 0) {
    const char* e = getenv("AFX_ATTN_FUSED_COMBINE");
    g_attn_mode = e && atoi(e) == 1 ? 1 : 0;
  }
  return g_attn_mode;
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

// Steps per wavefront (chunk = nstep * 4 * (512 / D) positions): the largest chunk that still
// puts about one workgroup on every CU, and never more than kMaxSplits splits.  Returns 0 if
// even the largest chunk leaves more than kMaxSplits splits.
static int choose_nstep(int D, int B, int Hkv, int L, int want) {
  const int pps = 512 / D;
  auto splits = [&](int ns) { const int c = ns * 4 * pps; return (L + c - 1) / c; };
  if (want == 1 || want == 2 || want == 4 || want == 8 || want == 16) return splits(want) <= kMaxSplits ? want : 0;
  const int target = attn_cus();
  for (int ns = 16; ns >= 1; ns >>= 1) {
    if (splits(ns) > kMaxSplits) return ns == 16 ? 0 : ns * 2;
    if ((long long)B * Hkv * splits(ns) >= target) return ns;
  }
  return 1;
}

}  // namespace afx

using namespace afx;

extern "C" {

// Workspace bytes needed by afx_decode_attn for a given shape (max_len = the longest ctx).
long long afx_decode_attn_ws_bytes(int B, int Hq, int Hkv, int D, int max_len, int nstep_hint) {
  if (D != 8 && D != 16 && D != 32 && D != 64 && D != 128 && D != 256) return -1;
  const int ns = choose_nstep(D, B, Hkv, max_len, nstep_hint);
  if (ns == 0) return -2;
  const int chunk = ns * 4 * (512 / D);
  const long long nsplit = (max_len + chunk - 1) / chunk;
  const long long nsp = (nsplit + 3) / 4 * 4;
  return (long long)B * Hq * nsp * (D + 2) * 4 + (long long)B * Hkv * 4;
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
  a.chunk = ns * 4 * (512 / D);
  a.nsplit = (max_len + a.chunk - 1) / a.chunk;
  a.nsp = (a.nsplit + 3) / 4 * 4;
  a.ws_o = (float*)ws;
  a.ws_ml = a.ws_o + (size_t)B * Hq * D * a.nsp;
  a.counters = (int*)(a.ws_ml + (size_t)B * Hq * 2 * a.nsp);
  const bool fused = attn_mode() == 1 && D == 128;
  attn_fn fn;
  if (fused)
    fn = pick_g<128, true>(G, ns);
  else
    fn = D == 8 ? pick_g<8, false>(G, ns) : D == 16 ? pick_g<16, false>(G, ns) : D == 32 ? pick_g<32, false>(G, ns)
       : D == 64 ? pick_g<64, false>(G, ns) : D == 128 ? pick_g<128, false>(G, ns) : pick_g<256, false>(G, ns);
  hipLaunchKernelGGL(fn, dim3(a.nsplit, Hkv, B), dim3(256), 0, (hipStream_t)stream, a);
  int rc = check_launch("afx_decode_attn");
  if (rc || fused) return rc;
  const int per4 = ((a.nsp / 4) + (256 / D) - 1) / (256 / D);   // float4 loads each combine thread needs
  attn_fn cf = D == 8 ? pick_combine<8>(per4) : D == 16 ? pick_combine<16>(per4) : D == 32 ? pick_combine<32>(per4)
             : D == 64 ? pick_combine<64>(per4) : D == 128 ? pick_combine<128>(per4) : pick_combine<256>(per4);
  hipLaunchKernelGGL(cf, dim3(Hq, B), dim3(256), 0, (hipStream_t)stream, a);
  return check_launch("afx_decode_attn(combine)");
}

}  // extern "C"
