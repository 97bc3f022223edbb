// Sparse MoE dispatch for decode (replaces the reference's dense all-expert compute,
// aneforge/moe.py:40-63, with identical math: unselected experts have gate weight 0).
//
//  afx_moe_topk     softmax over E router logits (fp32), probabilities rounded to fp16, k
//                   rounds of "row max, lowest index among exact fp16 ties" (moe.py:21-37),
//                   optional renormalisation (moe.py:55-56); then device-side bucketing:
//                   cnt[e] and list[e][i] = t*k + slot, in token order (deterministic).
//  afx_moe_gateup   per active expert e: act[t*k+slot] = silu(g) * u over the tokens routed to e,
//                   weights [E][2F][D] with gate/up rows interleaved (2i, 2i+1).
//  afx_moe_down     per active expert e: y[t*k+slot] = act[t*k+slot] @ Wd_e^T, Wd [E][D][F] (fp32 out).
//  afx_moe_combine  out[t] = fp16(h[t] + fp16(sum_slot g[t,slot] * fp16(y[t*k+slot]))) (+ shared).
// The grid covers all E experts; workgroups of experts with no tokens exit at once, so the
// launch shape is fixed and the whole layer is graph-capturable (no host round trip).
#include "afx_gemv_core.h"
#include "afx_gemv_impl.h"
#include "afx_mfma.h"

namespace afx {

// One token's routing, by one wavefront: lane l holds the logits of experts l, l + 64, ...
// (-inf past E).  Softmax in fp32, probabilities rounded to fp16, k rounds of "row max, lowest
// index among exact fp16 ties" (moe.py:21-37), optional renormalisation (moe.py:55-56).  Lane
// r < k ends with round r's expert and gate weight.
template <int J>
__device__ __forceinline__ void topk_token(const float (&lg)[J], int lane, int E, int k, int renorm, float& gate_r,
                                           int& sel_r) {
  if (J == 1 && E <= 16) {
    // up to 16 experts, all in lanes 0..15 (DPP row 0): the same steps with row reductions, whose
    // results lane 0 broadcasts
    const bool own = lane < E;
    const float m = lane0(row16_max(own ? lg[0] : -INFINITY));
    const float ex = own ? expf(lg[0] - m) : 0.0f;
    const float inv = 1.0f / lane0(row16_sum(ex));
    float p = own ? (float)(half_t)(ex * inv) : -1.0f;
    float tot = 0.0f, mine = 0.0f;
    int mine_e = 0;
    for (int r = 0; r < k; ++r) {
      const float wb = lane0(row16_max(p));
      const float cand = p == wb ? (float)lane : 3.0e38f;
      const int win = (int)lane0(-row16_max(-cand));   // lowest lane holding the maximum
      if (lane == win) p = -1.0f;                        // taken
      if (lane == r) { mine = wb; mine_e = win; }
      tot += wb;
    }
    gate_r = renorm ? mine / tot : mine;
    sel_r = mine_e;
    return;
  }
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < J; ++j) m = fmaxf(m, lg[j]);
  m = wave_max(m);
  float ex[J];
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    ex[j] = lane + 64 * j < E ? expf(lg[j] - m) : 0.0f;
    sum += ex[j];
  }
  const float inv = 1.0f / wave_sum(sum);
  // probabilities rounded to fp16 (-1 marks experts this lane does not own)
  float p[J];
#pragma unroll
  for (int j = 0; j < J; ++j) p[j] = lane + 64 * j < E ? (float)(half_t)(ex[j] * inv) : -1.0f;
  // k rounds: max of the fp16 probabilities, lowest index on exact ties; lane r keeps round r
  float tot = 0.0f, mine = 0.0f;
  int mine_e = 0;
  for (int r = 0; r < k; ++r) {
    float best = -1.0f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (p[j] > best) { best = p[j]; bi = lane + 64 * j; }   // ascending index: first max wins
    const float wb = wave_max(best);
    float cand = best == wb ? (float)bi : 3.0e38f;
    cand = -wave_max(-cand);                     // lowest index holding the maximum
    const int win = (int)cand;
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (lane + 64 * j == win) p[j] = -1.0f;    // taken
    if (lane == r) { mine = wb; mine_e = win; }
    tot += wb;
  }
  gate_r = renorm ? mine / tot : mine;
  sel_r = mine_e;
}

// Device bucketing of the T * k selections s_sel (token-major): cnt[e] and list[e][i] = t*k + slot
// in token order (deterministic), threads striding over the experts.
__device__ __forceinline__ void bucket_experts(const int* s_sel, int T, int E, int k, int* __restrict__ cnt,
                                               int* __restrict__ list) {
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int c = 0;
    for (int i = 0; i < T * k; ++i)
      if (s_sel[i] == e) list[(size_t)e * T + c++] = i;
    cnt[e] = c;
  }
}

// The same buckets from one wavefront for at most 64 selections (lane i holds entry i, -1 for none):
// per expert one ballot, each entry's place is the count of earlier entries with its expert.
__device__ __forceinline__ void bucket_experts_wave(int s, int lane, int T, int E, int* __restrict__ cnt,
                                                    int* __restrict__ list) {
  const unsigned long long below = (1ull << lane) - 1ull;
  for (int e = 0; e < E; ++e) {
    const unsigned long long m = __ballot(s == e);
    if (s == e) list[(size_t)e * T + __popcll(m & below)] = lane;
    if (lane == 0) cnt[e] = __popcll(m);
  }
}

// One wavefront per token (tokens w, w + W, ... for the workgroup's W wavefronts); lane l owns
// experts l, l + 64, ..., l + 64 * (J - 1), J = ceil(E / 64) rounded up to an instantiated count.
template <int J>
__global__ __launch_bounds__(1024) void moe_topk_kernel(const float* __restrict__ logits, int T, int E, int k,
                                                        int renorm, float* __restrict__ gate,
                                                        int* __restrict__ sel, int* __restrict__ cnt,
                                                        int* __restrict__ list) {
  extern __shared__ int s_sel[];   // [T][k]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  for (int tt = wave; tt < T; tt += nw) {
    const float* lr = logits + (size_t)tt * E;
    float lg[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int e = lane + 64 * j;
      lg[j] = e < E ? lr[e] : -INFINITY;
    }
    float g_r;
    int s_r;
    topk_token<J>(lg, lane, E, k, renorm, g_r, s_r);
    if (lane < k) {
      gate[(size_t)tt * k + lane] = g_r;
      sel[(size_t)tt * k + lane] = s_r;
      s_sel[tt * k + lane] = s_r;
    }
  }
  __syncthreads();
  bucket_experts(s_sel, T, E, k, cnt, list);
}

// The router in one workgroup for a decode batch (T <= 16 tokens, E <= 16 experts, D <= 4096):
// RMSNorm of h into hn (global and LDS), the logits hn @ router^T on MFMA, then top-k and
// bucketing.  Each part repeats the arithmetic of the stand-alone kernels step for step, so the
// outputs are those of afx_rmsnorm + afx_linear (fp16 router, fp32 logits, from 4 rows up, where
// afx_linear takes MFMA) + afx_moe_topk, bit for bit: the norm's per-thread partials of a 256-thread row reduction (lane l adds thread
// l + 64j's chunks into partial j, each partial summed across the wavefront, then the four in
// order), and the logits' K ranges, MFMA order and cross-wavefront sum of the skinny MFMA kernel
// with NWR wavefronts (its choice for this K).
constexpr int kRouteMaxD = 4096;
constexpr int kRouteRow = kRouteMaxD + 8;          // halves per LDS row of hn (16 bytes of padding)
template <int NWR>
__global__ __launch_bounds__(1024) void moe_route_kernel(const half_t* __restrict__ h, int ldh,
                                                         const half_t* __restrict__ gamma, float eps,
                                                         const half_t* __restrict__ router, int T, int E, int D,
                                                         int k, int renorm, half_t* __restrict__ hn, int ldo,
                                                         float* __restrict__ logits_out, float* __restrict__ gate,
                                                         int* __restrict__ sel, int* __restrict__ cnt,
                                                         int* __restrict__ list) {
  __shared__ __align__(16) half_t hn_l[16][kRouteRow];
  __shared__ f4 red[NWR][64];
  __shared__ float lg_l[16][16];                   // [token][expert]
  __shared__ int s_sel[16 * 64];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nv = D >> 3;                           // 16-byte chunks of a row
  constexpr int kCh = kRouteMaxD / 8 / 64;         // chunks per lane (lane l: chunks l + 64 i)
  // RMSNorm: wavefront t normalises token t, every load issued before the first sum
  if (wave < T) {
    const u4* xr = (const u4*)(h + (size_t)wave * ldh);
    const u4* gr = (const u4*)gamma;
    u4 xv[kCh], gv[kCh];
#pragma unroll
    for (int i = 0; i < kCh; ++i) {
      const int f = lane + 64 * i < nv ? lane + 64 * i : 0;
      xv[i] = xr[f];
      gv[i] = gr[f];
    }
    // thread 64 j + l of the 256-thread reduction holds chunks l + 64 j + 256 m, m = 0, 1, ...
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float part = 0.0f;
#pragma unroll
      for (int i = j; i < kCh; i += 4) {
        float q = dot2(as_h2(xv[i].x), as_h2(xv[i].x), 0.0f);
        q = dot2(as_h2(xv[i].y), as_h2(xv[i].y), q);
        q = dot2(as_h2(xv[i].z), as_h2(xv[i].z), q);
        q = dot2(as_h2(xv[i].w), as_h2(xv[i].w), q);
        part += lane + 64 * i < nv ? q : 0.0f;
      }
      ss += wave_sum(part);
    }
    const float rstd = 1.0f / __builtin_sqrtf(ss / (float)D + eps);
    u4* yr = (u4*)(hn + (size_t)wave * ldo);
#pragma unroll
    for (int i = 0; i < kCh; ++i) {
      if (lane + 64 * i >= nv) break;
      uint32_t* xw = (uint32_t*)&xv[i];
      const uint32_t* gw = (const uint32_t*)&gv[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const h2 xx = as_h2(xw[j]), gg = as_h2(gw[j]);
        h2 o;
        o.x = (half_t)(((float)xx.x * rstd) * (float)gg.x);
        o.y = (half_t)(((float)xx.y * rstd) * (float)gg.y);
        xw[j] = as_u32(o);
      }
      yr[lane + 64 * i] = xv[i];
      *(u4*)&hn_l[wave][8 * (lane + 64 * i)] = xv[i];
    }
  }
  __syncthreads();
  // logits on MFMA: wavefront w < NWR takes steps [nsteps * w / NWR, nsteps * (w + 1) / NWR) of 32;
  // all of its router loads are issued before the first product (buffer loads: a step past the
  // range reads zeros)
  const int r = lane & 15, g = lane >> 4;
  const int nsteps = D >> 5;
  constexpr int kMaxSteps = 16;                    // steps per wavefront for D <= 4096 under route_waves
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  if (wave < NWR) {
    const int s0 = nsteps * wave / NWR, s1 = nsteps * (wave + 1) / NWR;
    const __amdgpu_buffer_rsrc_t rrs = make_rsrc(router, E * D * 2);
    const int arow = (r < E ? r : E - 1) * D;     // rows past E computed, not kept
    u4 av[kMaxSteps];
#pragma unroll
    for (int i = 0; i < kMaxSteps; ++i)
      av[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(
                                         rrs, s0 + i < s1 ? (arow + 32 * (s0 + i) + 8 * g) * 2 : 0x7fff0000, 0, 0));
#pragma unroll
    for (int i = 0; i < kMaxSteps; ++i) {
      if (s0 + i >= s1) break;                     // wavefront-uniform
      const int s = s0 + i;
      const u4 bv = r < T ? *(const u4*)&hn_l[r][32 * s + 8 * g] : (u4){0u, 0u, 0u, 0u};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, av[i]), __builtin_bit_cast(h8, bv), acc, 0, 0, 0);
    }
    red[wave][lane] = acc;
  }
  __syncthreads();
  if (wave == 0) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = acc[i];
#pragma unroll
    for (int w = 1; w < NWR; ++w) {
      const f4 q = red[w][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] += q[i];
    }
    // lane: token r, experts 4g .. 4g + 3
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * g + i;
      if (r < T && e < E) {
        lg_l[r][e] = v[i];
        if (logits_out) logits_out[(size_t)r * E + e] = v[i];
      }
    }
  }
  __syncthreads();
  // top-k: wavefront t routes token t
  if (wave < T) {
    float lg[1] = {lane < E ? lg_l[wave][lane] : -INFINITY};
    float g_r;
    int s_r;
    topk_token<1>(lg, lane, E, k, renorm, g_r, s_r);
    if (lane < k) {
      gate[(size_t)wave * k + lane] = g_r;
      sel[(size_t)wave * k + lane] = s_r;
      s_sel[wave * k + lane] = s_r;
    }
  }
  __syncthreads();
  bucket_experts(s_sel, T, E, k, cnt, list);
}

// The same routing with one workgroup per token (grid T, NWR wavefronts), so the loads and the
// normalisation of the T rows run on T CUs instead of one.  Workgroup t repeats the single-workgroup
// kernel's arithmetic for its token: wavefront 0 normalises row t (the 256-thread reduction order),
// the NWR wavefronts compute the router MFMA over their K ranges with row t in B column t (the
// column it has in the batched product, other columns zero), and wavefront 0 sums the partials in
// the same order and routes the token; so hn, the logits, gate and sel are bit for bit those of
// moe_route_kernel.  The bucketing needs every token's choice: each workgroup takes a ticket from
// the caller's counter sync[0] (agent-scope atomic), publishes its k choices as tagged words
// sync[1 + t * k + slot] = (tag << 8) | expert (agent-scope stores, one word each, so a word is
// either old or whole), and the workgroup holding the call's last ticket reads all T * k words,
// waiting (bounded) until each carries the call's tag, then buckets.  Tickets of one call are
// base .. base + T - 1 with base a multiple of 16 (the last workgroup pads the counter to the next
// multiple), so tag = ticket / 16 + 1 names the call (never 0, the words' initial value).
constexpr int kRouteSyncWords = 1 + 16 * 16;
constexpr unsigned kRouteSpin = 1u << 20;        // polls per word before giving up (no arrival)
template <int NWR>
__global__ __launch_bounds__(NWR * 64) void moe_route_tok_kernel(const half_t* __restrict__ h, int ldh,
                                                                 const half_t* __restrict__ gamma, float eps,
                                                                 const half_t* __restrict__ router, int T, int E,
                                                                 int D, int k, int renorm, half_t* __restrict__ hn,
                                                                 int ldo, float* __restrict__ logits_out,
                                                                 float* __restrict__ gate, int* __restrict__ sel,
                                                                 int* __restrict__ cnt, int* __restrict__ list,
                                                                 unsigned* __restrict__ sync) {
  __shared__ __align__(16) half_t hn_l[kRouteRow];
  __shared__ f4 red[NWR][64];
  __shared__ float lg_l[16];
  __shared__ int s_sel[16 * 16];
  __shared__ unsigned s_ticket;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tok = blockIdx.x;
  const int nv = D >> 3;
  constexpr int kCh = kRouteMaxD / 8 / 64;
  // wavefront 0 requests its row and gamma before its router slice: the norm needs them first
  u4 xv[kCh], gv[kCh];
  if (wave == 0) {
    const u4* xr = (const u4*)(h + (size_t)tok * ldh);
    const u4* gr = (const u4*)gamma;
#pragma unroll
    for (int i = 0; i < kCh; ++i) {
      const int f = lane + 64 * i < nv ? lane + 64 * i : 0;
      xv[i] = xr[f];
      gv[i] = gr[f];
    }
  }
  // router loads of this wavefront's K range (rows past E, whose products are never kept, and steps
  // past the range read zeros without traffic)
  const int r = lane & 15, g = lane >> 4;
  const int nsteps = D >> 5;
  constexpr int kMaxSteps = NWR >= 16 ? 8 : 16;     // steps per wavefront (D <= 4096 under route_waves)
  const int s0 = nsteps * wave / NWR, s1 = nsteps * (wave + 1) / NWR;
  const __amdgpu_buffer_rsrc_t rrs = make_rsrc(router, E * D * 2);
  u4 av[kMaxSteps];
#pragma unroll
  for (int i = 0; i < kMaxSteps; ++i)
    av[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(
                                       rrs, s0 + i < s1 && r < E ? (r * D + 32 * (s0 + i) + 8 * g) * 2 : 0x7fff0000,
                                       0, 0));
  // RMSNorm of row tok by wavefront 0, in moe_route_kernel's order
  if (wave == 0) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float part = 0.0f;
#pragma unroll
      for (int i = j; i < kCh; i += 4) {
        float q = dot2(as_h2(xv[i].x), as_h2(xv[i].x), 0.0f);
        q = dot2(as_h2(xv[i].y), as_h2(xv[i].y), q);
        q = dot2(as_h2(xv[i].z), as_h2(xv[i].z), q);
        q = dot2(as_h2(xv[i].w), as_h2(xv[i].w), q);
        part += lane + 64 * i < nv ? q : 0.0f;
      }
      ss += wave_sum(part);
    }
    const float rstd = 1.0f / __builtin_sqrtf(ss / (float)D + eps);
    u4* yr = (u4*)(hn + (size_t)tok * ldo);
    auto nrm = [&](uint32_t xw, uint32_t gw) {
      const h2 xx = as_h2(xw), gg = as_h2(gw);
      h2 o;
      o.x = (half_t)(((float)xx.x * rstd) * (float)gg.x);
      o.y = (half_t)(((float)xx.y * rstd) * (float)gg.y);
      return as_u32(o);
    };
#pragma unroll
    for (int i = 0; i < kCh; ++i) {
      if (lane + 64 * i >= nv) break;
      const u4 o = {nrm(xv[i].x, gv[i].x), nrm(xv[i].y, gv[i].y), nrm(xv[i].z, gv[i].z), nrm(xv[i].w, gv[i].w)};
      yr[lane + 64 * i] = o;
      *(u4*)&hn_l[8 * (lane + 64 * i)] = o;
    }
  }
  __syncthreads();
  // logits of token tok: B column tok holds its row, the other columns zero (every LDS read issued
  // before the first product; steps past the wavefront's range are skipped, uniformly)
  u4 bvs[kMaxSteps];
#pragma unroll
  for (int i = 0; i < kMaxSteps; ++i) {
    const int s = s0 + i < s1 ? s0 + i : s0;
    bvs[i] = r == tok ? *(const u4*)&hn_l[32 * s + 8 * g] : (u4){0u, 0u, 0u, 0u};
  }
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < kMaxSteps; ++i)
    if (s0 + i < s1)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, av[i]), __builtin_bit_cast(h8, bvs[i]), acc,
                                                   0, 0, 0);
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = acc[i];
#pragma unroll
    for (int w = 1; w < NWR; ++w) {
      const f4 q = red[w][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] += q[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * g + i;
      if (r == tok && e < E) {
        lg_l[e] = v[i];
        if (logits_out) logits_out[(size_t)tok * E + e] = v[i];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float lg[1] = {lane < E ? lg_l[lane] : -INFINITY};
    float g_r;
    int s_r;
    topk_token<1>(lg, lane, E, k, renorm, g_r, s_r);
    unsigned ticket = 0;
    if (lane == 0) ticket = __hip_atomic_fetch_add(sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ticket = __builtin_amdgcn_readfirstlane(ticket);
    const unsigned tag = ((ticket >> 4) + 1u) & 0xffffffu;
    if (lane < k) {
      gate[(size_t)tok * k + lane] = g_r;
      sel[(size_t)tok * k + lane] = s_r;
      __hip_atomic_store(sync + 1 + tok * k + lane, (tag << 8) | (unsigned)s_r, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    if (lane == 0) s_ticket = ticket;
  }
  __syncthreads();
  const unsigned ticket = s_ticket;
  if ((int)(ticket & 15u) != T - 1) return;        // not the call's last workgroup (uniform)
  // the last workgroup: every token's tagged choices, then the buckets
  const unsigned tag = ((ticket >> 4) + 1u) & 0xffffffu;
  for (int i = threadIdx.x; i < T * k; i += NWR * 64) {
    unsigned w = 0;
    for (unsigned it = 0; it < kRouteSpin; ++it) {
      w = __hip_atomic_load(sync + 1 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((w >> 8) == tag) break;
    }
    s_sel[i] = (w >> 8) == tag ? (int)(w & 0xffu) : -1;   // -1 (never arrived): routed nowhere
  }
  __syncthreads();
  if (T * k <= 64) {
    if (wave == 0) bucket_experts_wave(lane < T * k ? s_sel[lane] : -1, lane, T, E, cnt, list);
  } else {
    bucket_experts(s_sel, T, E, k, cnt, list);
  }
  if (threadIdx.x == 0 && T < 16) __hip_atomic_fetch_add(sync, (unsigned)(16 - T), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct MoeArgs {
  const void* w;          // expert weights, expert stride w_es bytes
  const half_t* scale;    // I8: [E][N]; Q4: [E][N][K/32]
  long long w_es, s_es;   // per-expert strides (bytes for w, elements for scale)
  const half_t* x;        // activation rows, row r at x + r_src * ldx
  int ldx;
  void* y;
  int ldy;
  const int* cnt;
  const int* list;
  int T, k, N, K, epi;    // epi: 0 = fp32 store (down), 1 = SwiGLU fp16 (gate/up)
  int x_by_token;         // 1: x row = list/k (token), 0: x row = list entry (token*k+slot)
};

template <int FMT, int MG, int R>
__global__ __launch_bounds__(256) void moe_group_kernel(MoeArgs a) {
  const int e = blockIdx.y;
  const int n_e = a.cnt[e];
  if (n_e == 0) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  if (row0 >= a.N) return;
  const int K = a.K, N = a.N;
  const int* lst = a.list + (size_t)e * a.T;
  const size_t rb = Fmt<FMT>::row_bytes(K);
  const unsigned char* wbase = (const unsigned char*)a.w + (size_t)e * a.w_es;
  const half_t* sbase = a.scale ? a.scale + (size_t)e * a.s_es : nullptr;
  const unsigned char* wrow[R];
  const half_t* drow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r < N ? row0 + r : N - 1;
    wrow[r] = wbase + (size_t)row * rb;
    drow[r] = has_block_scales<FMT>() ? sbase + (size_t)row * scale_row_halves<FMT>(K) : nullptr;
  }
  const int nchunks = K / Fmt<FMT>::kWeightsPerChunk;
  typename Fmt<FMT>::Ctx fctx[R];
#pragma unroll
  for (int r = 0; r < R; ++r) fctx[r] = Fmt<FMT>::Ctx::make(sbase, row0 + r < N ? row0 + r : N - 1);
  const int rr = reduced_row_of_lane<R>(lane);
  const int row = row0 + rr;
  constexpr int GROUP = 64 / R;
  const bool writer = (lane & (GROUP - 1)) == 0;

  for (int mb = 0; mb < n_e; mb += MG) {
    const half_t* xp[MG];
    int ent[MG];
#pragma unroll
    for (int m = 0; m < MG; ++m) {
      const int i = mb + m < n_e ? mb + m : n_e - 1;
      ent[m] = lst[i];
      const int src = a.x_by_token ? ent[m] / a.k : ent[m];
      xp[m] = a.x + (size_t)src * a.ldx;
    }
    float acc[MG][R];
#pragma unroll
    for (int m = 0; m < MG; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;
    constexpr int U = 2;
    for (int cb = lane; cb < nchunks; cb += 64 * U) {
      u4 wv[U][R];
      typename Fmt<FMT>::S dv[U][R];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = cb + 64 * u;
        const int cc = c < nchunks ? c : nchunks - 1;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          wv[u][r] = *(const u4*)(wrow[r] + (size_t)cc * 16);
          dv[u][r] = load_scales<FMT>(drow[r], cc);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = cb + 64 * u;
        if (c < nchunks) {
#pragma unroll
          for (int m = 0; m < MG; ++m) {
            h2 xv[Fmt<FMT>::kXH2];
            Fmt<FMT>::load_x(xp[m], c, xv);
#pragma unroll
            for (int r = 0; r < R; ++r) acc[m][r] = Fmt<FMT>::dot(wv[u][r], xv, dv[u][r], fctx[r], acc[m][r]);
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MG; ++m) {
      const float sum = wave_reduce_rows<R>(acc[m], lane);
      const bool live = mb + m < n_e;
      const float sc = (FMT == FMT_I8 && row < N) ? (float)sbase[row] : 1.0f;
      const float v = sum * sc;
      if (a.epi == 1) {
        const float other = shfl_xor(v, GROUP);
        if (writer && live && row < N && (row & 1) == 0) {
          const float g16 = (float)(half_t)v, u16 = (float)(half_t)other;
          ((half_t*)a.y)[(size_t)ent[m] * a.ldy + (row >> 1)] = (half_t)(silu(g16) * u16);
        }
      } else {
        if (writer && live && row < N) ((float*)a.y)[(size_t)ent[m] * a.ldy + row] = v;
      }
    }
  }
}

__global__ void moe_combine_kernel(const half_t* __restrict__ h, const float* __restrict__ y,
                                   const float* __restrict__ gate, const half_t* __restrict__ shared,
                                   half_t* __restrict__ out, int T, int k, int D) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)T * D) return;
  const int t = (int)(i / D), d = (int)(i - (long long)t * D);
  float acc = 0.0f;
  for (int s = 0; s < k; ++s) {
    const float ys = (float)(half_t)y[((size_t)t * k + s) * D + d];
    acc = __builtin_fmaf(gate[(size_t)t * k + s], ys, acc);
  }
  float c = (float)(half_t)acc;
  if (shared) c = (float)(half_t)(c + (float)shared[i]);
  out[i] = (half_t)((float)h[i] + c);
}

// The K-split down's finishing sum fused with the combine: y[row][d] = the S slices of ws summed in
// slice order (the finishing kernel's order), then as moe_combine_kernel; with S = 1, ws is y.
__global__ void moe_combine_ws_kernel(const half_t* __restrict__ h, const float* __restrict__ ws, int S,
                                      long long slice, const float* __restrict__ gate,
                                      const half_t* __restrict__ shared, half_t* __restrict__ out, int T, int k,
                                      int D) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)T * D) return;
  const int t = (int)(i / D), d = (int)(i - (long long)t * D);
  float acc = 0.0f;
  for (int s = 0; s < k; ++s) {
    const float* yp = ws + ((size_t)t * k + s) * D + d;
    float v = 0.0f;
    for (int q = 0; q < S; ++q) v += yp[(size_t)q * slice];
    acc = __builtin_fmaf(gate[(size_t)t * k + s], (float)(half_t)v, acc);
  }
  float c = (float)(half_t)acc;
  if (shared) c = (float)(half_t)(c + (float)shared[i]);
  out[i] = (half_t)((float)h[i] + c);
}

typedef void (*moe_fn)(MoeArgs);
template <int FMT>
static moe_fn pick_moe(int R) {
  return R >= 4 ? moe_group_kernel<FMT, 4, 4> : R >= 2 ? moe_group_kernel<FMT, 4, 2> : moe_group_kernel<FMT, 4, 1>;
}

static int moe_launch(int fmt, MoeArgs& a, int E, int R, hipStream_t stream, const char* what) {
  AFX_REQUIRE(fmt >= 0 && fmt <= 6, "%s: unknown weight format %d", what, fmt);
  const int kq = fmt == FMT_I8 ? 16 : fmt == FMT_Q4 ? 128 : fmt == FMT_BW ? 64 : fmt == FMT_L4 ? 32
               : fmt == FMT_Q4K || fmt == FMT_Q6K ? 256 : 8;
  AFX_REQUIRE(a.K % kq == 0, "%s: K=%d must be a multiple of %d", what, a.K, kq);
  AFX_REQUIRE(a.w && a.x && a.y && a.cnt && a.list, "%s: null pointer", what);
  AFX_REQUIRE(fmt == FMT_F16 || a.scale, "%s: quantized weights need scales", what);
  moe_fn fn = fmt == FMT_I8 ? pick_moe<FMT_I8>(R) : fmt == FMT_Q4 ? pick_moe<FMT_Q4>(R)
            : fmt == FMT_BW ? pick_moe<FMT_BW>(R) : fmt == FMT_L4 ? pick_moe<FMT_L4>(R)
            : fmt == FMT_Q4K ? pick_moe<FMT_Q4K>(R) : fmt == FMT_Q6K ? pick_moe<FMT_Q6K>(R) : pick_moe<FMT_F16>(R);
  const int gx = (a.N + 4 * R - 1) / (4 * R);
  hipLaunchKernelGGL(fn, dim3(gx, E), dim3(256), 0, stream, a);
  return check_launch(what);
}

static long long fmt_row_bytes(int fmt, int K) {
  return fmt == FMT_I8 || fmt == FMT_BW ? K : fmt == FMT_Q4 || fmt == FMT_L4 || fmt == FMT_Q4K || fmt == FMT_Q6K ? K / 2
       : 2LL * K;
}
// Elements (halves) of one expert's scale array: rows of `rows` weights over K.
static long long fmt_scale_halves(int fmt, long long rows, int K) {
  return fmt == FMT_Q4 || fmt == FMT_BW ? rows * (K / 32) : fmt == FMT_L4 ? rows * 16
       : fmt == FMT_Q4K ? rows * (K / 256) * 10 : fmt == FMT_Q6K ? rows * (K / 32) * 6 : rows;
}

}  // namespace afx

using namespace afx;

namespace afx {

// The graph form of the top-k gate: y[t, e] = x[t, e] for the k experts a row picks, else 0.
// x holds fp16 probabilities; one wavefront per row, lane l owns experts l, l + 64, ...; each of
// the k rounds takes the row maximum and, among experts holding exactly that fp16 value, the
// lowest index, so a row never keeps more than k experts (aneforge/moe.py:21-37).
template <int J>
__global__ __launch_bounds__(256) void topk_mask_kernel(const half_t* __restrict__ x, int T, int E, int k,
                                                        half_t* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= T) return;
  const half_t* xr = x + (size_t)row * E;
  half_t* yr = y + (size_t)row * E;
  float v[J];
  bool keep[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? (float)xr[e] : -INFINITY;
    keep[j] = false;
  }
  for (int r = 0; r < k; ++r) {
    float best = -INFINITY;
    int at = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (lane + 64 * j < E && !keep[j] && (v[j] > best || at == 0x7fffffff)) { best = v[j]; at = lane + 64 * j; }
    const float top = wave_max(best);
    float cand = (at != 0x7fffffff && best == top) ? (float)at : 3.0e38f;
    const int win = (int)(-wave_max(-cand));
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (lane + 64 * j == win) keep[j] = true;
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = lane + 64 * j;
    if (e < E) yr[e] = keep[j] ? xr[e] : (half_t)0.0f;
  }
}

}  // namespace afx

using namespace afx;

extern "C" {

int afx_topk_mask(const void* x, int T, int E, int k, void* y, void* stream) {
  AFX_REQUIRE(x && y, "afx_topk_mask: null pointer");
  AFX_REQUIRE(k >= 1 && k <= E && E <= 2049, "afx_topk_mask: need 1 <= k <= E <= 2049; got k=%d E=%d", k, E);
  AFX_REQUIRE(T >= 1, "afx_topk_mask: T=%d", T);
  const int jn = (E + 63) / 64;
  auto fn = jn <= 1 ? topk_mask_kernel<1> : jn <= 2 ? topk_mask_kernel<2> : jn <= 4 ? topk_mask_kernel<4>
          : jn <= 8 ? topk_mask_kernel<8> : jn <= 16 ? topk_mask_kernel<16> : topk_mask_kernel<33>;
  hipLaunchKernelGGL(fn, dim3((T + 3) / 4), dim3(256), 0, (hipStream_t)stream, (const half_t*)x, T, E, k,
                     (half_t*)y);
  return check_launch("afx_topk_mask");
}

int afx_moe_topk(const float* logits, int T, int E, int k, int renorm, float* gate, int* sel, int* cnt,
                 int* list, void* stream) {
  AFX_REQUIRE(logits && gate && sel && cnt && list, "afx_moe_topk: null pointer");
  AFX_REQUIRE(k >= 1 && k <= E && E <= 2049 && k <= 64, "afx_moe_topk: need 1 <= k <= E <= 2049 (k <= 64); got k=%d E=%d", k, E);
  AFX_REQUIRE(T >= 1 && T * k <= 16384, "afx_moe_topk: T=%d out of range", T);
  const int jn = (E + 63) / 64;
  auto fn = jn <= 1 ? moe_topk_kernel<1> : jn <= 2 ? moe_topk_kernel<2> : jn <= 4 ? moe_topk_kernel<4>
          : jn <= 8 ? moe_topk_kernel<8> : jn <= 16 ? moe_topk_kernel<16> : moe_topk_kernel<33>;
  const int waves = T < 16 ? T : 16;               // one wavefront per token, up to 16 at a time
  hipLaunchKernelGGL(fn, dim3(1), dim3(64 * waves), (size_t)T * k * sizeof(int), (hipStream_t)stream,
                     logits, T, E, k, renorm, gate, sel, cnt, list);
  return check_launch("afx_moe_topk");
}

// W: [E][2F][D] gate/up interleaved rows (format fmt), x: normed hidden [T][D].
int afx_moe_gateup(int fmt, const void* w, const void* scale, const void* x, int T, int k, int E, int F, int D,
                   const int* cnt, const int* list, void* act, int rows_hint, void* stream) {
  if (rows_hint == 0 && mfma_supported(fmt, D) && F % 2 == 0) {
    MfmaArgs m = {};
    m.w = w; m.scale = (const half_t*)scale; m.x = (const half_t*)x; m.ldx = D; m.y = act; m.ldy = F;
    m.cnt = cnt; m.list = list; m.T = T; m.k = k; m.x_by_token = 1; m.N = 2 * F; m.K = D; m.epi = EPI_SWIGLU;
    m.w_es = fmt_row_bytes(fmt, D) * 2 * F;
    m.s_es = fmt == FMT_Q4 || fmt == FMT_BW ? 2LL * F * (D / 32) : fmt == FMT_I8 ? 2LL * F : 0;
    AFX_REQUIRE(T >= 1 && k >= 1 && E >= 1, "afx_moe_gateup: bad sizes");
    return mfma_launch(fmt, m, E, (hipStream_t)stream, "afx_moe_gateup");
  }
  MoeArgs a = {};
  a.w = w; a.scale = (const half_t*)scale; a.x = (const half_t*)x; a.ldx = D; a.y = act; a.ldy = F;
  a.cnt = cnt; a.list = list; a.T = T; a.k = k; a.N = 2 * F; a.K = D; a.epi = 1; a.x_by_token = 1;
  a.w_es = fmt_row_bytes(fmt, D) * 2 * F;
  a.s_es = fmt_scale_halves(fmt, 2LL * F, D);
  const int R = rows_hint == 1 || rows_hint == 2 || rows_hint == 4 ? (rows_hint < 2 ? 2 : rows_hint) : 4;
  return moe_launch(fmt, a, E, R, (hipStream_t)stream, "afx_moe_gateup");
}

// W: [E][D][F], act: [T*k][F] -> y: [T*k][D] fp32.
int afx_moe_down(int fmt, const void* w, const void* scale, const void* act, int T, int k, int E, int F, int D,
                 const int* cnt, const int* list, float* y, int rows_hint, void* ws, long long ws_bytes,
                 void* stream) {
  if (rows_hint == 0 && mfma_supported(fmt, F) && D % 4 == 0) {
    MfmaArgs m = {};
    m.w = w; m.scale = (const half_t*)scale; m.x = (const half_t*)act; m.ldx = F; m.y = y; m.ldy = D;
    m.cnt = cnt; m.list = list; m.T = T; m.k = k; m.x_by_token = 0; m.N = D; m.K = F; m.epi = EPI_F32;
    m.w_es = fmt_row_bytes(fmt, F) * D;
    m.s_es = fmt == FMT_Q4 || fmt == FMT_BW ? (long long)D * (F / 32) : fmt == FMT_I8 ? (long long)D : 0;
    m.ws = (float*)ws; m.ws_bytes = ws ? ws_bytes : 0;
    AFX_REQUIRE(T >= 1 && k >= 1 && E >= 1, "afx_moe_down: bad sizes");
    return mfma_launch(fmt, m, E, (hipStream_t)stream, "afx_moe_down");
  }
  MoeArgs a = {};
  a.w = w; a.scale = (const half_t*)scale; a.x = (const half_t*)act; a.ldx = F; a.y = y; a.ldy = D;
  a.cnt = cnt; a.list = list; a.T = T; a.k = k; a.N = D; a.K = F; a.epi = 0; a.x_by_token = 0;
  a.w_es = fmt_row_bytes(fmt, F) * D;
  a.s_es = fmt_scale_halves(fmt, D, F);
  const int R = rows_hint == 1 || rows_hint == 2 || rows_hint == 4 ? rows_hint : 4;
  return moe_launch(fmt, a, E, R, (hipStream_t)stream, "afx_moe_down");
}

// The skinny MFMA kernel's wavefront count for a dense fp16 linear of K = D (the persistent kernel's
// if each wavefront then has at most one batch, else the tile kernel's), so the fused router
// splits K as afx_linear would.
static int route_waves(int D) {
  const int nsteps = D / 32;
  for (int w = 16; w >= 4; w >>= 1)
    if (nsteps >= w && (nsteps + w - 1) / w <= 4) return w;
  auto batches = [&](int w) { return ((nsteps + w - 1) / w + 3) / 4; };
  return batches(4) <= 4 ? 4 : batches(8) <= 4 ? 8 : 16;
}

int afx_moe_route(const void* h, int ldh, const void* gamma, float eps, const void* router, int T, int E, int D,
                  int k, int renorm, void* hn, int ldo, float* logits, float* gate, int* sel, int* cnt, int* list,
                  unsigned* sync, void* stream) {
  AFX_REQUIRE(h && gamma && router && hn && gate && sel && cnt && list, "afx_moe_route: null pointer");
  AFX_REQUIRE(T >= 1 && T <= 16 && E >= 1 && E <= 16 && k >= 1 && k <= E,
              "afx_moe_route: needs 1 <= T <= 16 and 1 <= k <= E <= 16; got T=%d E=%d k=%d", T, E, k);
  AFX_REQUIRE(D % 32 == 0 && D >= 256 && D <= kRouteMaxD, "afx_moe_route: D=%d must be a multiple of 32 in [256, %d]",
              D, kRouteMaxD);
  AFX_REQUIRE(ldh % 8 == 0 && ldo % 8 == 0 && ldh >= D && ldo >= D &&
                  (((uintptr_t)h | (uintptr_t)gamma | (uintptr_t)router | (uintptr_t)hn) & 15) == 0,
              "afx_moe_route: rows must be 16-byte aligned (ldh, ldo multiples of 8)");
  const int nw = route_waves(D);
  AFX_REQUIRE((D / 32 + nw - 1) / nw <= 16, "afx_moe_route: D=%d splits into more than 16 steps per wavefront", D);
  if (sync) {                                    // one workgroup per token
    AFX_REQUIRE(((uintptr_t)sync & 3) == 0, "afx_moe_route: sync must be 4-byte aligned");
    auto fn = nw == 4 ? moe_route_tok_kernel<4> : nw == 8 ? moe_route_tok_kernel<8> : moe_route_tok_kernel<16>;
    hipLaunchKernelGGL(fn, dim3(T), dim3(nw * 64), 0, (hipStream_t)stream, (const half_t*)h, ldh,
                       (const half_t*)gamma, eps, (const half_t*)router, T, E, D, k, renorm, (half_t*)hn, ldo, logits,
                       gate, sel, cnt, list, sync);
    return check_launch("afx_moe_route");
  }
  auto fn = nw == 4 ? moe_route_kernel<4> : nw == 8 ? moe_route_kernel<8> : moe_route_kernel<16>;
  hipLaunchKernelGGL(fn, dim3(1), dim3(1024), 0, (hipStream_t)stream, (const half_t*)h, ldh, (const half_t*)gamma,
                     eps, (const half_t*)router, T, E, D, k, renorm, (half_t*)hn, ldo, logits, gate, sel, cnt, list);
  return check_launch("afx_moe_route");
}

int afx_moe_down_combine(int fmt, const void* w, const void* scale, const void* act, int T, int k, int E, int F,
                         int D, const int* cnt, const int* list, float* y, void* ws, long long ws_bytes,
                         const void* h, const float* gate, const void* shared, void* out, void* stream) {
  AFX_REQUIRE(h && gate && out && y, "afx_moe_down_combine: null pointer");
  int S = 1;
  if (mfma_supported(fmt, F) && D % 4 == 0) {
    MfmaArgs m = {};
    m.w = w; m.scale = (const half_t*)scale; m.x = (const half_t*)act; m.ldx = F; m.y = y; m.ldy = D;
    m.cnt = cnt; m.list = list; m.T = T; m.k = k; m.x_by_token = 0; m.N = D; m.K = F; m.epi = EPI_F32;
    m.w_es = fmt_row_bytes(fmt, F) * D;
    m.s_es = fmt == FMT_Q4 || fmt == FMT_BW ? (long long)D * (F / 32) : fmt == FMT_I8 ? (long long)D : 0;
    m.ws = (float*)ws; m.ws_bytes = ws ? ws_bytes : 0;
    AFX_REQUIRE(T >= 1 && k >= 1 && E >= 1, "afx_moe_down_combine: bad sizes");
    const int rc = mfma_launch(fmt, m, E, (hipStream_t)stream, "afx_moe_down_combine", &S);
    if (rc) return rc;
  } else {
    const int rc = afx_moe_down(fmt, w, scale, act, T, k, E, F, D, cnt, list, y, 0, nullptr, 0, stream);
    if (rc) return rc;
  }
  const long long n = (long long)T * D;
  hipLaunchKernelGGL(moe_combine_ws_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const half_t*)h, S > 1 ? (const float*)ws : (const float*)y, S, (long long)T * k * D, gate,
                     (const half_t*)shared, (half_t*)out, T, k, D);
  return check_launch("afx_moe_down_combine");
}

int afx_moe_combine(const void* h, const float* y, const float* gate, const void* shared, void* out, int T, int k,
                    int D, void* stream) {
  AFX_REQUIRE(h && y && gate && out, "afx_moe_combine: null pointer");
  const long long n = (long long)T * D;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const half_t*)h, y, gate, (const half_t*)shared, (half_t*)out, T, k, D);
  return check_launch("afx_moe_combine");
}

// 32-bit words of the afx_moe_route `sync` buffer (zeroed once by the caller).
int afx_moe_route_sync_words(void) { return kRouteSyncWords; }

}  // extern "C"
