// Small device kernels around the weight-streaming hot path: RMSNorm, RoPE, embedding
// gather, greedy token advance, and the generic tensor ops the af.compile graph executor
// lowers to (broadcast elementwise, unary activations, last-axis softmax/reductions,
// strided copies for reshape/transpose/slice/concat, and an fp16 batched matmul for
// activation x activation products).  None of these is bandwidth-significant in decode.
#include "afx_common.h"

namespace afx {

// ---- RMSNorm (aneforge/graph.py:293-301; textbook form as in tests/test_moe.py:26) ----
// Vector form: each thread keeps up to NV 16-byte vectors of its row in registers between the
// sum of squares and the scaling (D % 8 == 0, 16-byte aligned rows, D <= 2048 * NV).
template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(const half_t* __restrict__ x, int ldx,
                                                          const half_t* __restrict__ g, float eps,
                                                          half_t* __restrict__ y, int ldy, int D) {
  __shared__ float red[4];
  const int m = blockIdx.x, t = threadIdx.x;
  const int nv = D >> 3;
  const u4* xr = (const u4*)(x + (size_t)m * ldx);
  u4 xv[NV], gv[NV];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int f = t + 256 * i < nv ? t + 256 * i : nv - 1;
    xv[i] = xr[f];
    gv[i] = ((const u4*)g)[f];
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    float q = dot2(as_h2(xv[i].x), as_h2(xv[i].x), 0.0f);
    q = dot2(as_h2(xv[i].y), as_h2(xv[i].y), q);
    q = dot2(as_h2(xv[i].z), as_h2(xv[i].z), q);
    q = dot2(as_h2(xv[i].w), as_h2(xv[i].w), q);
    ss += t + 256 * i < nv ? q : 0.0f;
  }
  ss = wave_sum(ss);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  const float rstd = 1.0f / __builtin_sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)D + eps);
  u4* yr = (u4*)(y + (size_t)m * ldy);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (t + 256 * i >= nv) break;
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
    yr[t + 256 * i] = xv[i];
  }
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(const half_t* __restrict__ x, int ldx,
                                                      const half_t* __restrict__ g, float eps,
                                                      half_t* __restrict__ y, int ldy, int D) {
  __shared__ float red[4];
  const int m = blockIdx.x, t = threadIdx.x;
  const half_t* xr = x + (size_t)m * ldx;
  float ss = 0.0f;
  for (int i = t; i < D; i += 256) { const float v = (float)xr[i]; ss = __builtin_fmaf(v, v, ss); }
  ss = wave_sum(ss);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  const float rstd = 1.0f / __builtin_sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)D + eps);
  half_t* yr = y + (size_t)m * ldy;
  for (int i = t; i < D; i += 256) yr[i] = (half_t)(((float)xr[i] * rstd) * (float)g[i]);
}

// ---- RoPE, neox half-split layout (aneforge/llm.py:96-105): x*cos + rotate_half(x)*sin ----
// x rows of length dh; row r uses table row pos_of_row[r] (or pos0 + r / rows_per_pos).
__global__ void rope_kernel(const half_t* __restrict__ x, half_t* __restrict__ y, int rows, int dh,
                            const half_t* __restrict__ cos_t, const half_t* __restrict__ sin_t,
                            const int* __restrict__ pos_dev, int pos0, int rows_per_pos) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const int half = dh >> 1;
  if (i >= (long long)rows * half) return;
  const int r = (int)(i / half), j = (int)(i - (long long)r * half);
  const int p = (pos_dev ? pos_dev[0] : pos0) + r / rows_per_pos;
  const float x1 = (float)x[(size_t)r * dh + j], x2 = (float)x[(size_t)r * dh + j + half];
  const float c1 = (float)cos_t[(size_t)p * dh + j], s1 = (float)sin_t[(size_t)p * dh + j];
  const float c2 = (float)cos_t[(size_t)p * dh + j + half], s2 = (float)sin_t[(size_t)p * dh + j + half];
  y[(size_t)r * dh + j] = (half_t)(x1 * c1 - x2 * s1);
  y[(size_t)r * dh + j + half] = (half_t)(x2 * c2 + x1 * s2);
}

// ---- per-head RMSNorm then RoPE, in place (Qwen3 QK-norm, aneforge/llm.py:224-225 then :227) ----
// Head h of sequence m lives at x + m*seq_stride + h*head_stride + pos_mul*pos[m] (pos_mul = dh for
// a cache row, 0 for a q buffer).  One wavefront per (head, sequence); rows at pos outside
// [0, kv_len) are skipped.
__global__ __launch_bounds__(64) void head_norm_rope_kernel(half_t* __restrict__ x, long long seq_stride,
                                                            long long head_stride, int pos_mul,
                                                            const int* __restrict__ pos, int kv_len, int dh,
                                                            const half_t* __restrict__ g, float eps,
                                                            const half_t* __restrict__ cos_t,
                                                            const half_t* __restrict__ sin_t, int rope) {
  const int h = blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
  const int p = pos ? pos[m] : 0;
  if (pos && (p < 0 || p >= kv_len)) return;
  half_t* r = x + (size_t)m * seq_stride + (size_t)h * head_stride + (size_t)pos_mul * p;
  const int half = dh >> 1;
  float v[4];                                        // dh <= 256: 4 values per lane
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    v[i] = d < dh ? (float)r[d] : 0.0f;
    ss += v[i] * v[i];
  }
  ss = wave_sum(ss);
  const float rstd = 1.0f / __builtin_sqrtf(ss / (float)dh + eps);
  float n[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    n[i] = d < dh ? (float)(half_t)(v[i] * rstd * (float)g[d]) : 0.0f;   // fp16 norm output
  }
  __shared__ float sh[256];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    if (d < dh) sh[d] = n[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    if (d >= dh) continue;
    float o = n[i];
    if (rope) {
      const float c = (float)cos_t[(size_t)p * dh + d], s = (float)sin_t[(size_t)p * dh + d];
      const float rot = d < half ? -sh[d + half] : sh[d - half];
      o = o * c + rot * s;
    }
    r[d] = (half_t)o;
  }
}

// ---- embedding gather: out[m] = table[ids[m]] ----
__global__ void embed_kernel(const half_t* __restrict__ table, const int* __restrict__ ids,
                             half_t* __restrict__ out, int D, int vocab) {
  const int m = blockIdx.x;
  int id = ids[m];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  const u4* src = (const u4*)(table + (size_t)id * D);
  u4* dst = (u4*)(out + (size_t)m * D);
  for (int i = threadIdx.x; i < D / 8; i += blockDim.x) dst[i] = src[i];
}

// ---- one step of the device-resident decode loop ----
// The next token is forced[*step] while *step < *n_forced (prompt tokens, token-by-token
// prefill), else the greedy pick (lowest index on ties, like np.argmax; greedy _sample).  Then
// hist[*step] = token, ++*step, ++*pos, h = embed[token].  One workgroup; every input that
// changes between steps lives in device memory, so the step replays as a captured graph.
//
// The greedy pick comes from the lm_head's slot summaries when given (else from the logits), with
// the reference's near-tie rule (aneforge/llm.py:395-404): when the two largest logits are closer
// than margin * max |logit|, every logit inside that window of the largest is recomputed exactly
// (fp64 sum of the staged fp16 hidden row times the head row, fp32 head rows when the checkpoint's
// head is not fp16-exact) and the largest exact value wins, the lowest index on an exact tie.
struct AdvanceArgs {
  const float* logits;
  const float4* slots;     // optional: ceil(V / 8) summaries from afx_lm_head
  int V;
  const float* margin;     // optional (device): the tie margin; null = plain argmax
  const half_t* hn;        // the head's normalised input row [D]
  const half_t* head16;    // head rows [V][D], fp16 ...
  const float* head32;     // ... or fp32 (preferred when given)
  const int* forced;
  const int* n_forced;
  int* tok;
  int* pos;
  int* hist;
  int hist_cap;
  int* step;
  const half_t* embed;
  half_t* h;
  int D, vocab;
};

// One DPP step of a wavefront-wide top2_merge: lanes whose source lane is outside the pattern
// read the neutral summary, so they keep their own.
template <int CTRL, int RMASK>
__device__ __forceinline__ float4 top2_dpp(float4 v) {
  const int nx = __float_as_int(-INFINITY), ny = 0x7fffffff, nw = __float_as_int(0.0f);
  float4 o;
  o.x = __int_as_float(__builtin_amdgcn_update_dpp(nx, __float_as_int(v.x), CTRL, RMASK, 0xf, false));
  o.y = __int_as_float(__builtin_amdgcn_update_dpp(ny, __float_as_int(v.y), CTRL, RMASK, 0xf, false));
  o.z = __int_as_float(__builtin_amdgcn_update_dpp(nx, __float_as_int(v.z), CTRL, RMASK, 0xf, false));
  o.w = __int_as_float(__builtin_amdgcn_update_dpp(nw, __float_as_int(v.w), CTRL, RMASK, 0xf, false));
  return top2_merge(v, o);
}
// The wavefront's merged summary (row shifts, then row broadcasts into lane 63), wave-uniform.
__device__ __forceinline__ float4 top2_wave(float4 v) {
  v = top2_dpp<0x111, 0xf>(v);   // row_shr:1
  v = top2_dpp<0x112, 0xf>(v);   // row_shr:2
  v = top2_dpp<0x114, 0xf>(v);   // row_shr:4
  v = top2_dpp<0x118, 0xf>(v);   // row_shr:8: lane 15 of each row holds the row's summary
  v = top2_dpp<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
  v = top2_dpp<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3: lane 63 holds the total
  return float4{__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v.x), 63)),
                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v.y), 63)),
                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v.z), 63)),
                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v.w), 63))};
}

// The merged summary of the 16 per-wavefront summaries in lanes 0-15 (the other lanes hold the
// neutral summary), wave-uniform: the row shifts of top2_wave, read from lane 15.
__device__ __forceinline__ float4 top2_row0(float4 v) {
  v = top2_dpp<0x111, 0xf>(v);   // row_shr:1
  v = top2_dpp<0x112, 0xf>(v);   // row_shr:2
  v = top2_dpp<0x114, 0xf>(v);   // row_shr:4
  v = top2_dpp<0x118, 0xf>(v);   // row_shr:8: lane 15 holds row 0's summary
  return float4{__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v.x), 15)),
                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v.y), 15)),
                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v.z), 15)),
                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v.w), 15))};
}

constexpr int kAdvThreads = 1024;   // the launch's workgroup size (16 wavefronts)

// Every wavefront merges the 16 per-wavefront summaries itself and derives the same pick, so the
// common step (no near tie) has one barrier: the summary loads go out as soon as the arguments
// arrive, the step state's loads overlap them, and the token row is gathered by all threads
// while thread 0 records the token.
__global__ __launch_bounds__(kAdvThreads) void decode_advance_kernel(AdvanceArgs a) {
  constexpr int NT = kAdvThreads, NW = NT / 64;
  __shared__ float4 wpart[NW];
  __shared__ double xbest[NW];
  __shared__ int xidx[NW];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const float4 none = float4{-INFINITY, __int_as_float(0x7fffffff), -INFINITY, 0.0f};
  // 1. the step state and the margin, with no wait: their values are needed after the summaries
  // (an absent optional input reads the step word instead, and the value is not used)
  const int s = a.step[0];
  const int p0 = a.pos[0];
  const int nfr = *(a.n_forced ? a.n_forced : a.step);
  const float mraw = *(a.margin ? a.margin : (const float*)a.step);
  // 2. the summaries (or the logits): the long pole
  float4 acc = none;
  if (a.slots) {
    const int ns = (a.V + 7) >> 3;
    for (int b0 = 0; b0 < ns; b0 += 4 * NT) {
      float4 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = b0 + j * NT + t;
        v[j] = a.slots[i < ns ? i : ns - 1];   // a clamped duplicate is replaced below
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = top2_merge(acc, b0 + j * NT + t < ns ? v[j] : none);
    }
  } else if (a.logits) {
    for (int b0 = 0; b0 < a.V; b0 += 8 * NT) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = b0 + j * NT + t;
        v[j] = a.logits[i < a.V ? i : a.V - 1];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = b0 + j * NT + t;
        if (i < a.V) acc = top2_merge(acc, float4{v[j], __int_as_float(i), -INFINITY, fabsf(v[j])});
      }
    }
  }
  const int nf = a.n_forced ? nfr : 0;
  const float margin = a.margin ? mraw : 0.0f;
  const bool use_forced = a.forced && a.n_forced && s < nf;
  const int fz = use_forced ? a.forced[s] : 0;
  acc = top2_wave(acc);
  if (lane == 0) wpart[wave] = acc;
  __syncthreads();
  // 3. the total, in every wavefront
  float4 wp = wpart[lane & (NW - 1)];   // one LDS read in every lane; lanes past 15 take the neutral summary
  asm volatile("" : "+v"(wp.x), "+v"(wp.y), "+v"(wp.z), "+v"(wp.w));
  const float4 top = top2_row0(lane < NW ? wp : none);
  bool near_tie = false;
  if (!use_forced && a.margin && a.logits && a.hn && (a.head16 || a.head32) &&
      __builtin_isfinite(top.x) && __builtin_isfinite(top.w)) {
    const double gap = (double)top.x - (double)top.z;
    near_tie = gap < (double)margin * ((double)top.w + 1e-9);
  }
  int pick = __float_as_int(top.y);
  if (near_tie) {
    // every logit within the window of the largest, recomputed exactly; one wavefront per candidate
    const double lo = (double)top.x - (double)margin * ((double)top.w + 1e-9);
    double best = -INFINITY;
    int bi = 0x7fffffff;
    for (int base = wave * 64; base < a.V; base += NT) {
      const int i = base + lane;
      const float lv = i < a.V ? a.logits[i] : -INFINITY;
      unsigned long long m = __ballot((double)lv >= lo);
      while (m) {
        const int c = base + __ffsll((long long)m) - 1;
        m &= m - 1;
        double d = 0.0;
        if (a.head32) {
          const float* wr = a.head32 + (size_t)c * a.D;
          for (int k = lane; k < a.D; k += 64) d += (double)(float)a.hn[k] * (double)wr[k];
        } else {
          const half_t* wr = a.head16 + (size_t)c * a.D;
          for (int k = lane; k < a.D; k += 64) d += (double)(float)a.hn[k] * (double)(float)wr[k];
        }
#pragma unroll
        for (int sh = 32; sh >= 1; sh >>= 1) d += __shfl_xor(d, sh, 64);
        if (d > best || (d == best && c < bi)) { best = d; bi = c; }
      }
    }
    if (lane == 0) { xbest[wave] = best; xidx[wave] = bi; }
    __syncthreads();
    double b = xbest[0];
    int bx = xidx[0];
    for (int w = 1; w < NW; ++w)
      if (xbest[w] > b || (xbest[w] == b && xidx[w] < bx)) { b = xbest[w]; bx = xidx[w]; }
    if (bx != 0x7fffffff) pick = bx;
  }
  int bidx;
  if (use_forced) bidx = fz;
  else if (!a.logits && !a.slots) bidx = 0;   // a forced-only step run past its prompt: inert token
  else bidx = pick >= a.V || pick < 0 ? 0 : pick;   // all-NaN logits: deterministic fallback
  bidx = bidx < 0 ? 0 : (bidx >= a.vocab ? a.vocab - 1 : bidx);
  if (t == 0) {
    a.tok[0] = bidx;
    if (s < a.hist_cap) a.hist[s] = bidx;
    a.step[0] = s + 1;
    a.pos[0] = p0 + 1;
  }
  if (a.embed) {
    const u4* src = (const u4*)(a.embed + (size_t)bidx * a.D);
    u4* dst = (u4*)a.h;
    for (int i = t; i < a.D / 8; i += NT) dst[i] = src[i];
  }
}

// ---- argmax per row (lowest index among ties) ----
__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ x, int V, int* __restrict__ out) {
  __shared__ float bv[4];
  __shared__ int bi[4];
  const int m = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const float* xr = x + (size_t)m * V;
  float best = -INFINITY;
  int besti = 0x7fffffff;
  for (int i = t; i < V; i += 256) {
    const float v = xr[i];
    if (v > best || (v == best && i < besti)) { best = v; besti = i; }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    const float ov = __shfl_xor(best, s, 64);
    const int oi = __shfl_xor(besti, s, 64);
    if (ov > best || (ov == best && oi < besti)) { best = ov; besti = oi; }
  }
  if (lane == 0) { bv[wave] = best; bi[wave] = besti; }
  __syncthreads();
  if (t == 0) {
    float b = bv[0];
    int bidx = bi[0];
    for (int w = 1; w < 4; ++w)
      if (bv[w] > b || (bv[w] == b && bi[w] < bidx)) { b = bv[w]; bidx = bi[w]; }
    out[m] = bidx < V ? bidx : 0;
  }
}

// ---- int32 fill / set (graph-capturable replacement for memset of small device state) ----
__global__ void fill_i32_kernel(int* p, int n, int v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}
__global__ void fill_f16_kernel(half_t* p, long long n, float v) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = (half_t)v;
}

// ---- generic strided ops for the graph executor (rank <= 5, fp16) ----
struct Shape5 {
  int rank;
  long long n;
  int dim[5];
  long long sa[5], sb[5];   // element strides of the operands (0 = broadcast)
};

__device__ __forceinline__ void unravel(const Shape5& s, long long i, long long& oa, long long& ob) {
  oa = 0; ob = 0;
  for (int d = s.rank - 1; d >= 0; --d) {
    const long long q = i / s.dim[d];
    const int c = (int)(i - q * s.dim[d]);
    oa += c * s.sa[d];
    ob += c * s.sb[d];
    i = q;
  }
}

enum { EW_ADD = 0, EW_SUB = 1, EW_MUL = 2, EW_DIV = 3, EW_MAX = 4, EW_MIN = 5, EW_POW = 6,
       EW_GE = 7, EW_GT = 8, EW_EQ = 9, EW_LT = 10, EW_LE = 11, EW_NE = 12 };

__global__ void ew_binary_kernel(const half_t* __restrict__ a, const half_t* __restrict__ b,
                                 half_t* __restrict__ y, Shape5 s, int op) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= s.n) return;
  long long oa, ob;
  unravel(s, i, oa, ob);
  const float x = (float)a[oa], z = (float)b[ob];
  float r;
  switch (op) {
    case EW_ADD: r = x + z; break;
    case EW_SUB: r = x - z; break;
    case EW_MUL: r = x * z; break;
    case EW_DIV: r = x / z; break;
    case EW_MAX: r = fmaxf(x, z); break;
    case EW_MIN: r = fminf(x, z); break;
    case EW_POW: r = powf(x, z); break;
    case EW_GE: r = x >= z; break;
    case EW_GT: r = x > z; break;
    case EW_EQ: r = x == z; break;
    case EW_LT: r = x < z; break;
    case EW_LE: r = x <= z; break;
    default: r = x != z; break;
  }
  y[i] = (half_t)r;
}

// select(cond, a, b) with broadcasting (cond != 0 picks a); strides in s.sa (cond), s.sb (a), extra for b
__global__ void ew_select_kernel(const half_t* __restrict__ c, const half_t* __restrict__ a,
                                 const half_t* __restrict__ b, half_t* __restrict__ y, Shape5 s,
                                 Shape5 s2) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= s.n) return;
  long long oc, oa, ob, dummy;
  unravel(s, i, oc, oa);
  unravel(s2, i, ob, dummy);
  y[i] = ((float)c[oc] != 0.0f) ? a[oa] : b[ob];
}

enum { UN_SILU = 0, UN_SIGMOID = 1, UN_RELU = 2, UN_EXP = 3, UN_TANH = 4, UN_AFFINE = 5, UN_SQRT = 6,
       UN_ABS = 7, UN_NEG = 8, UN_RSQRT = 9, UN_GELU_TANH = 10, UN_LOG = 11, UN_SQUARE = 12,
       UN_INVERSE = 13 };

__global__ void ew_unary_kernel(const half_t* __restrict__ x, half_t* __restrict__ y, long long n, int op,
                                float alpha, float beta) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = (float)x[i];
  float r;
  switch (op) {
    case UN_SILU: r = v / (1.0f + expf(-v)); break;
    case UN_SIGMOID: r = 1.0f / (1.0f + expf(-v)); break;
    case UN_RELU: r = fmaxf(v, 0.0f); break;
    case UN_EXP: r = expf(v); break;
    case UN_TANH: r = tanhf(v); break;
    case UN_AFFINE: r = v * alpha + beta; break;
    case UN_SQRT: r = sqrtf(v); break;
    case UN_ABS: r = fabsf(v); break;
    case UN_NEG: r = -v; break;
    case UN_RSQRT: r = 1.0f / sqrtf(v + alpha); break;
    case UN_GELU_TANH: r = 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v))); break;
    case UN_LOG: r = logf(v + alpha); break;
    case UN_SQUARE: r = v * v; break;
    default: r = 1.0f / (v + alpha); break;
  }
  y[i] = (half_t)r;
}

// y = strided gather of x into a contiguous tensor (reshape/transpose/slice/concat pieces).
// Destination may be offset/strided too via s.sb.
__global__ void copy_strided_kernel(const half_t* __restrict__ x, half_t* __restrict__ y, Shape5 s) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= s.n) return;
  long long oa, ob;
  unravel(s, i, oa, ob);
  y[ob] = x[oa];
}

// last-axis softmax / reductions: one workgroup per row, fp32 math.
__global__ __launch_bounds__(256) void softmax_kernel(const half_t* __restrict__ x, half_t* __restrict__ y, int cols) {
  __shared__ float red[4];
  const int r = blockIdx.x, t = threadIdx.x;
  const half_t* xr = x + (size_t)r * cols;
  float m = -INFINITY;
  for (int i = t; i < cols; i += 256) m = fmaxf(m, (float)xr[i]);
  m = wave_max(m);
  if ((t & 63) == 0) red[t >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float s = 0.0f;
  for (int i = t; i < cols; i += 256) s += expf((float)xr[i] - m);
  s = wave_sum(s);
  if ((t & 63) == 0) red[t >> 6] = s;
  __syncthreads();
  s = red[0] + red[1] + red[2] + red[3];
  const float inv = 1.0f / s;
  for (int i = t; i < cols; i += 256) y[(size_t)r * cols + i] = (half_t)(expf((float)xr[i] - m) * inv);
}

enum { RED_SUM = 0, RED_MAX = 1, RED_MEAN = 2, RED_MIN = 3, RED_SUMSQ = 4 };
__global__ __launch_bounds__(256) void reduce_kernel(const half_t* __restrict__ x, half_t* __restrict__ y,
                                                     int cols, int op) {
  __shared__ float red[4];
  const int r = blockIdx.x, t = threadIdx.x;
  const half_t* xr = x + (size_t)r * cols;
  const bool mx = op == RED_MAX, mn = op == RED_MIN;
  float acc = mx ? -INFINITY : mn ? INFINITY : 0.0f;
  for (int i = t; i < cols; i += 256) {
    const float v = (float)xr[i];
    acc = mx ? fmaxf(acc, v) : mn ? fminf(acc, v) : op == RED_SUMSQ ? acc + v * v : acc + v;
  }
  acc = mx ? wave_max(acc) : mn ? -wave_max(-acc) : wave_sum(acc);
  if ((t & 63) == 0) red[t >> 6] = acc;
  __syncthreads();
  if (t == 0) {
    float v = red[0];
    for (int w = 1; w < 4; ++w) v = mx ? fmaxf(v, red[w]) : mn ? fminf(v, red[w]) : v + red[w];
    if (op == RED_MEAN) v /= (float)cols;
    y[r] = (half_t)v;
  }
}

// C[b] = A[b] @ B[b], fp16 in/out, fp32 accumulate; 16x16 output tile per workgroup via LDS.
__global__ __launch_bounds__(256) void bmm_kernel(const half_t* __restrict__ A, const half_t* __restrict__ B,
                                                  half_t* __restrict__ C, int M, int N, int K,
                                                  long long sa, long long sb, long long sc) {
  __shared__ float ta[16][17], tb[16][17];
  const int bz = blockIdx.z, tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int row = blockIdx.y * 16 + ty, col = blockIdx.x * 16 + tx;
  const half_t* a = A + bz * sa;
  const half_t* b = B + bz * sb;
  float acc = 0.0f;
  for (int k0 = 0; k0 < K; k0 += 16) {
    ta[ty][tx] = (row < M && k0 + tx < K) ? (float)a[(size_t)row * K + k0 + tx] : 0.0f;
    tb[ty][tx] = (k0 + ty < K && col < N) ? (float)b[(size_t)(k0 + ty) * N + col] : 0.0f;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) acc = __builtin_fmaf(ta[ty][k], tb[k][tx], acc);
    __syncthreads();
  }
  if (row < M && col < N) C[bz * sc + (size_t)row * N + col] = (half_t)acc;
}

static inline unsigned blocks_for(long long n, int bs) { return (unsigned)((n + bs - 1) / bs); }

static int make_shape(Shape5& s, int rank, const int* dim, const long long* sa, const long long* sb) {
  AFX_REQUIRE(rank >= 1 && rank <= 5, "rank %d outside [1, 5]", rank);
  s.rank = rank;
  s.n = 1;
  for (int d = 0; d < rank; ++d) {
    AFX_REQUIRE(dim[d] >= 1, "dimension %d is %d", d, dim[d]);
    s.dim[d] = dim[d];
    s.sa[d] = sa ? sa[d] : 0;
    s.sb[d] = sb ? sb[d] : 0;
    s.n *= dim[d];
  }
  return 0;
}


// ---- temperature / top-k / top-p sampling on the device (the reference's _sample,
// aneforge/llm.py:406-419, with np.random.choice's inverse-CDF draw) ----
// Logits are ranked by an order-preserving 32-bit key of their fp32 value: logits / T is monotone
// in the logit and fp32 -> fp64 is exact, so the k-th largest scaled logit and the top-p nucleus
// are thresholds on that key.  The selection: the top-k floor (the k-th largest key; ties kept, as
// lg < kth -> -inf keeps them) and the top-p nucleus edge (the key where the mass from the top
// first reaches top_p * Z) by 8-bit radix selects over bins of the key.  Ties at the nucleus edge
// keep the highest indices first (np.argsort(p)[::-1] of a stably sorted array).  The draw: the
// first index whose running kept mass (in index order) exceeds u * total, u = uniforms[*step].
// Four launches, so that whole-vocabulary passes run on many CUs:
// - max, one workgroup per 2048-logit chunk: the chunk's largest key;
// - prep, one workgroup per chunk: the largest key (from the chunk maxima), e_i = exp(x_i / T -
//   max / T) in fp64, and per chunk the sum of e and the count and mass of its logits in each of
//   256 bins of (max - x) / T, T / 8 wide from the top (bin 255 holds the maximum, bin 0 everything
//   32 T or more below it; masses summed in a fixed order).  The bin is monotone in the key;
// - gather, one workgroup per chunk: every workgroup merges the bins and derives the same window
//   of bins that holds what the cut needs: for top-k every bin from the one holding the k-th
//   largest key up, for top-p alone the one bin holding the nucleus edge (the bins above it are
//   kept whole).  Each chunk compacts its logits in the window, in index order, into the workspace
//   (up to kSmpWin logits);
// - pick, one workgroup of 256 threads: without a cut the draw needs the chunk sums and one chunk;
//   with a window the selection runs on its logits (for top-p alone with the per-chunk mass above
//   the edge for the draw), copied to LDS when at most kSmpCap, else read from the workspace; a
//   window above kSmpWin runs the selection over the whole vocabulary.
constexpr int kSampleThreads = 256;
constexpr int kSampleWaves = kSampleThreads / 64;
constexpr int kSmpPrepThreads = 256;
constexpr int kSmpPer = 8;                                    // logits per prep / gather thread
constexpr int kSmpChunk = kSmpPrepThreads * kSmpPer;          // logits per chunk
constexpr int kSmpCap = 6144;                                 // window logits the pick kernel holds in LDS
constexpr int kSmpWin = 1 << 16;                              // window logits gather compacts into the workspace
constexpr int kSmpMaxChunks = 1024;                           // V <= 2^21

__host__ __device__ inline long long smp_nb(int V) { return ((long long)V + kSmpChunk - 1) / kSmpChunk; }
__host__ __device__ inline long long smp_stats_off(int V) { return ((long long)V * 8 + 255) / 256 * 256; }
// The window of bins the cut needs (see the section comment); mode 0: no cut.
struct SmpWin {
  int lo, hi, mode;
  long long ncand;
  double above;                                      // top-p alone: the mass of the bins above hi
};
// Workspace: e[V] (fp64); a 64-byte header (the largest key, the vocabulary's mass, the window);
// per chunk its sum bsum[NB]; per chunk and bin the mass smass[NB][256] and count scnt[NB][256] of
// that bin and every bin above it (suffix sums from the top); the window's e ce[kSmpWin] (fp64);
// window offsets coff[NB + 1]; the window's keys ckey[kSmpWin] and indices cidx[kSmpWin]; chunk
// maxima cmax[NB].
struct SmpHdr {
  unsigned maxkey;
  int pad;
  double Z_all;
  SmpWin win;
};
static_assert(sizeof(SmpHdr) <= 64, "sampling workspace header");
__host__ __device__ inline long long smp_ws_bytes(int V) {
  const long long nb = smp_nb(V);
  return smp_stats_off(V) + 64 + nb * 8 + nb * 256 * 8 + (long long)kSmpWin * 8 + nb * 256 * 4 + (nb + 1) * 4 +
         (long long)kSmpWin * 8 + nb * 4;
}
struct SmpWs {
  SmpHdr* hdr;
  double *e, *bsum, *smass, *ce;
  unsigned *scnt, *coff, *ckey, *cmax;
  int* cidx;
};
__device__ __forceinline__ SmpWs smp_ws(double* ws, int V) {
  unsigned char* s = (unsigned char*)ws + smp_stats_off(V);
  const long long nb = smp_nb(V);
  SmpWs w;
  w.e = ws;
  w.hdr = (SmpHdr*)s;
  w.bsum = (double*)(s + 64);
  w.smass = w.bsum + nb;
  w.ce = w.smass + nb * 256;
  w.scnt = (unsigned*)(w.ce + kSmpWin);
  w.coff = w.scnt + nb * 256;
  w.ckey = w.coff + nb + 1;
  w.cidx = (int*)(w.ckey + kSmpWin);
  w.cmax = (unsigned*)(w.cidx + kSmpWin);
  return w;
}

__device__ __forceinline__ uint32_t logit_key(float x) {
  if (x != x) x = -INFINITY;                         // NaN ranks below every number
  const uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_logit(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
template <class T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const T o = __shfl_up(v, m, 64);
    if (lane >= m) v += o;
  }
  return v;
}

// The bin of logit x: 255 - floor((maxv - x) * s) with s = 8 / T, clamped to [0, 255]; NaN and
// -inf land in bin 0.  Monotone in the key (float subtraction and scaling are monotone).
__device__ __forceinline__ int smp_bin(float x, float maxv, float s) {
  if (x != x) return 0;
  if (!(x < maxv)) return 255;
  const float d = (maxv - x) * s;
  return d >= 255.0f ? 0 : 255 - (int)d;
}

__global__ __launch_bounds__(kSmpPrepThreads) void sample_max_kernel(const float* __restrict__ logits, int V,
                                                                     const double* __restrict__ params,
                                                                     double* __restrict__ ws) {
  __shared__ unsigned s_max[kSmpPrepThreads / 64];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, b = blockIdx.x;
  if (!(params[0] > 0.0)) return;
  const SmpWs w = smp_ws(ws, V);
  const int c0 = b * kSmpChunk + t * kSmpPer;
  float x[kSmpPer];
#pragma unroll
  for (int j = 0; j < kSmpPer; ++j) x[j] = logits[c0 + j < V ? c0 + j : V - 1];   // clamped: a real logit
  unsigned mk = 0u;
#pragma unroll
  for (int j = 0; j < kSmpPer; ++j) mk = max(mk, logit_key(x[j]));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) mk = max(mk, (unsigned)__shfl_xor((int)mk, m, 64));
  if (lane == 0) s_max[wave] = mk;
  __syncthreads();
  if (t == 0) w.cmax[b] = max(max(s_max[0], s_max[1]), max(s_max[2], s_max[3]));
}

__global__ __launch_bounds__(kSmpPrepThreads) void sample_prep_kernel(const float* __restrict__ logits, int V,
                                                                      const double* __restrict__ params,
                                                                      double* __restrict__ ws) {
  constexpr int NW = kSmpPrepThreads / 64;
  __shared__ unsigned s_max[NW];
  __shared__ double s_sum[NW];
  __shared__ unsigned h_cnt[256];
  __shared__ double h_mass[NW][256];                 // one copy per wavefront: a fixed summation order
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, b = blockIdx.x;
  const double temp = params[0];
  if (!(temp > 0.0)) return;                         // greedy: the pick kernel scans the logits
  const SmpWs w = smp_ws(ws, V);
  h_cnt[t] = 0u;
#pragma unroll
  for (int j = 0; j < NW; ++j) h_mass[j][t] = 0.0;
  // 1. the largest key, from the chunk maxima
  const int nb = (int)smp_nb(V);
  unsigned mk = 0u;
  for (int c = t; c < nb; c += kSmpPrepThreads) mk = max(mk, w.cmax[c]);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) mk = max(mk, (unsigned)__shfl_xor((int)mk, m, 64));
  if (lane == 0) s_max[wave] = mk;
  __syncthreads();                                   // also orders the bin clears before the adds
  mk = max(max(s_max[0], s_max[1]), max(s_max[2], s_max[3]));
  if (b == 0 && t == 0) w.hdr->maxkey = mk;
  const double lgmax = (double)key_logit(mk) / temp;
  const float maxv = key_logit(mk), sb = (float)(8.0 / temp);
  // 2. this chunk: e, the chunk sum, and counts and masses per bin
  const int c0 = b * kSmpChunk + t * kSmpPer;
  float x[kSmpPer];
#pragma unroll
  for (int j = 0; j < kSmpPer; ++j) x[j] = logits[c0 + j < V ? c0 + j : V - 1];
  double part = 0.0;
#pragma unroll
  for (int j = 0; j < kSmpPer; ++j) {
    if (c0 + j >= V) break;
    const int bin = smp_bin(x[j], maxv, sb);
    const double v = x[j] == x[j] ? exp((double)x[j] / temp - lgmax) : 0.0;
    w.e[c0 + j] = v;
    part += v;
    atomicAdd(&h_cnt[bin], 1u);
    atomicAdd(&h_mass[wave][bin], v);
  }
  part = wave_sum_f64(part);
  if (lane == 0) s_sum[wave] = part;
  __syncthreads();
  if (t == 0) w.bsum[b] = ((s_sum[0] + s_sum[1]) + s_sum[2]) + s_sum[3];
  // suffix sums over the bins (bin t and every bin above it), in a fixed order
  unsigned sc = h_cnt[t];
  double sm = ((h_mass[0][t] + h_mass[1][t]) + h_mass[2][t]) + h_mass[3][t];
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const unsigned oc = __shfl_down(sc, m, 64);
    const double om = __shfl_down(sm, m, 64);
    if (lane + m < 64) { sc += oc; sm += om; }
  }
  __syncthreads();                                   // the bins are read: reuse s_max / s_sum
  if (lane == 0) { s_max[wave] = sc; s_sum[wave] = sm; }
  __syncthreads();
  for (int ww = NW - 1; ww > wave; --ww) { sc += s_max[ww]; sm += s_sum[ww]; }
  w.scnt[(size_t)b * 256 + t] = sc;
  w.smass[(size_t)b * 256 + t] = sm;
}

// The vocabulary's mass from the chunk sums: lane l of a wavefront owns chunks [l * g, l * g + g)
// (lsum, summed in order), incl is the inclusive scan over the lanes; returns the total.  The
// gather and pick kernels compute it with the same code, so they agree to the bit.
__device__ __forceinline__ double smp_total(const double* csum, int nb, double& lsum, double& incl) {
  const int lane = threadIdx.x & 63, g = (nb + 63) / 64;
  lsum = 0.0;
  for (int j = 0; j < g; ++j) {
    const int c = lane * g + j;
    lsum += c < nb ? csum[c] : 0.0;
  }
  incl = wave_incl_scan(lsum);
  return __shfl(incl, 63, 64);
}

// Wavefront 0's walk of 256 bins from the top (lane l holds bins 4l .. 4l + 3): the highest bin
// b >= 1 whose inclusive sum from the top, started at `start`, reaches `need` (else bin 0), and the
// sum strictly above it.  Counts are exact in any order; masses add in a fixed tree order.
template <class T>
__device__ __forceinline__ int bin_walk(const T (&v)[4], T start, T need, T& above) {
  const int lane = threadIdx.x & 63;
  const T lsum = ((v[3] + v[2]) + v[1]) + v[0];
  T suf = lsum;                                      // sum over the lanes at and above this one
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const T o = __shfl_down(suf, m, 64);
    if (lane + m < 64) suf += o;
  }
  const T sa = suf - lsum;                           // lanes above (exact for counts)
  const unsigned long long reach = __ballot(start + suf >= need);
  int b = 0;
  T acc;
  if (reach) {
    const int L = 63 - __clzll((long long)reach);
    acc = start + __shfl(sa, L, 64);
    bool found = false;
    for (int j = 3; j >= (L == 0 ? 1 : 0); --j) {
      const T c = __shfl(v[j], L, 64);
      if (acc + c >= need) { b = 4 * L + j; found = true; break; }
      acc += c;
    }
    if (!found) b = 0;                               // only lane 0's bin 0 is left
  } else {
    acc = start + __shfl(suf, 0, 64) - __shfl(v[0], 0, 64);   // every bin from 1 up
  }
  above = acc;
  return b;
}

// Wavefront 0's search of 256 suffix sums S (lane l holds bins 4l .. 4l + 3; non-increasing in
// the bin): the highest bin b >= 1 with S[b] >= need (else bin 0), and S[b + 1] (0 past the top).
template <class T>
__device__ __forceinline__ int suffix_walk(const T (&S)[4], T need, T& next) {
  const int lane = threadIdx.x & 63;
  int jb = -1;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if ((lane > 0 || j > 0) && S[j] >= need) jb = j;
  const unsigned long long has = __ballot(jb >= 0);
  const T up = __shfl_down(S[0], 1, 64);             // the next lane's first bin
  const T after[4] = {S[1], S[2], S[3], lane < 63 ? up : (T)0};
  if (!has) {
    next = __shfl(S[1], 0, 64);
    return 0;
  }
  const int L = 63 - __clzll((long long)has);
  const int j = __shfl(jb, L, 64);
  const T a0 = __shfl(after[0], L, 64), a1 = __shfl(after[1], L, 64), a2 = __shfl(after[2], L, 64),
          a3 = __shfl(after[3], L, 64);
  next = j == 0 ? a0 : j == 1 ? a1 : j == 2 ? a2 : a3;
  return 4 * L + j;
}

// Called by every thread of the workgroup (>= 256 threads); mc / mm: LDS scratch of 256 entries.
// The merged suffix sums: counts exact, masses added over the chunks in order; the top-k window
// needs the counts only.  Every gather workgroup merges for itself: a merge by one workgroup needs
// a device-scope fence per chunk, which measured slower at every vocabulary size up to 2^21.
__device__ void smp_window(const SmpWs& w, int nb, int V, double top_p, long long top_k, double Z_all, unsigned* mc,
                           double* mm, SmpWin& out) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const bool cut_k = top_k > 0 && top_k < V, cut_p = top_p > 0.0 && top_p < 1.0;
  if (!cut_k && !cut_p) {
    if (t == 0) out = SmpWin{0, -1, 0, 0, 0.0};
    __syncthreads();
    return;
  }
  if (t < 256 && cut_k) {
    unsigned c = 0;
    for (int b0 = 0; b0 < nb; b0 += 32) {
      unsigned cv[32];
#pragma unroll
      for (int j = 0; j < 32; ++j) cv[j] = w.scnt[(size_t)(b0 + j < nb ? b0 + j : nb - 1) * 256 + t];
#pragma unroll
      for (int j = 0; j < 32; ++j)
        if (b0 + j < nb) c += cv[j];
    }
    mc[t] = c;
  } else if (t < 256) {
    unsigned c = 0;
    double m = 0.0;
    for (int b0 = 0; b0 < nb; b0 += 16) {
      unsigned cv[16];
      double mv[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int b = b0 + j < nb ? b0 + j : nb - 1;
        cv[j] = w.scnt[(size_t)b * 256 + t];
        mv[j] = w.smass[(size_t)b * 256 + t];
      }
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (b0 + j < nb) { c += cv[j]; m += mv[j]; }
    }
    mc[t] = c;
    mm[t] = m;
  }
  __syncthreads();
  if (wave == 0) {
    if (cut_k) {
      long long v[4], next;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = mc[4 * lane + j];
      const int b1 = suffix_walk<long long>(v, top_k, next);
      if (lane == 0) out = SmpWin{b1, 255, 1, (long long)mc[b1], 0.0};
    } else {
      double v[4], next;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = mm[4 * lane + j];
      const int be = suffix_walk<double>(v, top_p * Z_all, next);
      const long long n = (long long)mc[be] - (be < 255 ? (long long)mc[be + 1] : 0ll);
      if (lane == 0) out = SmpWin{be, be, 2, n, next};
    }
  }
  __syncthreads();
}

__device__ __forceinline__ bool smp_use_window(const SmpWin& win, int nb) {
  return win.mode != 0 && win.ncand >= 1 && win.ncand <= kSmpWin && nb <= kSmpMaxChunks;
}

__global__ __launch_bounds__(kSmpPrepThreads) void sample_gather_kernel(const float* __restrict__ logits, int V,
                                                                        const double* __restrict__ params,
                                                                        double* __restrict__ ws) {
  constexpr int NW = kSmpPrepThreads / 64;
  __shared__ unsigned mc[256];
  __shared__ double mm[256];
  __shared__ SmpWin win;
  __shared__ unsigned wc[kSmpMaxChunks];
  __shared__ unsigned s_u[NW];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, c = blockIdx.x;
  const double temp = params[0], top_p = params[1];
  const long long top_k = (long long)params[2];
  if (!(temp > 0.0)) return;
  const SmpWs w = smp_ws(ws, V);
  const int nb = (int)smp_nb(V);
  double lsum, incl;
  const double Z_all = smp_total(w.bsum, nb, lsum, incl);
  smp_window(w, nb, V, top_p, top_k, Z_all, mc, mm, win);
  if (c == 0 && t == 0) {                            // the pick kernel takes the window from here
    w.hdr->Z_all = Z_all;
    w.hdr->win = win;
  }
  if (!smp_use_window(win, nb)) return;              // workgroup-uniform
  const int lo = win.lo, hi = win.hi;
  const float maxv = key_logit(w.hdr->maxkey), sb = (float)(8.0 / temp);
  // the window's logits per chunk (suffix counts: [lo, hi] = S[lo] - S[hi + 1]) and this chunk's offset
  for (int cc = t; cc < nb; cc += kSmpPrepThreads)
    wc[cc] = w.scnt[(size_t)cc * 256 + lo] - (hi < 255 ? w.scnt[(size_t)cc * 256 + hi + 1] : 0u);
  __syncthreads();
  unsigned before = 0;
  for (int cc = t; cc < c; cc += kSmpPrepThreads) before += wc[cc];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) before += (unsigned)__shfl_xor((int)before, m, 64);
  if (lane == 0) s_u[wave] = before;
  __syncthreads();
  const unsigned off = (s_u[0] + s_u[1]) + (s_u[2] + s_u[3]);
  if (t == 0) {
    w.coff[c] = off;
    if (c == nb - 1) w.coff[nb] = off + wc[c];
  }
  // compact the chunk's window logits in index order: thread t owns 8 consecutive logits
  const int c0 = c * kSmpChunk + t * kSmpPer;
  float x[kSmpPer];
  int n = 0;
#pragma unroll
  for (int j = 0; j < kSmpPer; ++j) x[j] = logits[c0 + j < V ? c0 + j : V - 1];
#pragma unroll
  for (int j = 0; j < kSmpPer; ++j) {
    const int bin = smp_bin(x[j], maxv, sb);
    n += c0 + j < V && bin >= lo && bin <= hi;
  }
  const int inc = wave_incl_scan(n);
  __syncthreads();
  if (lane == 63) s_u[wave] = inc;
  __syncthreads();
  int pos = (int)off + inc - n;
  for (int ww = 0; ww < wave; ++ww) pos += s_u[ww];
#pragma unroll
  for (int j = 0; j < kSmpPer; ++j) {
    const int bin = smp_bin(x[j], maxv, sb);
    if (c0 + j >= V || bin < lo || bin > hi || pos >= kSmpWin) continue;
    w.ckey[pos] = logit_key(x[j]);
    w.cidx[pos] = c0 + j;
    w.ce[pos] = w.e[c0 + j];
    ++pos;
  }
}

struct SampleSmem {
  union {
    unsigned cnt[kSampleWaves][256];
    double mass[kSampleWaves][256];
  } h;
  unsigned ckey[kSmpCap];                            // the window's logits, in index order
  int cidx[kSmpCap];
  double ce[kSmpCap];
  double km[kSmpMaxChunks];                          // per-chunk kept mass (top-p alone)
  double wsum[kSampleWaves];
  unsigned wmax[kSampleWaves], wmin[kSampleWaves];
  unsigned prefix, mask;
  long long remaining;
  double above, target;
  long long wtie[kSampleWaves];
  int token, last, tie_cut;
};

// The whole vocabulary (keys from the logits, e from the workspace) or the window in LDS.
struct SmpAll {
  const float* logits;
  const double* e;
  int n;
  __device__ unsigned key(int i) const { return logit_key(logits[i]); }
  __device__ double mass(int i) const { return e[i]; }
  __device__ int index(int i) const { return i; }
};
struct SmpCand {
  const unsigned* k;
  const int* idx;
  const double* e;
  int n;
  __device__ unsigned key(int i) const { return k[i]; }
  __device__ double mass(int i) const { return e[i]; }
  __device__ int index(int i) const { return idx[i]; }
};

constexpr int kSmpBatch = 8;   // loads in flight per thread in the passes

// Radix select over keys >= floor_key matching the current prefix, from bit `top` down.  COUNT: the
// key holding the remaining-th largest element; otherwise the key at which the mass from the top
// first reaches target.
template <bool COUNT, class Acc>
__device__ void radix_select(const Acc& A, unsigned floor_key, SampleSmem& sm, int top = 24) {
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  for (int shift = top; shift >= 0; shift -= 8) {
    for (int i = t; i < kSampleWaves * 256; i += kSampleThreads) {
      if (COUNT) (&sm.h.cnt[0][0])[i] = 0u;
      else (&sm.h.mass[0][0])[i] = 0.0;
    }
    __syncthreads();
    const unsigned prefix = sm.prefix, mask = sm.mask;
    for (int b0 = 0; b0 < A.n; b0 += kSmpBatch * kSampleThreads) {
      unsigned k[kSmpBatch];
      double m[kSmpBatch];
#pragma unroll
      for (int j = 0; j < kSmpBatch; ++j) {
        const int i = b0 + j * kSampleThreads + t;
        const int ic = i < A.n ? i : A.n - 1;
        k[j] = A.key(ic);
        m[j] = COUNT ? 0.0 : A.mass(ic);
      }
#pragma unroll
      for (int j = 0; j < kSmpBatch; ++j) {
        if (b0 + j * kSampleThreads + t >= A.n || k[j] < floor_key || (k[j] & mask) != prefix) continue;
        const int bin = (k[j] >> shift) & 255;
        if (COUNT) atomicAdd(&sm.h.cnt[wave][bin], 1u);
        else atomicAdd(&sm.h.mass[wave][bin], m[j]);
      }
    }
    __syncthreads();
    if (t < 256) {                                   // merge the wavefront copies in a fixed order
      if (COUNT) {
        unsigned c = 0;
        for (int w = 0; w < kSampleWaves; ++w) c += sm.h.cnt[w][t];
        sm.h.cnt[0][t] = c;
      } else {
        double ms = 0.0;
        for (int w = 0; w < kSampleWaves; ++w) ms += sm.h.mass[w][t];
        sm.h.mass[0][t] = ms;
      }
    }
    __syncthreads();
    if (wave == 0) {
      int b;
      if (COUNT) {
        long long v[4], above;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = sm.h.cnt[0][4 * lane + j];
        b = bin_walk<long long>(v, 0ll, sm.remaining, above);
        if (lane == 0) sm.remaining -= above;
      } else {
        double v[4], above;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = sm.h.mass[0][4 * lane + j];
        b = bin_walk<double>(v, sm.above, sm.target, above);
        if (lane == 0) sm.above = above;
      }
      if (lane == 0) {
        sm.prefix |= (unsigned)b << shift;
        sm.mask |= 255u << shift;
      }
    }
    __syncthreads();
  }
}

// The same radix select run by wavefront 0 alone on one LDS histogram (no workgroup barrier per
// pass), for windows of at most kSmpWaveSel logits; the caller follows it with a barrier.  LDS
// operations of one wavefront complete in order, so a fence and wave barrier order each pass.
constexpr int kSmpWaveSel = 1024;
__device__ __forceinline__ void smp_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
template <bool COUNT, class Acc>
__device__ void radix_select_wave(const Acc& A, unsigned floor_key, SampleSmem& sm, int top = 24) {
  const int lane = threadIdx.x & 63;
  unsigned prefix = sm.prefix, mask = sm.mask;
  long long remaining = sm.remaining;
  double above = sm.above;
  const double target = sm.target;
  for (int shift = top; shift >= 0; shift -= 8) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (COUNT) sm.h.cnt[0][4 * lane + j] = 0u;
      else sm.h.mass[0][4 * lane + j] = 0.0;
    }
    smp_wave_sync();
    for (int i = lane; i < A.n; i += 64) {
      const unsigned k = A.key(i);
      if (k < floor_key || (k & mask) != prefix) continue;
      const int bin = (k >> shift) & 255;
      if (COUNT) atomicAdd(&sm.h.cnt[0][bin], 1u);
      else atomicAdd(&sm.h.mass[0][bin], A.mass(i));
    }
    smp_wave_sync();
    int b;
    if (COUNT) {
      long long v[4], ab;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = sm.h.cnt[0][4 * lane + j];
      b = bin_walk<long long>(v, 0ll, remaining, ab);
      remaining -= ab;
    } else {
      double v[4], ab;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = sm.h.mass[0][4 * lane + j];
      b = bin_walk<double>(v, above, target, ab);
      above = ab;
    }
    prefix |= (unsigned)b << shift;
    mask |= 255u << shift;
    smp_wave_sync();                                 // the bins are read before the next pass clears them
  }
  if (lane == 0) {
    sm.prefix = prefix;
    sm.mask = mask;
    sm.remaining = remaining;
    sm.above = above;
  }
}

// The two-level draw: the chunk whose running kept mass first exceeds u * total (chunk masses
// cm(c), inclusive scan over the lanes in a fixed order), then the position inside it (two logits
// per thread, kept(i, key) selects; e from the workspace).  Rounding that leaves no crossing takes
// the chunk's last kept logit.
template <class CM, class KEPT>
__device__ int smp_chunk_draw(const float* logits, const double* e, int V, int nb, double u, CM cm, KEPT kept,
                              SampleSmem& sm) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, g = (nb + 63) / 64;
  double lsum = 0.0;
  for (int j = 0; j < g; ++j) {
    const int c = lane * g + j;
    lsum += c < nb ? cm(c) : 0.0;
  }
  const double incl = wave_incl_scan(lsum);
  const double total = __shfl(incl, 63, 64);
  const double target = u * total;
  const unsigned long long over = __ballot(incl > target);
  int cb = -1;
  double base = 0.0;
  if (over) {
    const int L = __ffsll((long long)over) - 1;
    double run = __shfl(incl - lsum, L, 64);
    int lastc = -1;
    double lastbase = 0.0;
    for (int j = 0; j < g; ++j) {
      const int c = L * g + j;
      if (c >= nb) break;
      const double m = cm(c);
      if (m > 0.0) { lastc = c; lastbase = run; }
      if (run + m > target) { cb = c; base = run; break; }
      run += m;
    }
    if (cb < 0) { cb = lastc; base = lastbase; }     // rounding inside the lane's chunks
  }
  if (cb < 0) {                                      // target at the very end: the last chunk with mass
    cb = nb - 1;
    while (cb > 0 && !(cm(cb) > 0.0)) --cb;
    base = -INFINITY;                                // no crossing inside: its last kept logit
  }
  constexpr int PT = kSmpChunk / kSampleThreads;     // consecutive logits per thread
  const int e0 = cb * kSmpChunk + PT * t;
  float x[PT];
  double a[PT];
#pragma unroll
  for (int j = 0; j < PT; ++j) {
    x[j] = logits[e0 + j < V ? e0 + j : V - 1];
    a[j] = e[e0 + j < V ? e0 + j : V - 1];
  }
  double loc = 0.0;
  int lastp = -1;
#pragma unroll
  for (int j = 0; j < PT; ++j) {
    a[j] = e0 + j < V && kept(e0 + j, logit_key(x[j])) ? a[j] : 0.0;
    loc += a[j];
    if (a[j] > 0.0) lastp = e0 + j;
  }
  const double inc = wave_incl_scan(loc);
  __syncthreads();
  if (lane == 63) sm.wsum[wave] = inc;
  if (t == 0) { sm.token = 0x7fffffff; sm.last = -1; }
  __syncthreads();
  double ex = inc - loc;
  for (int ww = 0; ww < wave; ++ww) ex += sm.wsum[ww];
  const double tg = target - base;
  if (loc > 0.0 && ex <= tg && tg < ex + loc) {
    double run = ex;
    int pk = -1;
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      if (pk >= 0 || a[j] == 0.0) continue;
      run += a[j];
      if (run > tg) pk = e0 + j;
    }
    atomicMin(&sm.token, pk >= 0 ? pk : lastp);     // rounding inside the range: its last kept logit
  }
  atomicMax(&sm.last, lastp);
  __syncthreads();
  return sm.token != 0x7fffffff ? sm.token : (sm.last >= 0 ? sm.last : 0);
}

// Top-k floor, top-p edge, the kept set and the draw over A (positions in index order); returns
// the vocabulary index.  Z_all: the vocabulary's mass (used without a top-k cut).
// The radix passes start below the key bytes that every element of A shares (cp_prefix under
// cp_mask, first pass at bit cp_top).
template <class Acc>
__device__ int smp_select_draw(const Acc& A, int V, double temp, double lgmax, double top_p, long long top_k,
                               double u, double Z_all, unsigned cp_prefix, unsigned cp_mask, int cp_top,
                               SampleSmem& sm) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  if (t == 0) { sm.prefix = cp_prefix; sm.mask = cp_mask; sm.above = 0.0; sm.token = 0x7fffffff; sm.last = -1; }
  __syncthreads();
  // top-k: keep the logits >= the k-th largest (ties included)
  unsigned kfloor = 0u;
  const bool cut_k = top_k > 0 && top_k < V;
  const bool small = A.n <= kSmpWaveSel;
  if (cut_k) {
    if (t == 0) sm.remaining = top_k;
    __syncthreads();
    if (small) {
      if (wave == 0) radix_select_wave<true>(A, 0u, sm, cp_top);
      __syncthreads();
    } else {
      radix_select<true>(A, 0u, sm, cp_top);
    }
    kfloor = sm.prefix;
    __syncthreads();
    if (t == 0) { sm.prefix = cp_prefix; sm.mask = cp_mask; }
  }
  // Z: the kept mass after top-k
  double Z = Z_all;
  if (cut_k) {
    double part = 0.0;
    for (int b0 = 0; b0 < A.n; b0 += kSmpBatch * kSampleThreads) {
      unsigned k[kSmpBatch];
      double m[kSmpBatch];
#pragma unroll
      for (int j = 0; j < kSmpBatch; ++j) {
        const int i = b0 + j * kSampleThreads + t;
        const int ic = i < A.n ? i : A.n - 1;
        k[j] = A.key(ic);
        m[j] = A.mass(ic);
      }
#pragma unroll
      for (int j = 0; j < kSmpBatch; ++j)
        if (b0 + j * kSampleThreads + t < A.n && k[j] >= kfloor) part += m[j];
    }
    part = wave_sum_f64(part);
    __syncthreads();
    if (lane == 0) sm.wsum[wave] = part;
    __syncthreads();
    Z = 0.0;
    for (int w = 0; w < kSampleWaves; ++w) Z += sm.wsum[w];
  }
  // top-p: the smallest top set whose mass reaches top_p * Z
  unsigned pkey = kfloor;
  long long ntie = 0;                                // tied logits kept at pkey (0: no top-p cut)
  if (top_p > 0.0 && top_p < 1.0) {
    __syncthreads();
    if (t == 0) sm.target = top_p * Z;
    __syncthreads();
    if (small) {
      if (wave == 0) radix_select_wave<false>(A, kfloor, sm, cp_top);
      __syncthreads();
    } else {
      radix_select<false>(A, kfloor, sm, cp_top);
    }
    pkey = sm.prefix;
    const double q = exp((double)key_logit(pkey) / temp - lgmax);
    const double need = sm.target - sm.above;
    ntie = need > 0.0 ? (long long)ceil(need / q) : 1;
    if (ntie < 1) ntie = 1;
  }
  __syncthreads();
  // the kept set: keys above pkey, and at pkey the first ntie ties counted from the highest index
  // down (all of them without a top-p cut).  Thread t owns positions [i0, i1), read kSmpBatch at a time.
  const int per = (A.n + kSampleThreads - 1) / kSampleThreads;
  const int i0 = min(A.n, t * per), i1 = min(A.n, i0 + per);
  auto load = [&](int base, unsigned (&k)[kSmpBatch], double (&m)[kSmpBatch], bool with_mass) {
#pragma unroll
    for (int j = 0; j < kSmpBatch; ++j) {
      const int i = base + j < i1 ? base + j : i1 - 1;
      k[j] = A.key(i);
      m[j] = with_mass ? A.mass(i) : 0.0;
    }
  };
  long long rties = 0;                               // ties at pkey in this thread's range
  if (ntie)
    for (int b = i0; b < i1; b += kSmpBatch) {
      unsigned k[kSmpBatch];
      double m[kSmpBatch];
      load(b, k, m, false);
#pragma unroll
      for (int j = 0; j < kSmpBatch; ++j) rties += b + j < i1 && k[j] == pkey;
    }
  long long ties_after = 0;                          // ties at pkey in higher threads' ranges
  if (ntie) {
    long long suf = rties;                           // inclusive suffix sum within the wavefront
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      const long long o = __shfl_down(suf, m, 64);
      if (lane + m < 64) suf += o;
    }
    if (lane == 0) sm.wtie[wave] = suf;
    __syncthreads();
    ties_after = suf - rties;
    for (int w = wave + 1; w < kSampleWaves; ++w) ties_after += sm.wtie[w];
  }
  double local = 0.0;                                // kept mass of the range, in index order
  {
    long long higher = ties_after + rties;           // ties at positions >= i (before visiting i)
    for (int b = i0; b < i1; b += kSmpBatch) {
      unsigned k[kSmpBatch];
      double m[kSmpBatch];
      load(b, k, m, true);
#pragma unroll
      for (int j = 0; j < kSmpBatch; ++j) {
        if (b + j >= i1) break;
        const bool tie = ntie && k[j] == pkey;
        if (tie) --higher;                           // now: ties at positions > i
        if (k[j] >= pkey && (!tie || higher < ntie)) local += m[j];
      }
    }
  }
  const double incl = wave_incl_scan(local);         // exclusive prefix over threads, fixed order
  __syncthreads();
  if (lane == 63) sm.wsum[wave] = incl;
  __syncthreads();
  double excl = incl - local, total = 0.0;
  for (int w = 0; w < kSampleWaves; ++w) {
    if (w < wave) excl += sm.wsum[w];
    total += sm.wsum[w];
  }
  // np.random.choice: the first position whose cumulative probability exceeds u
  const double target = u * total;
  int pick = 0x7fffffff, last = -1;
  if (local > 0.0 && target < excl + local) {
    double run = excl;
    long long higher = ties_after + rties;
    bool done = false;
    for (int b = i0; b < i1 && !done; b += kSmpBatch) {
      unsigned k[kSmpBatch];
      double m[kSmpBatch];
      load(b, k, m, true);
#pragma unroll
      for (int j = 0; j < kSmpBatch; ++j) {
        if (done || b + j >= i1) continue;
        const bool tie = ntie && k[j] == pkey;
        if (tie) --higher;
        if (!(k[j] >= pkey && (!tie || higher < ntie)) || m[j] == 0.0) continue;
        last = b + j;
        run += m[j];
        if (run > target) { pick = b + j; done = true; }
      }
    }
    if (pick == 0x7fffffff && excl <= target) pick = last;   // rounding inside the range
  }
  if (excl <= target || local > 0.0) atomicMin(&sm.token, pick);
  __syncthreads();
  if (sm.token == 0x7fffffff) {                      // target at the very end: the highest kept position
    int hi = -1;
    long long higher = ties_after + rties;
    for (int b = i0; b < i1; b += kSmpBatch) {
      unsigned k[kSmpBatch];
      double m[kSmpBatch];
      load(b, k, m, true);
#pragma unroll
      for (int j = 0; j < kSmpBatch; ++j) {
        if (b + j >= i1) break;
        const bool tie = ntie && k[j] == pkey;
        if (tie) --higher;
        if (k[j] >= pkey && (!tie || higher < ntie) && m[j] > 0.0) hi = b + j;
      }
    }
    atomicMax(&sm.last, hi);
    __syncthreads();
    if (t == 0) sm.token = sm.last < 0 ? 0 : sm.last;
  }
  __syncthreads();
  const int p = sm.token;
  return p >= 0 && p < A.n ? A.index(p) : 0;
}

// The key bytes every window logit shares: their prefix, its mask, and the first radix pass below them.
__device__ void smp_common_prefix(const SmpCand& A, SampleSmem& sm, unsigned& prefix, unsigned& mask, int& top) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  unsigned mn = 0xffffffffu, mx = 0u;
#pragma unroll 8
  for (int i = t; i < A.n; i += kSampleThreads) {
    mn = min(mn, A.k[i]);
    mx = max(mx, A.k[i]);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    mn = min(mn, (unsigned)__shfl_xor((int)mn, m, 64));
    mx = max(mx, (unsigned)__shfl_xor((int)mx, m, 64));
  }
  __syncthreads();
  if (lane == 0) { sm.wmax[wave] = mx; sm.wmin[wave] = mn; }
  __syncthreads();
  for (int w = 0; w < kSampleWaves; ++w) {
    mn = min(mn, sm.wmin[w]);
    mx = max(mx, sm.wmax[w]);
  }
  const unsigned diff = mn ^ mx;
  const int nbytes = diff == 0u ? 4 : __clz(diff) / 8;
  mask = nbytes == 0 ? 0u : nbytes == 4 ? 0xffffffffu : ~(0xffffffffu >> (8 * nbytes));
  prefix = mx & mask;
  top = 24 - 8 * nbytes;
}

// The draw over the window's n logits A (in LDS, or in the workspace above the LDS cap), in index
// order.  A top-k cut (mode 1) runs the whole selection over the window; top-p alone (mode 2) runs
// the radix select over the edge bin's logits with the mass of the bins above it, then the two-level
// draw with each chunk's kept mass (its bins above the edge plus its kept window logits).
__device__ __forceinline__ int smp_pick_window(const SmpCand& A, const float* logits, const SmpWs& w,
                                               const SmpWin& win, int V, int nb, double temp, double lgmax,
                                               double top_p, long long top_k, double u, double Z_all,
                                               SampleSmem& sm) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, n = A.n;
  unsigned cp, cm;
  int ctop;
  smp_common_prefix(A, sm, cp, cm, ctop);
  if (win.mode == 1) return smp_select_draw(A, V, temp, lgmax, top_p, top_k, u, Z_all, cp, cm, ctop, sm);
  if (t == 0) {
    sm.prefix = cp;
    sm.mask = cm;
    sm.above = win.above;
    sm.target = top_p * Z_all;
  }
  __syncthreads();
  if (n <= kSmpWaveSel) {
    if (wave == 0) radix_select_wave<false>(A, 0u, sm, ctop);
    __syncthreads();
  } else {
    radix_select<false>(A, 0u, sm, ctop);
  }
  const unsigned pkey = sm.prefix;
  const double q = exp((double)key_logit(pkey) / temp - lgmax);
  const double need = sm.target - sm.above;
  long long ntie = need > 0.0 ? (long long)ceil(need / q) : 1;
  if (ntie < 1) ntie = 1;
  // ties at pkey are window logits; the kept ones are the ntie of highest index
  const int per = (n + kSampleThreads - 1) / kSampleThreads;
  const int i0 = min(n, t * per), i1 = min(n, i0 + per);
  int nt = 0;
  for (int b = i0; b < i1; b += kSmpBatch) {
    unsigned k[kSmpBatch];
#pragma unroll
    for (int j = 0; j < kSmpBatch; ++j) k[j] = A.k[b + j < i1 ? b + j : i1 - 1];
#pragma unroll
    for (int j = 0; j < kSmpBatch; ++j) nt += b + j < i1 && k[j] == pkey;
  }
  const int inc = wave_incl_scan(nt);
  if (lane == 63) sm.wmax[wave] = (unsigned)inc;
  if (t == 0) sm.tie_cut = -1;
  __syncthreads();
  int ex = inc - nt, tot = 0;
  for (int ww = 0; ww < kSampleWaves; ++ww) {
    if (ww < wave) ex += (int)sm.wmax[ww];
    tot += (int)sm.wmax[ww];
  }
  const long long skip = (long long)tot - ntie;     // ties below the kept ones
  if (skip > 0 && ex <= skip && skip < ex + nt) {
    int r = ex;
    for (int i = i0; i < i1; ++i)
      if (A.k[i] == pkey && r++ == skip) { sm.tie_cut = A.idx[i]; break; }
  }
  __syncthreads();
  const int tie_cut = sm.tie_cut;
  auto kept = [&](int i, unsigned k) { return k > pkey || (k == pkey && i >= tie_cut); };
  // per-chunk kept mass, the chunk's window logits added in index order
  for (int c = t; c < nb; c += kSampleThreads) {
    double m = win.lo < 255 ? w.smass[(size_t)c * 256 + win.lo + 1] : 0.0;
    const int a = (int)w.coff[c], b = (int)w.coff[c + 1];
    for (int b0 = a; b0 < b; b0 += kSmpBatch) {
      unsigned k[kSmpBatch];
      int ix[kSmpBatch];
      double e[kSmpBatch];
#pragma unroll
      for (int j = 0; j < kSmpBatch; ++j) {
        const int i = b0 + j < b ? b0 + j : b - 1;
        k[j] = A.k[i];
        ix[j] = A.idx[i];
        e[j] = A.e[i];
      }
#pragma unroll
      for (int j = 0; j < kSmpBatch; ++j)
        if (b0 + j < b && kept(ix[j], k[j])) m += e[j];
    }
    sm.km[c] = m;
  }
  __syncthreads();
  return smp_chunk_draw(logits, w.e, V, nb, u, [&](int c) { return sm.km[c]; }, kept, sm);
}

__global__ __launch_bounds__(kSampleThreads) void sample_kernel(
    const float* __restrict__ logits, int V, const double* __restrict__ params, const double* __restrict__ uniforms,
    const int* __restrict__ step, int* __restrict__ forced, int* __restrict__ n_forced, int* __restrict__ out,
    double* __restrict__ ws) {
  __shared__ SampleSmem sm;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const double temp = params[0], top_p = params[1];
  const long long top_k = (long long)params[2];
  const int s = step ? step[0] : 0;
  const double u = uniforms[s];
  int tok = 0;
  if (!(temp > 0.0)) {
    // greedy: the lowest index holding the largest key, like np.argmax
    unsigned mk = 0;
#pragma unroll 8
    for (int i = t; i < V; i += kSampleThreads) mk = max(mk, logit_key(logits[i]));
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) mk = max(mk, (unsigned)__shfl_xor((int)mk, m, 64));
    if (lane == 0) sm.wmax[wave] = mk;
    if (t == 0) sm.token = 0x7fffffff;
    __syncthreads();
    mk = sm.wmax[0];
    for (int w = 1; w < kSampleWaves; ++w) mk = max(mk, sm.wmax[w]);
    for (int i = t; i < V; i += kSampleThreads)
      if (logit_key(logits[i]) == mk) { atomicMin(&sm.token, i); break; }
    __syncthreads();
    tok = sm.token;
  } else {
    const SmpWs w = smp_ws(ws, V);
    const int nb = (int)smp_nb(V);
    const SmpHdr hdr = *w.hdr;                       // the largest key, the mass and the window (gather)
    const double lgmax = (double)key_logit(hdr.maxkey) / temp;
    const double Z_all = hdr.Z_all;
    const SmpWin win = hdr.win;
    if (win.mode == 0) {
      tok = smp_chunk_draw(logits, w.e, V, nb, u, [&](int c) { return w.bsum[c]; },
                           [](int, unsigned) { return true; }, sm);
    } else if (!smp_use_window(win, nb)) {
      SmpAll A{logits, w.e, V};
      tok = smp_select_draw(A, V, temp, lgmax, top_p, top_k, u, Z_all, 0u, 0u, 24, sm);
    } else {
      const int n = (int)win.ncand;
      if (n <= kSmpCap) {                            // the window into LDS
        for (int b0 = 0; b0 < n; b0 += 4 * kSampleThreads) {
          unsigned kk[4];
          int ii[4];
          double ee[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int i = b0 + j * kSampleThreads + t < n ? b0 + j * kSampleThreads + t : n - 1;
            kk[j] = w.ckey[i];
            ii[j] = w.cidx[i];
            ee[j] = w.ce[i];
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int i = b0 + j * kSampleThreads + t;
            if (i >= n) continue;
            sm.ckey[i] = kk[j];
            sm.cidx[i] = ii[j];
            sm.ce[i] = ee[j];
          }
        }
        __syncthreads();
        tok = smp_pick_window(SmpCand{sm.ckey, sm.cidx, sm.ce, n}, logits, w, win, V, nb, temp, lgmax, top_p,
                              top_k, u, Z_all, sm);
      } else {                                       // a larger window is read where gather left it
        tok = smp_pick_window(SmpCand{w.ckey, w.cidx, w.ce, n}, logits, w, win, V, nb, temp, lgmax, top_p, top_k,
                              u, Z_all, sm);
      }
    }
  }
  if (t == 0) {
    if (tok < 0 || tok >= V) tok = 0;
    if (forced) forced[s] = tok;
    if (n_forced) n_forced[0] = s + 1;
    if (out) out[0] = tok;
  }
}
}  // namespace afx

using namespace afx;

extern "C" {

int afx_rmsnorm(const void* x, int ldx, const void* gamma, float eps, void* y, int ldy, int M, int D, void* stream) {
  AFX_REQUIRE(x && gamma && y && M >= 1 && D >= 1, "afx_rmsnorm: bad arguments");
  const bool vec = D % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 && D <= 8192 && (((uintptr_t)x | (uintptr_t)y |
                   (uintptr_t)gamma) & 15) == 0;
  if (vec) {
    const int nv = (D / 8 + 255) / 256;
    auto fn = nv <= 1 ? rmsnorm_vec_kernel<1> : nv <= 2 ? rmsnorm_vec_kernel<2> : rmsnorm_vec_kernel<4>;
    hipLaunchKernelGGL(fn, dim3(M), dim3(256), 0, (hipStream_t)stream, (const half_t*)x, ldx, (const half_t*)gamma,
                       eps, (half_t*)y, ldy, D);
    return check_launch("afx_rmsnorm");
  }
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(M), dim3(256), 0, (hipStream_t)stream, (const half_t*)x, ldx,
                     (const half_t*)gamma, eps, (half_t*)y, ldy, D);
  return check_launch("afx_rmsnorm");
}

int afx_rope(const void* x, void* y, int rows, int dh, const void* cos_tab, const void* sin_tab,
             const int* pos_dev, int pos0, int rows_per_pos, void* stream) {
  AFX_REQUIRE(x && y && cos_tab && sin_tab && dh % 2 == 0 && rows >= 1 && rows_per_pos >= 1,
              "afx_rope: bad arguments");
  const long long n = (long long)rows * (dh / 2);
  hipLaunchKernelGGL(rope_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const half_t*)x, (half_t*)y, rows, dh, (const half_t*)cos_tab, (const half_t*)sin_tab,
                     pos_dev, pos0, rows_per_pos);
  return check_launch("afx_rope");
}

int afx_head_norm_rope(void* x, long long seq_stride, long long head_stride, int pos_mul, const int* pos,
                       int kv_len, int heads, int M, int dh, const void* gamma, float eps, const void* cos_tab,
                       const void* sin_tab, int rope, void* stream) {
  AFX_REQUIRE(x && gamma && dh >= 2 && dh <= 256 && dh % 2 == 0 && heads >= 1 && M >= 1,
              "afx_head_norm_rope: bad arguments (dh=%d)", dh);
  AFX_REQUIRE(!rope || (cos_tab && sin_tab && pos), "afx_head_norm_rope: rope needs tables and positions");
  hipLaunchKernelGGL(head_norm_rope_kernel, dim3(heads, M), dim3(64), 0, (hipStream_t)stream, (half_t*)x,
                     seq_stride, head_stride, pos_mul, pos, kv_len, dh, (const half_t*)gamma, eps,
                     (const half_t*)cos_tab, (const half_t*)sin_tab, rope);
  return check_launch("afx_head_norm_rope");
}

int afx_embed(const void* table, const int* ids, void* out, int M, int D, int vocab, void* stream) {
  AFX_REQUIRE(table && ids && out && D % 8 == 0, "afx_embed: D must be a multiple of 8");
  hipLaunchKernelGGL(embed_kernel, dim3(M), dim3(256), 0, (hipStream_t)stream, (const half_t*)table, ids,
                     (half_t*)out, D, vocab);
  return check_launch("afx_embed");
}

int afx_decode_advance(const float* logits, const float* slots, int V, const float* tie_margin, const void* hn,
                       const void* head16, const float* head32, const int* forced, const int* n_forced, int* tok,
                       int* pos, int* hist, int hist_cap, int* step, const void* embed, void* h, int D, int vocab,
                       void* stream) {
  AFX_REQUIRE(tok && pos && step && (logits || slots || forced), "afx_decode_advance: bad arguments");
  AFX_REQUIRE(!(logits || slots) || V >= 1, "afx_decode_advance: V must be positive");
  AFX_REQUIRE(!embed || (h && D % 8 == 0 && vocab >= 1), "afx_decode_advance: embed gather needs h, D %% 8 == 0");
  AFX_REQUIRE(logits || slots || n_forced, "afx_decode_advance: a forced-only step needs n_forced");
  AFX_REQUIRE(!slots || ((uintptr_t)slots & 15) == 0, "afx_decode_advance: slots must be 16-byte aligned");
  AFX_REQUIRE(!tie_margin || (logits && hn && (head16 || head32) && D >= 1),
              "afx_decode_advance: the tie margin needs the logits, the head's input row and its weights");
  AdvanceArgs a = {};
  a.logits = logits; a.slots = (const float4*)slots; a.V = V; a.margin = tie_margin;
  a.hn = (const half_t*)hn; a.head16 = (const half_t*)head16; a.head32 = head32;
  a.forced = forced; a.n_forced = n_forced; a.tok = tok; a.pos = pos; a.hist = hist; a.hist_cap = hist_cap;
  a.step = step; a.embed = (const half_t*)embed; a.h = (half_t*)h; a.D = D; a.vocab = vocab > 0 ? vocab : V;
  hipLaunchKernelGGL(decode_advance_kernel, dim3(1), dim3(kAdvThreads), 0, (hipStream_t)stream, a);
  return check_launch("afx_decode_advance");
}

// Workspace bytes afx_sample needs for V logits.
long long afx_sample_ws_bytes(int V) { return V >= 1 && smp_nb(V) <= kSmpMaxChunks ? smp_ws_bytes(V) : -1; }

// params: device {temperature, top_p, top_k} as doubles; u = uniforms[*step] (uniforms[0] without
// step).  The token goes to forced[*step] (and n_forced = *step + 1, so afx_decode_advance takes
// it) and/or out[0].  ws: afx_sample_ws_bytes(V) bytes.
int afx_sample(const float* logits, int V, const double* params, const double* uniforms, const int* step,
               int* forced, int* n_forced, int* out, double* ws, long long ws_bytes, void* stream) {
  AFX_REQUIRE(logits && params && uniforms && ws && V >= 1, "afx_sample: bad arguments");
  AFX_REQUIRE(smp_nb(V) <= kSmpMaxChunks, "afx_sample: V = %d exceeds %d", V, kSmpMaxChunks * kSmpChunk);
  AFX_REQUIRE(forced || out, "afx_sample: no output");
  AFX_REQUIRE(((uintptr_t)ws & 7) == 0, "afx_sample: the workspace must be 8-byte aligned");
  AFX_REQUIRE(ws_bytes >= smp_ws_bytes(V), "afx_sample: workspace %lld B < %lld B (afx_sample_ws_bytes)", ws_bytes,
              smp_ws_bytes(V));
  hipLaunchKernelGGL(sample_max_kernel, dim3((unsigned)smp_nb(V)), dim3(kSmpPrepThreads), 0, (hipStream_t)stream,
                     logits, V, params, ws);
  hipLaunchKernelGGL(sample_prep_kernel, dim3((unsigned)smp_nb(V)), dim3(kSmpPrepThreads), 0, (hipStream_t)stream,
                     logits, V, params, ws);
  hipLaunchKernelGGL(sample_gather_kernel, dim3((unsigned)smp_nb(V)), dim3(kSmpPrepThreads), 0,
                     (hipStream_t)stream, logits, V, params, ws);
  hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(kSampleThreads), 0, (hipStream_t)stream, logits, V, params,
                     uniforms, step, forced, n_forced, out, ws);
  return check_launch("afx_sample");
}

int afx_argmax(const float* x, int M, int V, int* out, void* stream) {
  AFX_REQUIRE(x && out && M >= 1 && V >= 1, "afx_argmax: bad arguments");
  hipLaunchKernelGGL(argmax_kernel, dim3(M), dim3(256), 0, (hipStream_t)stream, x, V, out);
  return check_launch("afx_argmax");
}

int afx_fill_i32(int* p, int n, int v, void* stream) {
  AFX_REQUIRE(p && n >= 0, "afx_fill_i32: bad arguments");
  if (n == 0) return 0;
  hipLaunchKernelGGL(fill_i32_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, (hipStream_t)stream, p, n, v);
  return check_launch("afx_fill_i32");
}

int afx_fill_f16(void* p, long long n, float v, void* stream) {
  AFX_REQUIRE(p && n >= 0, "afx_fill_f16: bad arguments");
  if (n == 0) return 0;
  hipLaunchKernelGGL(fill_f16_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, (hipStream_t)stream,
                     (half_t*)p, n, v);
  return check_launch("afx_fill_f16");
}

int afx_ew_binary(int op, const void* a, const long long* sa, const void* b, const long long* sb, void* y,
                  int rank, const int* dim, void* stream) {
  Shape5 s;
  if (make_shape(s, rank, dim, sa, sb)) return -1;
  AFX_REQUIRE(a && b && y && op >= 0 && op <= EW_NE, "afx_ew_binary: bad arguments");
  hipLaunchKernelGGL(ew_binary_kernel, dim3(blocks_for(s.n, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const half_t*)a, (const half_t*)b, (half_t*)y, s, op);
  return check_launch("afx_ew_binary");
}

int afx_ew_select(const void* c, const long long* sc, const void* a, const long long* sa, const void* b,
                  const long long* sb, void* y, int rank, const int* dim, void* stream) {
  Shape5 s, s2;
  if (make_shape(s, rank, dim, sc, sa)) return -1;
  if (make_shape(s2, rank, dim, sb, nullptr)) return -1;
  AFX_REQUIRE(c && a && b && y, "afx_ew_select: null pointer");
  hipLaunchKernelGGL(ew_select_kernel, dim3(blocks_for(s.n, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const half_t*)c, (const half_t*)a, (const half_t*)b, (half_t*)y, s, s2);
  return check_launch("afx_ew_select");
}

int afx_ew_unary(int op, const void* x, void* y, long long n, float alpha, float beta, void* stream) {
  AFX_REQUIRE(x && y && n >= 0 && op >= 0 && op <= UN_INVERSE, "afx_ew_unary: bad arguments");
  if (n == 0) return 0;
  hipLaunchKernelGGL(ew_unary_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const half_t*)x, (half_t*)y, n, op, alpha, beta);
  return check_launch("afx_ew_unary");
}

// dst element i (row-major over dim) = src[sum c_d * ss[d]] written at sum c_d * sd[d].
int afx_copy_strided(const void* src, const long long* ss, void* dst, const long long* sd, int rank,
                     const int* dim, void* stream) {
  Shape5 s;
  if (make_shape(s, rank, dim, ss, sd)) return -1;
  AFX_REQUIRE(src && dst, "afx_copy_strided: null pointer");
  hipLaunchKernelGGL(copy_strided_kernel, dim3(blocks_for(s.n, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const half_t*)src, (half_t*)dst, s);
  return check_launch("afx_copy_strided");
}

int afx_softmax(const void* x, void* y, int rows, int cols, void* stream) {
  AFX_REQUIRE(x && y && rows >= 1 && cols >= 1, "afx_softmax: bad arguments");
  hipLaunchKernelGGL(softmax_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, (const half_t*)x,
                     (half_t*)y, cols);
  return check_launch("afx_softmax");
}

int afx_reduce(int op, const void* x, void* y, int rows, int cols, void* stream) {
  AFX_REQUIRE(x && y && rows >= 1 && cols >= 1 && op >= 0 && op <= RED_SUMSQ, "afx_reduce: bad arguments");
  hipLaunchKernelGGL(reduce_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, (const half_t*)x,
                     (half_t*)y, cols, op);
  return check_launch("afx_reduce");
}

int afx_bmm_f16(const void* A, const void* B, void* C, int batch, int M, int N, int K, long long sa, long long sb,
                long long sc, void* stream) {
  AFX_REQUIRE(A && B && C && batch >= 1 && M >= 1 && N >= 1 && K >= 1, "afx_bmm_f16: bad arguments");
  hipLaunchKernelGGL(bmm_kernel, dim3((N + 15) / 16, (M + 15) / 16, batch), dim3(256), 0, (hipStream_t)stream,
                     (const half_t*)A, (const half_t*)B, (half_t*)C, M, N, K, sa, sb, sc);
  return check_launch("afx_bmm_f16");
}

}  // extern "C"
