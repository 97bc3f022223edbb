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
// prefill), else argmax(logits) (lowest index on ties, like np.argmax; greedy _sample).  Then
// hist[*step] = token, ++*step, ++*pos, h = embed[token].  One workgroup; every input that
// changes between steps lives in device memory, so the step replays as a captured graph.
__global__ __launch_bounds__(1024) void decode_advance_kernel(
    const float* __restrict__ logits, int V, const int* __restrict__ forced, const int* __restrict__ n_forced,
    int* __restrict__ tok, int* __restrict__ pos, int* __restrict__ hist, int hist_cap, int* __restrict__ step,
    const half_t* __restrict__ embed, half_t* __restrict__ h, int D, int vocab) {
  __shared__ float bv[16];
  __shared__ int bi[16];
  __shared__ int chosen;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int s = step[0];
  const bool use_forced = forced && n_forced && s < n_forced[0];
  if (!use_forced && logits) {
    float best = -INFINITY;
    int besti = 0x7fffffff;
    // batches of 8 float4 per thread, all loads issued before the compares
    const int nv4 = V >> 2;
    const bool al = (((uintptr_t)logits) & 15) == 0;
    for (int b0 = 0; al && b0 < nv4; b0 += 8 * (int)blockDim.x) {
      float4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i4 = b0 + j * (int)blockDim.x + t;
        v[j] = i4 < nv4 ? ((const float4*)logits)[i4] : float4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int base = 4 * (b0 + j * (int)blockDim.x + t);
        const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (e[k] > best || (e[k] == best && base + k < besti)) { best = e[k]; besti = base + k; }
      }
    }
    for (int i = (al ? 4 * nv4 : 0) + t; i < V; i += blockDim.x) {
      const float v = logits[i];
      if (v > best || (v == best && i < besti)) { best = v; besti = i; }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const float ov = __shfl_xor(best, m, 64);
      const int oi = __shfl_xor(besti, m, 64);
      if (ov > best || (ov == best && oi < besti)) { best = ov; besti = oi; }
    }
    if (lane == 0) { bv[wave] = best; bi[wave] = besti; }
  }
  __syncthreads();
  if (t == 0) {
    int bidx;
    if (use_forced) {
      bidx = forced[s];
    } else if (!logits) {
      bidx = 0;                  // a forced-only step run past its prompt: inert token
    } else {
      const int nw = blockDim.x >> 6;
      float b = bv[0];
      bidx = bi[0];
      for (int w = 1; w < nw; ++w)
        if (bv[w] > b || (bv[w] == b && bi[w] < bidx)) { b = bv[w]; bidx = bi[w]; }
      if (bidx >= V) bidx = 0;   // all-NaN logits: deterministic fallback
    }
    bidx = bidx < 0 ? 0 : (bidx >= vocab ? vocab - 1 : bidx);
    chosen = bidx;
    tok[0] = bidx;
    if (s < hist_cap) hist[s] = bidx;
    step[0] = s + 1;
    pos[0] = pos[0] + 1;
  }
  __syncthreads();
  if (embed) {
    const u4* src = (const u4*)(embed + (size_t)chosen * D);
    u4* dst = (u4*)h;
    for (int i = t; i < D / 8; i += blockDim.x) dst[i] = src[i];
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

int afx_decode_advance(const float* logits, int V, const int* forced, const int* n_forced, int* tok, int* pos,
                       int* hist, int hist_cap, int* step, const void* embed, void* h, int D, int vocab,
                       void* stream) {
  AFX_REQUIRE(tok && pos && step && (logits || forced), "afx_decode_advance: bad arguments");
  AFX_REQUIRE(!logits || V >= 1, "afx_decode_advance: V must be positive");
  AFX_REQUIRE(!embed || (h && D % 8 == 0 && vocab >= 1), "afx_decode_advance: embed gather needs h, D % 8 == 0");
  AFX_REQUIRE(logits || n_forced, "afx_decode_advance: a forced-only step needs n_forced");
  hipLaunchKernelGGL(decode_advance_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, logits, V, forced,
                     n_forced, tok, pos, hist, hist_cap, step, (const half_t*)embed, (half_t*)h, D,
                     vocab > 0 ? vocab : V);
  return check_launch("afx_decode_advance");
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
