// Weight-streaming GEMV / skinny GEMM (M <= 8 activation rows) for the quantized decode path.
//
//   y[m, n] = sum_k x[m, k] * W^[n, k]        (fp32 accumulation)
//
// Weight formats (the reference's `compress=` encodings, aneforge/_compile.py:112-188, and
// the GGUF Q4_0 codes that aneforge/_gguf.py:34-39 dequantizes on the host):
//   FMT_I8  : int8 codes [N, K] row-major + fp16 per-output-row scale s[N]
//             (constexpr_affine_dequantize(axis=0), aneforge/_compile.py:171-179): W^ = q*s[n]
//   FMT_Q4  : Q4_0 blocks of 32 along K, one fp16 scale d per block, repacked into the
//             "superblock" layout (afx_q4_0_repack): W^ = (nibble-8)*d[n, k/32]
//   FMT_F16 : plain fp16 [N, K] (lm_head, router)
//
// Work decomposition (HBM-bound, ~1 flop/byte): a 256-thread workgroup = 4 wavefronts; each
// wavefront owns R consecutive output rows and its 64 lanes split K into 16-byte chunks, so
// every load instruction of a wavefront reads 1 KiB of contiguous weight bytes.  All U*R
// chunk loads of an unrolled step are issued before any math, giving 16-64 KiB in flight
// per CU.  Codes are unpacked in registers to exact fp16 pairs and consumed by
// v_dot2_f32_f16; the R row partials are reduced across lanes with a transposed butterfly.
//
// Optional RMSNorm prologue (aneforge/graph.py:293-301, textbook form of the reference's
// numpy oracles, tests/test_moe.py:26): the workgroup normalises x into LDS once
// (xn = fp16(x * rsqrt(mean(x^2) + eps) * gamma)) and the wavefronts read xn from LDS.
//
// Epilogues (runtime-selected, run once per output row):
//   EPI_F16    y = fp16(acc*s + bias)
//   EPI_RESID  y = fp16(resid + fp16(acc*s + bias))              (x + a.linear(W), llm.py:237)
//   EPI_F32    y = acc*s + bias  as fp32                          (logits)
//   EPI_SWIGLU rows interleaved (gate_i, up_i): act[i] = fp16(silu(g16) * u16)  (llm.py:171-175)
//   EPI_QKV    fused q|k|v rows; q and k rows are interleaved per head as (d, d+dh/2) pairs so
//              RoPE (llm.py:96-105) is applied in registers; k and v are written straight into
//              the resident cache at row pos (replaces the masked O(M) rewrite, llm.py:233).
#include <stdlib.h>
#include "afx_gemv_core.h"

namespace afx {

enum { EPI_F16 = 0, EPI_RESID = 1, EPI_F32 = 2, EPI_SWIGLU = 3, EPI_QKV = 4 };

struct GemvArgs {
  const void* w;          // weights (format above)
  const half_t* scale;    // I8: s[N]; Q4: d[N][K/32]; F16: unused
  const half_t* x;        // activations [M][ldx] (the raw input when the norm prologue is on)
  const half_t* gamma;    // RMSNorm weight [K] (prologue only)
  const half_t* bias;     // [N] or null
  const half_t* resid;    // [M][ldy] or null (EPI_RESID)
  void* y;                // output
  const half_t* cos_tab;  // EPI_QKV: rope tables [Mmax][dh] fp16
  const half_t* sin_tab;
  const int* pos;         // EPI_QKV: per-sequence position [M] (device)
  half_t* kcache;         // EPI_QKV: [M][KVH][Mmax][dh]
  half_t* vcache;
  long long kv_seq_stride;   // elements between sequences in the cache
  long long kv_head_stride;  // elements between kv heads (= Mmax*dh)
  int kv_len;             // EPI_QKV: cache rows (Mmax); rows at pos >= kv_len are not written
  int ldx, ldy;
  int M, N, K;
  int epi;
  float eps;
  int nq, nk;             // EPI_QKV: number of q rows (H*dh) and k rows (KVH*dh); v rows follow
  int dh, rope;           // EPI_QKV: head dim; rope on/off
};

// ---- RMSNorm prologue: xn[m][k] = fp16(x * rsqrt(mean(x^2)+eps) * gamma) into LDS ----
template <int M>
__device__ void rms_prologue(const GemvArgs& a, half_t* xn, float* red) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int K = a.K, nv = K >> 3;
  for (int m = 0; m < M; ++m) {
    const int mm = m < a.M ? m : a.M - 1;
    const half_t* xr = a.x + (size_t)mm * a.ldx;
    float ss = 0.0f;
    for (int v = t; v < nv; v += 256) {
      h2 xv[4];
      load_x<1>(xr + 8 * v, xv);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a0 = (float)xv[i].x, a1 = (float)xv[i].y;
        ss = __builtin_fmaf(a0, a0, ss);
        ss = __builtin_fmaf(a1, a1, ss);
      }
    }
    ss = wave_sum(ss);
    if (lane == 0) red[m * 4 + wave] = ss;
  }
  __syncthreads();
  for (int m = 0; m < M; ++m) {
    const int mm = m < a.M ? m : a.M - 1;
    const half_t* xr = a.x + (size_t)mm * a.ldx;
    const float tot = red[m * 4 + 0] + red[m * 4 + 1] + red[m * 4 + 2] + red[m * 4 + 3];
    const float rstd = 1.0f / __builtin_sqrtf(tot / (float)K + a.eps);
    for (int v = t; v < nv; v += 256) {
      h2 xv[4], gv[4];
      load_x<1>(xr + 8 * v, xv);
      load_x<1>(a.gamma + 8 * v, gv);
      u4 o;
      uint32_t* op = (uint32_t*)&o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h2 r;
        r.x = (half_t)(((float)xv[i].x * rstd) * (float)gv[i].x);
        r.y = (half_t)(((float)xv[i].y * rstd) * (float)gv[i].y);
        op[i] = as_u32(r);
      }
      *(u4*)(xn + (size_t)m * K + 8 * v) = o;
    }
  }
  __syncthreads();
}

__device__ __forceinline__ float row_scale(const GemvArgs& a, int fmt, int row) {
  return fmt == FMT_I8 ? (float)a.scale[row] : 1.0f;
}

// Copy the activations into LDS once per workgroup (the wavefronts re-read them per row tile).
template <int M>
__device__ void stage_x(const GemvArgs& a, half_t* xs) {
  const int nv = a.K >> 3;
  for (int m = 0; m < M; ++m) {
    const half_t* xr = a.x + (size_t)(m < a.M ? m : a.M - 1) * a.ldx;
    for (int v = threadIdx.x; v < nv; v += 256) *(u4*)(xs + (size_t)m * a.K + 8 * v) = *(const u4*)(xr + 8 * v);
  }
  __syncthreads();
}

// Row-tile epilogue: reduce the wavefront's R row partials and apply the selected epilogue.
template <int FMT, int M, int R>
__device__ __forceinline__ void gemv_epilogue(const GemvArgs& a, float (&acc)[M][R], int row0, int lane) {
  const int N = a.N;
  const int rr = reduced_row_of_lane<R>(lane);
  const int row = row0 + rr;
  constexpr int GROUP = 64 / R;          // lanes holding the same row
  const bool writer = (lane & (GROUP - 1)) == 0;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const float sum = wave_reduce_rows<R>(acc[m], lane);
    const bool live = m < a.M;
    const int rs = row < N ? row : 0;
    const float v = (row < N) ? sum * row_scale(a, FMT, rs) + (a.bias ? (float)a.bias[rs] : 0.0f) : 0.0f;
    switch (a.epi) {
      case EPI_F16:
        if (writer && live && row < N) ((half_t*)a.y)[(size_t)m * a.ldy + row] = (half_t)v;
        break;
      case EPI_RESID:
        if (writer && live && row < N) {
          const half_t o16 = (half_t)v;
          const float r = (float)a.resid[(size_t)m * a.ldy + row];
          ((half_t*)a.y)[(size_t)m * a.ldy + row] = (half_t)(r + (float)o16);
        }
        break;
      case EPI_F32:
        if (writer && live && row < N) ((float*)a.y)[(size_t)m * a.ldy + row] = v;
        break;
      case EPI_SWIGLU: {
        // rows come in (gate, up) pairs; the partner row lives GROUP lanes away
        const float other = shfl_xor(v, GROUP);
        if (writer && live && row < N && (row & 1) == 0) {
          const float g16 = (float)(half_t)v, u16 = (float)(half_t)other;
          ((half_t*)a.y)[(size_t)m * a.ldy + (row >> 1)] = (half_t)(silu(g16) * u16);
        }
        break;
      }
      case EPI_QKV: {
        const float other = shfl_xor(v, GROUP);
        const int p = live ? a.pos[m] : -1;          // pos has a.M entries; padded rows store nothing
        if (writer && live && row < N && p >= 0 && p < a.kv_len) {
          const int dh = a.dh, half = dh >> 1;
          const float self16 = (float)(half_t)v, other16 = (float)(half_t)other;
          if (row < a.nq + a.nk) {
            const bool isk = row >= a.nq;
            const int rl = isk ? row - a.nq : row;
            const int head = rl / dh, j = rl - head * dh;      // j: packed index within head
            const int i = j >> 1;
            const bool hi = j & 1;
            const int dim = hi ? i + half : i;
            float o = self16;
            if (a.rope) {
              const float c = (float)a.cos_tab[(size_t)p * dh + dim];
              const float s = (float)a.sin_tab[(size_t)p * dh + dim];
              o = hi ? self16 * c + other16 * s : self16 * c - other16 * s;
            }
            if (isk) {
              a.kcache[(size_t)m * a.kv_seq_stride + (size_t)head * a.kv_head_stride +
                       (size_t)p * dh + dim] = (half_t)o;
            } else {
              ((half_t*)a.y)[(size_t)m * a.ldy + head * dh + dim] = (half_t)o;
            }
          } else {
            const int rl = row - a.nq - a.nk;
            const int head = rl / dh, dim = rl - head * dh;
            a.vcache[(size_t)m * a.kv_seq_stride + (size_t)head * a.kv_head_stride +
                     (size_t)p * dh + dim] = (half_t)self16;
          }
        }
        break;
      }
      default:
        break;
    }
  }
}

// Chunks per lane per pipeline unit (each lane has U*R 16-byte loads in flight per unit).
template <int FMT, int M, int R>
struct Units {
  static constexpr int value = FMT == FMT_Q4 ? 2 : 4;
};

// Persistent, software-pipelined GEMV.  A row tile is 4 wavefronts x R rows; workgroups
// stride over tiles.  Each wavefront walks (tile, chunk batch) units and keeps two register
// buffers: the next unit's weight loads are in flight while the current unit is computed.
// The first unit is requested before the x prologue (LDS staging or RMSNorm), so the
// prologue's latency overlaps the first weight fetch.
//   XS: 0 = x read from global memory, 1 = x staged in LDS, 2 = RMSNorm(x) into LDS.
template <int FMT, int M, int R, int XS>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int U = Units<FMT, M, R>::value;
  constexpr int XH = Fmt<FMT>::kXH2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int K = a.K, N = a.N;
  const int nchunks = K / Fmt<FMT>::kWeightsPerChunk;
  const int ntiles = (N + 4 * R - 1) / (4 * R);
  const size_t rb = Fmt<FMT>::row_bytes(K);
  const unsigned char* wbase = (const unsigned char*)a.w;

  auto tile_live = [&](int t) { return t < ntiles && (t * 4 + wave) * R < N; };
  auto load_unit = [&](u4 (&w)[U][R], u2 (&d)[U][R], int t, int c0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int row = (t * 4 + wave) * R + r;
      row = row < N ? row : N - 1;                       // tail rows: computed, never stored
      const unsigned char* wr = wbase + (size_t)row * rb;
      const half_t* dr = FMT == FMT_Q4 ? a.scale + (size_t)row * (K >> 5) : nullptr;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int c = c0 + 64 * u + lane;
        c = c < nchunks ? c : nchunks - 1;
        w[u][r] = __builtin_nontemporal_load((const u4*)(wr + (size_t)c * 16));
        d[u][r] = load_scales<FMT>(dr, c);
      }
    }
  };

  int t0 = blockIdx.x;
  const bool live = tile_live(t0);
  u4 wA[U][R], wB[U][R];
  u2 dA[U][R], dB[U][R];
  if (live) load_unit(wA, dA, t0, 0);

  const half_t* xbase = a.x;
  int ldx = a.ldx;
  if constexpr (XS != 0) {
    half_t* xs = (half_t*)smem;
    if constexpr (XS == 2) rms_prologue<M>(a, xs, (float*)(smem + (size_t)M * K * sizeof(half_t)));
    else stage_x<M>(a, xs);
    xbase = xs;
    ldx = K;
  }
  if (!live) return;   // no barrier follows

  const half_t* xp[M];
#pragma unroll
  for (int m = 0; m < M; ++m) xp[m] = xbase + (size_t)(m < a.M ? m : a.M - 1) * ldx;

  float acc[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

  auto compute = [&](const u4 (&w)[U][R], const u2 (&d)[U][R], int c0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 64 * u + lane;
      if (c < nchunks) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
          h2 xv[XH];
          Fmt<FMT>::load_x(xp[m], c, xv);
#pragma unroll
          for (int r = 0; r < R; ++r) acc[m][r] = Fmt<FMT>::dot(w[u][r], xv, d[u][r], acc[m][r]);
        }
      }
    }
  };
  auto finish_tile = [&](int t) {
    gemv_epilogue<FMT, M, R>(a, acc, (t * 4 + wave) * R, lane);
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;
  };

  int c0 = 0;
  const int step = 64 * U;
  for (;;) {
    int t1 = t0, c1 = c0 + step;
    if (c1 >= nchunks) { c1 = 0; t1 = t0 + gridDim.x; }
    bool nxt = tile_live(t1);
    if (nxt) load_unit(wB, dB, t1, c1);
    compute(wA, dA, c0);
    if (c1 == 0) finish_tile(t0);
    if (!nxt) break;
    t0 = t1; c0 = c1;

    t1 = t0; c1 = c0 + step;
    if (c1 >= nchunks) { c1 = 0; t1 = t0 + gridDim.x; }
    nxt = tile_live(t1);
    if (nxt) load_unit(wA, dA, t1, c1);
    compute(wB, dB, c0);
    if (c1 == 0) finish_tile(t0);
    if (!nxt) break;
    t0 = t1; c0 = c1;
  }
}

// ---------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------
typedef void (*gemv_fn)(GemvArgs);

template <int FMT, int M, int R>
static gemv_fn pick_xs(int xs) {
  return xs == 2 ? gemv_kernel<FMT, M, R, 2> : xs == 1 ? gemv_kernel<FMT, M, R, 1> : gemv_kernel<FMT, M, R, 0>;
}
template <int FMT, int M>
static gemv_fn pick_r(int R, int xs) {
  return R >= 4 ? pick_xs<FMT, M, 4>(xs) : pick_xs<FMT, M, 2>(xs);
}
template <int FMT>
static gemv_fn pick_m(int M, int R, int xs) {
  if (M <= 1) return pick_r<FMT, 1>(R, xs);
  if (M <= 2) return pick_r<FMT, 2>(R, xs);
  if (M <= 4) return pick_r<FMT, 4>(R, xs);
  return pick_r<FMT, 8>(R, xs);
}
static int mtile(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

static int g_cu_count = 0;
static int cu_count() {
  if (g_cu_count == 0) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    hipDeviceProp_t p;
    g_cu_count = (hipGetDeviceProperties(&p, dev) == hipSuccess) ? p.multiProcessorCount : 256;
  }
  return g_cu_count;
}

// Workgroups resident per CU the persistent grid is sized for (register-limited occupancy
// of the two-buffer pipeline is about 2 workgroups of 4 wavefronts per CU).
static int g_wg_per_cu = 0;
static int wg_per_cu() {
  if (g_wg_per_cu == 0) {
    const char* e = getenv("AFX_GEMV_WG_PER_CU");
    const int v = e ? atoi(e) : 0;
    g_wg_per_cu = v >= 1 && v <= 16 ? v : 2;
  }
  return g_wg_per_cu;
}

static int launch(int fmt, GemvArgs& a, bool norm, int rows_hint, hipStream_t stream, const char* what) {
  AFX_REQUIRE(a.w && a.x && a.y, "%s: null pointer argument", what);
  AFX_REQUIRE(a.M >= 1 && a.M <= 8, "%s: M=%d must be in [1, 8]", what, a.M);
  AFX_REQUIRE(a.N >= 1 && a.K >= 1, "%s: bad shape N=%d K=%d", what, a.N, a.K);
  const int kq = fmt == FMT_I8 ? 16 : fmt == FMT_Q4 ? 128 : 8;
  AFX_REQUIRE(a.K % kq == 0, "%s: K=%d must be a multiple of %d", what, a.K, kq);
  AFX_REQUIRE(a.ldx % 8 == 0, "%s: ldx=%d must be a multiple of 8", what, a.ldx);
  AFX_REQUIRE(((uintptr_t)a.x & 15) == 0 && ((uintptr_t)a.w & 15) == 0,
              "%s: x and weights must be 16-byte aligned", what);
  AFX_REQUIRE(fmt != FMT_I8 || a.scale, "%s: int8 weights need a scale vector", what);
  AFX_REQUIRE(fmt != FMT_Q4 || (a.scale && ((uintptr_t)a.scale & 7) == 0),
              "%s: Q4_0 weights need an 8-byte aligned block-scale array", what);
  if (a.epi == EPI_SWIGLU) AFX_REQUIRE(a.N % 2 == 0, "%s: SwiGLU needs interleaved gate/up rows", what);
  if (a.epi == EPI_RESID) AFX_REQUIRE(a.resid, "%s: residual pointer required", what);
  if (a.epi == EPI_QKV)
    AFX_REQUIRE(a.dh % 2 == 0 && a.nq % a.dh == 0 && a.nk % a.dh == 0 && a.pos && a.kcache && a.vcache,
                "%s: bad fused-QKV arguments", what);
  const int mt = mtile(a.M);
  int R = rows_hint == 2 || rows_hint == 4 ? rows_hint : (mt >= 4 ? 2 : 4);
  const size_t xbytes = (size_t)mt * a.K * sizeof(half_t);
  int xs;
  size_t smem = 0;
  if (norm) {
    AFX_REQUIRE(a.gamma, "%s: RMSNorm prologue needs gamma", what);
    smem = xbytes + 8 * 4 * sizeof(float);
    AFX_REQUIRE(smem <= 65536, "%s: M*K=%d too large for the LDS norm prologue", what, a.M * a.K);
    xs = 2;
  } else if (xbytes <= 65536) {
    smem = xbytes;
    xs = 1;
  } else {
    xs = 0;
  }
  gemv_fn fn = fmt == FMT_I8 ? pick_m<FMT_I8>(a.M, R, xs)
             : fmt == FMT_Q4 ? pick_m<FMT_Q4>(a.M, R, xs)
                             : pick_m<FMT_F16>(a.M, R, xs);
  const int ntiles = (a.N + 4 * R - 1) / (4 * R);
  const int cap = cu_count() * wg_per_cu();
  const int grid = ntiles < cap ? ntiles : cap;
  hipLaunchKernelGGL(fn, dim3(grid), dim3(256), smem, stream, a);
  return check_launch(what);
}

static GemvArgs base_args(const void* w, const void* scale, const void* x, int ldx, void* y, int ldy,
                          int M, int N, int K, const void* bias, int epi) {
  GemvArgs a = {};
  a.w = w; a.scale = (const half_t*)scale; a.x = (const half_t*)x; a.ldx = ldx;
  a.y = y; a.ldy = ldy; a.M = M; a.N = N; a.K = K; a.bias = (const half_t*)bias; a.epi = epi;
  return a;
}

}  // namespace afx

using namespace afx;

extern "C" {

// fmt: 0 = int8 per-row scale, 1 = Q4_0 superblock, 2 = fp16.
// out_f32: 0 -> y fp16, 1 -> y fp32.  residual (fp16 [M][ldy], may alias y) adds in place.
int afx_linear(int fmt, const void* w, const void* scale, const void* x, int ldx, void* y, int ldy,
               int M, int N, int K, const void* bias, const void* residual, int out_f32,
               int rows_hint, void* stream) {
  AFX_REQUIRE(fmt >= 0 && fmt <= 2, "afx_linear: unknown weight format %d", fmt);
  AFX_REQUIRE(!(residual && out_f32), "afx_linear: residual add needs an fp16 output");
  GemvArgs a = base_args(w, scale, x, ldx, y, ldy, M, N, K, bias,
                         residual ? EPI_RESID : out_f32 ? EPI_F32 : EPI_F16);
  a.resid = (const half_t*)residual;
  return launch(fmt, a, false, rows_hint, (hipStream_t)stream, "afx_linear");
}

// RMSNorm(x) fused into the GEMV prologue: y = rms_norm(x, gamma, eps) @ W^T (+bias).
int afx_linear_rms(int fmt, const void* w, const void* scale, const void* x, int ldx, const void* gamma,
                   float eps, void* y, int ldy, int M, int N, int K, const void* bias, int out_f32,
                   int rows_hint, void* stream) {
  AFX_REQUIRE(fmt >= 0 && fmt <= 2, "afx_linear_rms: unknown weight format %d", fmt);
  GemvArgs a = base_args(w, scale, x, ldx, y, ldy, M, N, K, bias, out_f32 ? EPI_F32 : EPI_F16);
  a.gamma = (const half_t*)gamma; a.eps = eps;
  return launch(fmt, a, true, rows_hint, (hipStream_t)stream, "afx_linear_rms");
}

// SwiGLU MLP front half: act[m][i] = silu(g_i) * u_i with (g, u) = rms_norm(x) @ Wgu^T, where
// Wgu interleaves gate row i and up row i as rows 2i, 2i+1 (N = 2*F).  norm=0 skips the norm.
int afx_linear_swiglu(int fmt, const void* w, const void* scale, const void* x, int ldx, const void* gamma,
                      float eps, int norm, void* act, int ld_act, int M, int N, int K, int rows_hint,
                      void* stream) {
  AFX_REQUIRE(fmt >= 0 && fmt <= 2, "afx_linear_swiglu: unknown weight format %d", fmt);
  GemvArgs a = base_args(w, scale, x, ldx, act, ld_act, M, N, K, nullptr, EPI_SWIGLU);
  a.gamma = (const half_t*)gamma; a.eps = eps;
  return launch(fmt, a, norm != 0, rows_hint, (hipStream_t)stream, "afx_linear_swiglu");
}

// Fused attention input projection for decode: [q|k|v] = rms_norm(h) @ Wqkv^T (+bias), RoPE on
// q and k (rows interleaved per head as (d, d+dh/2)), q -> qout[M][nq], k/v -> the caches at
// row pos[m]:  cache[m*seq_stride + kvh*head_stride + pos*dh + d]; pos outside [0, kv_len) is skipped.
int afx_qkv_rope_kv(int fmt, const void* w, const void* scale, const void* h, int ldh, const void* gamma,
                    float eps, int norm, const void* bias, int nq, int nk, int nv, int dh,
                    const void* cos_tab, const void* sin_tab, int rope, const int* pos, void* qout,
                    int ldq, void* kcache, void* vcache, long long kv_seq_stride,
                    long long kv_head_stride, int kv_len, int M, int K, int rows_hint, void* stream) {
  AFX_REQUIRE(fmt >= 0 && fmt <= 2, "afx_qkv_rope_kv: unknown weight format %d", fmt);
  AFX_REQUIRE(nv == nk, "afx_qkv_rope_kv: k and v row counts differ (%d vs %d)", nk, nv);
  AFX_REQUIRE(!rope || (cos_tab && sin_tab), "afx_qkv_rope_kv: rope tables required");
  GemvArgs a = base_args(w, scale, h, ldh, qout, ldq, M, nq + nk + nv, K, bias, EPI_QKV);
  a.gamma = (const half_t*)gamma; a.eps = eps;
  a.nq = nq; a.nk = nk; a.dh = dh; a.rope = rope;
  a.cos_tab = (const half_t*)cos_tab; a.sin_tab = (const half_t*)sin_tab; a.pos = pos;
  a.kcache = (half_t*)kcache; a.vcache = (half_t*)vcache;
  a.kv_seq_stride = kv_seq_stride; a.kv_head_stride = kv_head_stride; a.kv_len = kv_len;
  AFX_REQUIRE(kv_len >= 1 && kv_head_stride >= (long long)kv_len * dh, "afx_qkv_rope_kv: bad cache geometry");
  return launch(fmt, a, norm != 0, rows_hint, (hipStream_t)stream, "afx_qkv_rope_kv");
}

}  // extern "C"
