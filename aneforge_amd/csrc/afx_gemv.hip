// C-ABI entry points of the weight-streaming GEMV (kernel and formats: afx_gemv_impl.h).
// Host-side validation happens here, before any launch, so a bad call returns an error code
// instead of reaching a kernel with extents it does not expect.
#include <stdlib.h>
#include "afx_gemv_impl.h"
#include "afx_mfma.h"

namespace afx {

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

static int mtile(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

// Activation rows from which a linear runs on MFMA (AFX_MFMA_MIN_M overrides; 0 disables).
static int g_mfma_min = -1;
// Fast path without a norm: 2 (default) stages x through LDS once per workgroup, so the four
// wavefronts share one read of it; 0 (AFX_GEMV_XSTAGE=0) has every lane read its x chunks from
// global memory, which costs L1 bandwidth the weight stream needs (x is twice the int8 row).
static int xstage_mode() {
  static int mode = -1;
  if (mode < 0) {
    const char* e = getenv("AFX_GEMV_XSTAGE");
    mode = e && atoi(e) == 0 ? 0 : 2;
  }
  return mode;
}

static int mfma_min_rows() {
  if (g_mfma_min < 0) {
    const char* e = getenv("AFX_MFMA_MIN_M");
    const int v = e ? atoi(e) : -1;
    g_mfma_min = v == 0 ? 1 << 30 : v > 0 ? v : 4;
  }
  return g_mfma_min;
}

// Rows per group: 2 when the epilogue pairs rows (SwiGLU, RoPE), else 1 (a hint of 2 or the
// AFX_GEMV_R environment variable selects row pairs for plain epilogues too).
// Rows per wavefront: paired epilogues need 2; a RMSNorm prologue is paid once per workgroup,
// so it takes 2 (half the workgroups); otherwise 1 (measured on MI355X for the 7B shapes).
static int choose_rows(int hint, bool paired, bool norm) {
  if (paired) return 2;
  int R = hint;
  if (R != 1 && R != 2) {
    const char* e = getenv("AFX_GEMV_R");
    R = e ? atoi(e) : (norm ? 2 : 1);
  }
  return R == 2 ? 2 : 1;
}

// Grid: one row group per wavefront, four wavefronts per workgroup.
static int grid_for(int ngroups) { return (ngroups + 3) / 4; }

static int launch(int fmt, GemvArgs& a, int eg, int rows_hint, hipStream_t stream, const char* what) {
  AFX_REQUIRE(a.w && a.x && a.y, "%s: null pointer argument", what);
  AFX_REQUIRE(a.M >= 1, "%s: M=%d must be >= 1", what, a.M);
  AFX_REQUIRE(a.N >= 1 && a.K >= 1, "%s: bad shape N=%d K=%d", what, a.N, a.K);
  const int kq = fmt == FMT_I8 ? 16 : fmt == FMT_Q4 ? 128 : fmt == FMT_BW ? 64 : fmt == FMT_L4 ? 32
               : fmt == FMT_Q4K || fmt == FMT_Q6K ? 256 : 8;
  AFX_REQUIRE(a.K % kq == 0, "%s: K=%d must be a multiple of %d", what, a.K, kq);
  AFX_REQUIRE(a.ldx % 8 == 0 && a.ldx >= a.K, "%s: ldx=%d must be a multiple of 8 and >= K", what, a.ldx);
  AFX_REQUIRE(((uintptr_t)a.x & 15) == 0 && ((uintptr_t)a.w & 15) == 0,
              "%s: x and weights must be 16-byte aligned", what);
  AFX_REQUIRE(!a.gamma || ((uintptr_t)a.gamma & 15) == 0, "%s: gamma must be 16-byte aligned", what);
  AFX_REQUIRE(fmt != FMT_I8 || a.scale, "%s: int8 weights need a scale vector", what);
  AFX_REQUIRE(fmt != FMT_L4 || (a.scale && ((uintptr_t)a.scale & 15) == 0),
              "%s: int4 weights need 16-byte aligned codebooks [N][16]", what);
  AFX_REQUIRE(fmt != FMT_BW || (a.scale && ((uintptr_t)a.scale & 3) == 0),
              "%s: blockwise weights need a 4-byte aligned block-scale array", what);
  AFX_REQUIRE(fmt != FMT_Q4 || (a.scale && ((uintptr_t)a.scale & 7) == 0),
              "%s: Q4_0 weights need an 8-byte aligned block-scale array", what);
  AFX_REQUIRE(fmt != FMT_Q4K || (a.scale && ((uintptr_t)a.scale & 3) == 0),
              "%s: Q4_K weights need a 4-byte aligned super-block header array", what);
  AFX_REQUIRE(fmt != FMT_Q6K || (a.scale && ((uintptr_t)a.scale & 3) == 0),
              "%s: Q6_K weights need a 4-byte aligned side-word array", what);
  if (eg == EG_SWIGLU) AFX_REQUIRE(a.N % 2 == 0, "%s: SwiGLU needs interleaved gate/up rows", what);
  if (a.epi == EPI_RESID) AFX_REQUIRE(a.resid, "%s: residual pointer required", what);
  if (eg == EG_QKV)
    AFX_REQUIRE(a.dh >= 2 && a.dh % 2 == 0 && a.nq % a.dh == 0 && a.nk % a.dh == 0 && a.pos && a.kcache &&
                    a.vcache,
                "%s: bad fused-QKV arguments", what);
  // 4+ activation rows without a norm prologue: the dot products go to MFMA (any row count, in
  // groups of 16); the vector kernels below take at most 8 rows
  if (a.M >= mfma_min_rows() && eg != EG_QKV && !a.gamma && mfma_supported(fmt, a.K) && a.N % 4 == 0) {
    MfmaArgs m = {};
    m.w = a.w; m.scale = a.scale; m.x = a.x; m.ldx = a.ldx; m.y = a.y; m.ldy = a.ldy;
    m.bias = a.bias; m.resid = a.resid; m.M = a.M; m.N = a.N; m.K = a.K; m.epi = a.epi;
    m.ws = a.ws; m.ws_bytes = a.ws_bytes;
    return mfma_launch(fmt, m, 1, stream, what);
  }
  // the vector kernels take up to 8 rows a launch; with a norm prologue, as many as fit the 64 KB of
  // LDS that stage the normalised rows (8 rows up to K = 3633, 4 to 6547, 2 to 10917, 1 to 16380)
  int mmax = 8;
  while (a.gamma && mmax > 1 && gemv_lds_bytes(mmax, a.K, true) > 65536) mmax >>= 1;
  if (a.M > mmax) {
    const size_t ysz = a.epi == EPI_F32 ? 4 : 2;
    for (int r0 = 0; r0 < a.M; r0 += mmax) {
      GemvArgs c = a;
      c.M = a.M - r0 < mmax ? a.M - r0 : mmax;
      c.x = a.x + (size_t)r0 * a.ldx;
      c.y = (unsigned char*)a.y + (size_t)r0 * a.ldy * ysz;
      if (a.resid) c.resid = a.resid + (size_t)r0 * a.ldy;
      if (eg == EG_QKV) {
        c.pos = a.pos + r0;
        c.kcache = a.kcache + (size_t)r0 * a.kv_seq_stride;
        c.vcache = a.vcache + (size_t)r0 * a.kv_seq_stride;
      }
      const int rc = launch(fmt, c, eg, rows_hint, stream, what);   // c.M <= mmax: no further split
      if (rc) return rc;
    }
    return 0;
  }
  const int mt = mtile(a.M);
  const bool norm = a.gamma != nullptr;
  const int R = choose_rows(rows_hint, eg != EG_PLAIN, norm);
  size_t smem = gemv_lds_bytes(mt, a.K, norm);
  int xs = 1;
  if (smem > 65536) {
    AFX_REQUIRE(!norm, "%s: M*K=%d too large for the LDS norm prologue", what, a.M * a.K);
    xs = 0;
    smem = 0;
  }
  AFX_REQUIRE((long long)a.K * (fmt == FMT_F16 ? 2 : 1) < (1LL << 31), "%s: K=%d too large", what, a.K);
  const int ntiles = grid_for((a.N + R - 1) / R);
  const int nchunks = a.K / (fmt == FMT_I8 || fmt == FMT_BW ? 16
                             : fmt == FMT_Q4 || fmt == FMT_L4 || fmt == FMT_Q4K || fmt == FMT_Q6K ? 32 : 8);
  const int fu = a.M == 1 ? fast_units(fmt, nchunks) : 0;
  if (fu) {
    // a whole row fits the lanes' registers: the register-resident fast path (static LDS only)
    const int nm = norm ? 1 : xstage_mode();     // 2: x staged through LDS once per workgroup
    gemv_fn fr = fmt == FMT_I8 ? pick_gemv_row_i8(eg, R, nm, fu)
               : fmt == FMT_Q4 ? pick_gemv_row_q4(eg, R, nm, fu)
               : fmt == FMT_BW ? pick_gemv_row_bw(eg, R, nm, fu)
               : fmt == FMT_L4 ? pick_gemv_row_l4(eg, R, nm, fu)
               : fmt == FMT_Q4K ? pick_gemv_row_q4k(eg, R, nm, fu)
               : fmt == FMT_Q6K ? pick_gemv_row_q6k(eg, R, nm, fu)
                               : pick_gemv_row_f16(eg, R, nm, fu);
    hipLaunchKernelGGL(fr, dim3(ntiles), dim3(256), 0, stream, a);
    return check_launch(what);
  }
  gemv_fn fn = fmt == FMT_I8 ? pick_gemv_i8(mt, eg, R, xs)
             : fmt == FMT_Q4 ? pick_gemv_q4(mt, eg, R, xs)
             : fmt == FMT_BW ? pick_gemv_bw(mt, eg, R, xs)
             : fmt == FMT_L4 ? pick_gemv_l4(mt, eg, R, xs)
             : fmt == FMT_Q4K ? pick_gemv_q4k(mt, eg, R, xs)
             : fmt == FMT_Q6K ? pick_gemv_q6k(mt, eg, R, xs)
                             : pick_gemv_f16(mt, eg, R, xs);
  hipLaunchKernelGGL(fn, dim3(ntiles), dim3(256), smem, stream, a);
  return check_launch(what);
}

// Greedy-pick summaries of logits rows [8s, 8s + 8) for slot s (the lm_head's generic path; the
// fused head kernel writes the same slots from its workgroups of 8 rows).
__global__ __launch_bounds__(256) void head_slots_kernel(const float* __restrict__ y, int N, float4* __restrict__ slots) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s * 8 >= N) return;
  float4 acc = float4{-INFINITY, __int_as_float(0x7fffffff), -INFINITY, 0.0f};
  for (int r = s * 8; r < s * 8 + 8 && r < N; ++r) {
    const float v = y[r];
    acc = top2_merge(acc, float4{v, __int_as_float(r), -INFINITY, fabsf(v)});
  }
  slots[s] = acc;
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

// fmt: 0 = int8 per-row scale, 1 = Q4_0 superblock, 2 = fp16, 3 = int8 with an fp16 scale per
// 32-weight block (compress="blockwise"; K a multiple of 64), 4 = 4-bit indices into a 16-entry fp16
// codebook per row, scale[N][16] (compress="int4"; K a multiple of 32).
// out_f32: 0 -> y fp16, 1 -> y fp32.  residual (fp16 [M][ldy], may alias y) adds in place.
int afx_linear(int fmt, const void* w, const void* scale, const void* x, int ldx, void* y, int ldy,
               int M, int N, int K, const void* bias, const void* residual, int out_f32,
               int rows_hint, void* ws, long long ws_bytes, void* stream) {
  AFX_REQUIRE(fmt >= 0 && fmt <= 6, "afx_linear: unknown weight format %d", fmt);
  AFX_REQUIRE(!(residual && out_f32), "afx_linear: residual add needs an fp16 output");
  AFX_REQUIRE(ldy >= N, "afx_linear: ldy=%d < N=%d", ldy, N);
  GemvArgs a = base_args(w, scale, x, ldx, y, ldy, M, N, K, bias,
                         residual ? EPI_RESID : out_f32 ? EPI_F32 : EPI_F16);
  a.resid = (const half_t*)residual;
  a.ws = (float*)ws; a.ws_bytes = ws ? ws_bytes : 0;
  return launch(fmt, a, EG_PLAIN, rows_hint, (hipStream_t)stream, "afx_linear");
}

// RMSNorm(x) fused into the GEMV prologue: y = rms_norm(x, gamma, eps) @ W^T (+bias).
int afx_linear_rms(int fmt, const void* w, const void* scale, const void* x, int ldx, const void* gamma,
                   float eps, void* y, int ldy, int M, int N, int K, const void* bias, int out_f32,
                   int rows_hint, void* stream) {
  AFX_REQUIRE(fmt >= 0 && fmt <= 6, "afx_linear_rms: unknown weight format %d", fmt);
  AFX_REQUIRE(gamma, "afx_linear_rms: RMSNorm prologue needs gamma");
  AFX_REQUIRE(ldy >= N, "afx_linear_rms: ldy=%d < N=%d", ldy, N);
  GemvArgs a = base_args(w, scale, x, ldx, y, ldy, M, N, K, bias, out_f32 ? EPI_F32 : EPI_F16);
  a.gamma = (const half_t*)gamma; a.eps = eps;
  return launch(fmt, a, EG_PLAIN, rows_hint, (hipStream_t)stream, "afx_linear_rms");
}

// The lm_head (aneforge/llm.py:338-404) for one hidden row: logits[N] (fp32) = rms_norm(x, gamma, eps)
// @ W^T, plus slots[ceil(N/8)] greedy-pick summaries of the logits (rows 8s .. 8s + 7 each) and,
// when hn_out is given, the fp16 normalised row the products used.
int afx_lm_head(int fmt, const void* w, const void* scale, const void* x, const void* gamma, float eps,
                float* logits, int N, int K, float* slots, void* hn_out, void* stream) {
  AFX_REQUIRE(fmt == FMT_F16, "afx_lm_head: the head streams fp16 weights (fmt 2), got fmt %d", fmt);
  AFX_REQUIRE(gamma && slots && logits, "afx_lm_head: needs gamma, logits and slots");
  AFX_REQUIRE(((uintptr_t)slots & 15) == 0 && (!hn_out || ((uintptr_t)hn_out & 15) == 0),
              "afx_lm_head: slots and hn_out must be 16-byte aligned");
  GemvArgs a = base_args(w, scale, x, K, logits, N, 1, N, K, nullptr, EPI_F32);
  a.gamma = (const half_t*)gamma; a.eps = eps;
  a.slots = slots; a.hn_out = (half_t*)hn_out;
  const int fu = K % 8 == 0 ? fast_units(fmt, K / 8) : 0;
  if (fu) {
    // the fused kernel: 4 wavefronts of 2 rows per workgroup, one slot per workgroup
    AFX_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)gamma & 15) == 0,
                "afx_lm_head: x, gamma and weights must be 16-byte aligned");
    gemv_fn fr = pick_gemv_row_f16(EG_HEAD, 2, 1, fu);
    AFX_REQUIRE(fr, "afx_lm_head: no fused kernel for K=%d", K);
    hipLaunchKernelGGL(fr, dim3(grid_for((N + 1) / 2)), dim3(256), 0, (hipStream_t)stream, a);
    return check_launch("afx_lm_head");
  }
  const int rc = launch(fmt, a, EG_PLAIN, 0, (hipStream_t)stream, "afx_lm_head");
  if (rc) return rc;
  const int ns = (N + 7) / 8;
  hipLaunchKernelGGL(head_slots_kernel, dim3((ns + 255) / 256), dim3(256), 0, (hipStream_t)stream, logits, N,
                     (float4*)slots);
  return check_launch("afx_lm_head(slots)");
}

// SwiGLU MLP front half: act[m][i] = silu(g_i) * u_i with (g, u) = rms_norm(x) @ Wgu^T, where
// Wgu interleaves gate row i and up row i as rows 2i, 2i+1 (N = 2*F).  norm=0 skips the norm.
int afx_linear_swiglu(int fmt, const void* w, const void* scale, const void* x, int ldx, const void* gamma,
                      float eps, int norm, void* act, int ld_act, int M, int N, int K, int rows_hint,
                      void* stream) {
  AFX_REQUIRE(fmt >= 0 && fmt <= 6, "afx_linear_swiglu: unknown weight format %d", fmt);
  AFX_REQUIRE(!norm || gamma, "afx_linear_swiglu: RMSNorm prologue needs gamma");
  AFX_REQUIRE(ld_act >= N / 2, "afx_linear_swiglu: ld_act=%d < N/2=%d", ld_act, N / 2);
  GemvArgs a = base_args(w, scale, x, ldx, act, ld_act, M, N, K, nullptr, EPI_SWIGLU);
  a.gamma = norm ? (const half_t*)gamma : nullptr; a.eps = eps;
  return launch(fmt, a, EG_SWIGLU, rows_hint, (hipStream_t)stream, "afx_linear_swiglu");
}

// GeGLU MLP front half (Gemma, aneforge/llm.py:185-196): act[m][i] = gelu_tanh(g_i) * u_i, otherwise
// exactly afx_linear_swiglu (same arguments, kernels and row interleaving).
int afx_linear_geglu(int fmt, const void* w, const void* scale, const void* x, int ldx, const void* gamma,
                     float eps, int norm, void* act, int ld_act, int M, int N, int K, int rows_hint,
                     void* stream) {
  AFX_REQUIRE(fmt >= 0 && fmt <= 6, "afx_linear_geglu: unknown weight format %d", fmt);
  AFX_REQUIRE(!norm || gamma, "afx_linear_geglu: RMSNorm prologue needs gamma");
  AFX_REQUIRE(ld_act >= N / 2, "afx_linear_geglu: ld_act=%d < N/2=%d", ld_act, N / 2);
  GemvArgs a = base_args(w, scale, x, ldx, act, ld_act, M, N, K, nullptr, EPI_GEGLU);
  a.gamma = norm ? (const half_t*)gamma : nullptr; a.eps = eps;
  return launch(fmt, a, EG_SWIGLU, rows_hint, (hipStream_t)stream, "afx_linear_geglu");
}

// Fused attention input projection for decode: [q|k|v] = rms_norm(h) @ Wqkv^T (+bias), RoPE on
// q and k (rows interleaved per head as (d, d+dh/2)), q -> qout[M][nq], k/v -> the caches at
// row pos[m]:  cache[m*seq_stride + kvh*head_stride + pos*dh + d]; pos outside [0, kv_len) is skipped.
// The rope tables must hold kv_len rows of dh entries.
int afx_qkv_rope_kv(int fmt, const void* w, const void* scale, const void* h, int ldh, const void* gamma,
                    float eps, int norm, const void* bias, int nq, int nk, int nv, int dh,
                    const void* cos_tab, const void* sin_tab, int rope, const int* pos, void* qout,
                    int ldq, void* kcache, void* vcache, long long kv_seq_stride,
                    long long kv_head_stride, int kv_len, int M, int K, int rows_hint, void* stream) {
  AFX_REQUIRE(fmt >= 0 && fmt <= 6, "afx_qkv_rope_kv: unknown weight format %d", fmt);
  AFX_REQUIRE(nv == nk, "afx_qkv_rope_kv: k and v row counts differ (%d vs %d)", nk, nv);
  AFX_REQUIRE(!rope || (cos_tab && sin_tab), "afx_qkv_rope_kv: rope tables required");
  AFX_REQUIRE(!norm || gamma, "afx_qkv_rope_kv: RMSNorm prologue needs gamma");
  AFX_REQUIRE(ldq >= nq, "afx_qkv_rope_kv: ldq=%d < nq=%d", ldq, nq);
  GemvArgs a = base_args(w, scale, h, ldh, qout, ldq, M, nq + nk + nv, K, bias, EPI_QKV);
  a.gamma = norm ? (const half_t*)gamma : nullptr; a.eps = eps;
  a.nq = nq; a.nk = nk; a.dh = dh; a.rope = rope;
  a.cos_tab = (const half_t*)cos_tab; a.sin_tab = (const half_t*)sin_tab; a.pos = pos;
  a.kcache = (half_t*)kcache; a.vcache = (half_t*)vcache;
  a.kv_seq_stride = kv_seq_stride; a.kv_head_stride = kv_head_stride; a.kv_len = kv_len;
  AFX_REQUIRE(kv_len >= 1 && kv_head_stride >= (long long)kv_len * dh, "afx_qkv_rope_kv: bad cache geometry");
  return launch(fmt, a, EG_QKV, rows_hint, (hipStream_t)stream, "afx_qkv_rope_kv");
}

}  // extern "C"
