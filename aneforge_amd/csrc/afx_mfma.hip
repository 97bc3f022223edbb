// MFMA skinny GEMM: Y[t, n] = sum_k X[t, k] * W^[n, k] for up to 16 activation rows ("tokens")
// per token group, with the weights streamed once from HBM in their packed formats.
//
// This is the batched path of the quantized linears (the reference's compress="int8" matmul,
// aneforge/_compile.py:171-179 and 375-385, and the GGUF Q4_0 weights of aneforge/_gguf.py:34-39)
// and of the MoE experts (aneforge/moe.py:40-63, computed only for the experts a token routed
// to).  With 4+ tokens the dot2 path spends more VALU per weight byte than HBM supplies; here
// the dot products run on v_mfma_f32_16x16x32_f16, with the weights as the 16-row A operand:
//   lane l: A row l % 16, k = 8 * (l / 16) .. + 7;  B column (token) l % 16, same k;
//   D rows 4 * (l / 16) .. + 3 of token l % 16.
// A k-permutation shared by A and B is free, so every lane decodes the k values of its own
// 16-byte weight chunk:
//   int8 : a chunk = 16 codes -> two A operands (exact fp16 codes; the row scale is applied to
//          the fp32 result, so the dequantised weight is exactly q * s);
//   Q4_0 : a superblock chunk = 8 codes of each of 4 blocks -> four A operands, each
//          fp16((nibble - 8) * d): the fp16-rounded dequantised weight the reference multiplies
//          with (it converts the ggml dequantisation to float16, aneforge/_gguf.py:34-39);
//   fp16 : a chunk = 8 weights -> one A operand.
// A workgroup owns 16 output rows; its 4 wavefronts split K evenly (each streams a quarter of
// every row, all loads of a step issued before its MFMAs) and their partial 16x16 tiles are
// summed through LDS by wavefront 0, which applies the epilogue.  MoE: the grid's y dimension
// is the expert; workgroups of experts with no tokens exit at once (fixed launch shape, so the
// layer stays graph-capturable).
#include "afx_gemv_impl.h"
#include "afx_mfma.h"

namespace afx {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

template <int FMT> struct MfmaFmt;
template <> struct MfmaFmt<FMT_I8> { static constexpr int kK = 64, kMfma = 2; };    // k per step (64 lanes)
template <> struct MfmaFmt<FMT_Q4> { static constexpr int kK = 128, kMfma = 4; };
template <> struct MfmaFmt<FMT_F16> { static constexpr int kK = 32, kMfma = 1; };

constexpr int kStepsPerBatch = 4;   // steps whose loads are in flight together

__device__ __forceinline__ h8 pack8(h2 a, h2 b, h2 c, h2 d) {
  h8 r;
  r[0] = a.x; r[1] = a.y; r[2] = b.x; r[3] = b.y; r[4] = c.x; r[5] = c.y; r[6] = d.x; r[7] = d.y;
  return r;
}
__device__ __forceinline__ h8 as_h8(u4 v) { return __builtin_bit_cast(h8, v); }

template <int FMT, int EG>
__global__ __launch_bounds__(256) void mfma_kernel(MfmaArgs a) {
  constexpr int KS = MfmaFmt<FMT>::kK, NM = MfmaFmt<FMT>::kMfma;
  __shared__ f4 red[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int e = blockIdx.y;
  const int N = a.N, K = a.K;
  const int n0 = blockIdx.x * 16;
  int ntok = a.M;
  const int* lst = nullptr;
  if (a.cnt) {
    ntok = a.cnt[e];
    if (ntok <= 0) return;                       // whole workgroup: no barrier reached
    lst = a.list + (size_t)e * a.T;
  }
  const unsigned char* wbase = (const unsigned char*)a.w + (size_t)e * a.w_es;
  const half_t* sbase = a.scale ? a.scale + (size_t)e * a.s_es : nullptr;
  const int row = n0 + r < N ? n0 + r : N - 1;   // A row of this lane (tail rows computed, not stored)
  const size_t rowbytes = Fmt<FMT>::row_bytes(K);
  const u4* wrow = (const u4*)(wbase + (size_t)row * rowbytes);
  const half_t* drow = FMT == FMT_Q4 ? sbase + (size_t)row * (K >> 5) : nullptr;
  const int nsteps = K / KS;
  const int s0 = nsteps * wave / 4, s1 = nsteps * (wave + 1) / 4;   // this wavefront's K quarter

  for (int tg = 0; tg < ntok; tg += 16) {
    const int ti = tg + r;                        // B column (token) of this lane
    const bool tok_ok = ti < ntok;
    const int tc = tok_ok ? ti : ntok - 1;
    int xr = tc;
    if (lst) {
      const int ent = lst[tc];
      xr = a.x_by_token ? ent / a.k : ent;
    }
    const half_t* xrow = a.x + (size_t)xr * a.ldx;
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int sb = s0; sb < s1; sb += kStepsPerBatch) {
      u4 wv[kStepsPerBatch];
      u2 dv[kStepsPerBatch];
      u4 xv[kStepsPerBatch][NM];
#pragma unroll
      for (int i = 0; i < kStepsPerBatch; ++i) {
        const int s = sb + i < s1 ? sb + i : s1 - 1;   // a clamped repeat is masked below
        const int c = s * 4 + g;                       // 16-byte chunk of this lane
        wv[i] = __builtin_nontemporal_load(wrow + c);
        if constexpr (FMT == FMT_Q4) dv[i] = *(const u2*)(drow + 4 * s);
#pragma unroll
        for (int j = 0; j < NM; ++j) {
          int kx;
          if constexpr (FMT == FMT_I8) kx = s * KS + 16 * g + 8 * j;
          else if constexpr (FMT == FMT_Q4) kx = 32 * (4 * s + j) + 8 * g;
          else kx = s * KS + 8 * g;
          xv[i][j] = *(const u4*)(xrow + kx);
        }
      }
#pragma unroll
      for (int i = 0; i < kStepsPerBatch; ++i) {
        if (sb + i >= s1) break;                       // wavefront-uniform
#pragma unroll
        for (int j = 0; j < NM; ++j) {
          h8 av;
          if constexpr (FMT == FMT_I8) {
            h2 q0, q1, q2, q3;
            i8x4_to_h2(j == 0 ? wv[i].x : wv[i].z, q0, q1);
            i8x4_to_h2(j == 0 ? wv[i].y : wv[i].w, q2, q3);
            av = pack8(q0, q1, q2, q3);
          } else if constexpr (FMT == FMT_Q4) {
            const uint32_t wd = j == 0 ? wv[i].x : j == 1 ? wv[i].y : j == 2 ? wv[i].z : wv[i].w;
            const h2 dd = as_h2(j < 2 ? dv[i].x : dv[i].y);
            const half_t d = (j & 1) ? dd.y : dd.x;
            const h2 d2 = {d, d};
            h2 q[4];
            q4_word_to_h2(wd, q);
            av = pack8(q[0] * d2, q[1] * d2, q[2] * d2, q[3] * d2);   // fp16((nibble - 8) * d)
          } else {
            av = as_h8(wv[i]);
          }
          h8 bv = as_h8(xv[i][j]);
          if (!tok_ok) bv = (h8){0, 0, 0, 0, 0, 0, 0, 0};
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
        }
      }
    }
    // sum the four K quarters; wavefront 0 finishes the tile
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
      const f4 p1 = red[1][lane], p2 = red[2][lane], p3 = red[3][lane];
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = acc[i] + p1[i] + p2[i] + p3[i];
      const int rb = n0 + 4 * g;                   // output rows rb .. rb + 3 of token ti
      if constexpr (FMT == FMT_I8) {
        const u2 sv = *(const u2*)(sbase + (rb < N ? rb : 0));
        const h2 s01 = as_h2(sv.x), s23 = as_h2(sv.y);
        v[0] *= (float)s01.x; v[1] *= (float)s01.y; v[2] *= (float)s23.x; v[3] *= (float)s23.y;
      }
      if (a.bias) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] += rb + i < N ? (float)a.bias[rb + i] : 0.0f;
      }
      if (tok_ok && rb < N) {
        const int yr = lst ? lst[ti] : ti;          // entry (MoE) or activation row (dense)
        if constexpr (EG == EG_SWIGLU) {
          half_t* yp = (half_t*)a.y + (size_t)yr * a.ldy + (rb >> 1);
          const float g0 = (float)(half_t)v[0], u0 = (float)(half_t)v[1];
          const float g1 = (float)(half_t)v[2], u1 = (float)(half_t)v[3];
          yp[0] = (half_t)(silu(g0) * u0);
          yp[1] = (half_t)(silu(g1) * u1);
        } else if (a.epi == EPI_F32) {
          float* yp = (float*)a.y + (size_t)yr * a.ldy + rb;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (rb + i < N) yp[i] = v[i];
        } else {
          half_t* yp = (half_t*)a.y + (size_t)yr * a.ldy + rb;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (rb + i >= N) break;
            float o = v[i];
            if (a.epi == EPI_RESID) o = (float)a.resid[(size_t)yr * a.ldy + rb + i] + (float)(half_t)o;
            yp[i] = (half_t)o;
          }
        }
      }
    }
    __syncthreads();                               // red is reused by the next token group
  }
}

typedef void (*mfma_fn)(MfmaArgs);

bool mfma_supported(int fmt, int K) {
  const int ks = fmt == FMT_I8 ? 64 : fmt == FMT_Q4 ? 128 : 32;
  return K % ks == 0 && K / ks >= 4;
}

int mfma_launch(int fmt, const MfmaArgs& a, int E, hipStream_t stream, const char* what) {
  AFX_REQUIRE(fmt >= 0 && fmt <= 2, "%s: unknown weight format %d", what, fmt);
  AFX_REQUIRE(a.w && a.x && a.y, "%s: null pointer", what);
  AFX_REQUIRE(a.N >= 1 && a.N % 4 == 0, "%s: N=%d must be a multiple of 4", what, a.N);
  AFX_REQUIRE(mfma_supported(fmt, a.K), "%s: K=%d does not fit the MFMA split", what, a.K);
  AFX_REQUIRE(a.ldx % 8 == 0 && ((uintptr_t)a.x & 15) == 0 && ((uintptr_t)a.w & 15) == 0,
              "%s: x and weights must be 16-byte aligned (ldx %% 8 == 0)", what);
  AFX_REQUIRE(fmt != FMT_I8 || (a.scale && ((uintptr_t)a.scale & 7) == 0), "%s: int8 needs aligned row scales", what);
  AFX_REQUIRE(fmt != FMT_Q4 || (a.scale && ((uintptr_t)a.scale & 7) == 0), "%s: Q4_0 needs aligned block scales", what);
  AFX_REQUIRE(a.cnt ? (a.list && a.T >= 1 && a.k >= 1) : (a.M >= 1), "%s: bad token description", what);
  AFX_REQUIRE(a.epi != EPI_RESID || a.resid, "%s: residual pointer required", what);
  const bool swiglu = a.epi == EPI_SWIGLU;
  mfma_fn fn;
  if (fmt == FMT_I8) fn = swiglu ? mfma_kernel<FMT_I8, EG_SWIGLU> : mfma_kernel<FMT_I8, EG_PLAIN>;
  else if (fmt == FMT_Q4) fn = swiglu ? mfma_kernel<FMT_Q4, EG_SWIGLU> : mfma_kernel<FMT_Q4, EG_PLAIN>;
  else fn = swiglu ? mfma_kernel<FMT_F16, EG_SWIGLU> : mfma_kernel<FMT_F16, EG_PLAIN>;
  hipLaunchKernelGGL(fn, dim3((a.N + 15) / 16, E), dim3(256), 0, stream, a);
  return check_launch(what);
}

}  // namespace afx
