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
//   FMT_L4  : 4-bit indices [N, K/2] (column 2j in the low nibble of byte j) into a 16-entry fp16
//             codebook per row, scale[N, 16] (compress="int4", aneforge/_blob.py:28-43; each row holds
//             its source tensor's codebook): W^ = codebook[n][index]
//   FMT_BW  : int8 codes [N, K] + fp16 scale per 32-weight block s[N, K/32] (compress="blockwise",
//             aneforge/_blob.py:46-56): W^ = fp16(q * s[n, k/32])
//
// Work decomposition.  The kernel is HBM-bound, and at decode sizes (17-90 MB) it only gets
// near the bandwidth floor with many small, independent work items and nothing serialised
// behind the weight stream.  So:
//  * the N rows are cut into groups of R rows (R = 2 when an epilogue pairs rows: SwiGLU
//    gate/up, RoPE partners) and each wavefront takes one group; a persistent grid measured
//    slower at every decode shape on MI355X, because the dispatcher balances many small
//    workgroups better than a static split;
//  * a wavefront walks K in "units" (U 16-byte chunks per lane per row, i.e. U KiB of each
//    row: a whole 4096-wide int8 or Q4 row); the next unit's loads are in flight while the
//    current one is computed (two register buffers);
//  * weight rows are read through buffer descriptors sized to the row, so chunks past K read
//    as zero in hardware (no clamping or masking of weights in the loop);
//  * the small operands of the epilogue (row scale, bias, residual, RoPE table entries) are
//    requested right behind the first weights, with no branch between the loads;
//  * x is staged once per workgroup into LDS (and, with the RMSNorm prologue, normalised there
//    in place from a single global read of x and gamma), before the loop starts;
//  * codes are unpacked in registers to exact fp16 pairs and consumed by v_dot2_f32_f16; each
//    row's 64 lane partials are summed with DPP (row_shr / row_bcast) into a wave-uniform value.
//
// RMSNorm prologue (aneforge/graph.py:293-301, the textbook form of the reference's numpy
// oracles, tests/test_moe.py:26): xn = fp16(x * rsqrt(mean(x^2) + eps) * gamma).
//
// Epilogue groups (template parameter EG, so each group is a distinct kernel symbol):
//   EG_PLAIN   runtime-selected store: EPI_F16  y = fp16(acc*s + bias)
//                                      EPI_RESID y = fp16(resid + fp16(acc*s + bias))  (llm.py:237)
//                                      EPI_F32  y = acc*s + bias as fp32 (logits)
//   EG_SWIGLU  rows interleaved (gate_i, up_i): act[i] = fp16(silu(g16) * u16)   (llm.py:171-175),
//              or fp16(gelu_tanh(g16) * u16) when epi is EPI_GEGLU (Gemma, llm.py:185-196)
//   EG_QKV     fused q|k|v rows; q and k rows are interleaved per head as (d, d+dh/2) pairs so
//              RoPE (llm.py:96-105) is applied to the pair; k and v are written straight into
//              the resident cache at row pos (replaces the masked O(M) rewrite, llm.py:233).
//   EG_HEAD    the lm_head (llm.py:338-404): fp32 logits, and per workgroup one slot with its
//              rows' largest logit, that logit's row (the lowest on ties), the second largest
//              and the largest magnitude, so the greedy pick and its tie margin need no rescan.
#pragma once
#include "afx_gemv_core.h"

namespace afx {

enum { EPI_F16 = 0, EPI_RESID = 1, EPI_F32 = 2, EPI_SWIGLU = 3, EPI_QKV = 4, EPI_GEGLU = 5 };
enum { EG_PLAIN = 0, EG_SWIGLU = 1, EG_QKV = 2, EG_HEAD = 3 };

struct GemvArgs {
  const void* w;          // weights (format above)
  const half_t* scale;    // I8: s[N]; Q4: d[N][K/32]; F16: unused
  const half_t* x;        // activations [M][ldx] (the raw input when the norm prologue is on)
  const half_t* gamma;    // RMSNorm weight [K] (null: no norm)
  const half_t* bias;     // [N] or null
  const half_t* resid;    // [M][ldy] or null (EPI_RESID)
  void* y;                // output
  const half_t* cos_tab;  // EG_QKV: rope tables [kv_len][dh] fp16
  const half_t* sin_tab;
  const int* pos;         // EG_QKV: per-sequence position [M] (device)
  half_t* kcache;         // EG_QKV: [M][KVH][Mmax][dh]
  half_t* vcache;
  long long kv_seq_stride;   // elements between sequences in the cache
  long long kv_head_stride;  // elements between kv heads (= Mmax*dh)
  int kv_len;             // EG_QKV: cache rows (Mmax); rows at pos outside [0, kv_len) are not written
  int ldx, ldy;
  int M, N, K;
  int epi;
  float eps;
  int nq, nk;             // EG_QKV: number of q rows (H*dh) and k rows (KVH*dh); v rows follow
  int dh, rope;           // EG_QKV: head dim; rope on/off
  float* ws;              // MFMA K-split partials (optional workspace, afx_linear)
  long long ws_bytes;
  float* slots;           // EG_HEAD: per workgroup {top-1, its row (int bits), top-2, max |y|}
  half_t* hn_out;         // norm prologue: workgroup 0 also writes the fp16 normalised row here
};

constexpr int kStageUnroll = 4;     // 16-byte staging loads per thread in flight per batch
constexpr int kBufDword3 = 0x00020000;   // raw buffer descriptor word 3 (gfx9 family)

template <int FMT> struct Units {
  static constexpr int value = FMT == FMT_Q4 || FMT == FMT_L4 || FMT == FMT_Q4K || FMT == FMT_Q6K ? 2 : 4;
};

// Bytes of LDS the kernel needs: staged x rows, gamma, and the cross-wave norm partials.
__host__ __device__ inline size_t gemv_lds_bytes(int Mt, int K, bool norm) {
  return (size_t)Mt * K * 2 + (norm ? (size_t)K * 2 + (size_t)Mt * 4 * sizeof(float) : 0);
}

// Sum over the 64 lanes (DPP row shifts, then row broadcasts), returned wave-uniform.
__device__ __forceinline__ float wave_sum_uniform(float v) {
#define AFX_DPP_ADD(ctrl, rmask, bc) \
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, rmask, 0xf, bc))
  AFX_DPP_ADD(0x111, 0xf, true);    // row_shr:1
  AFX_DPP_ADD(0x112, 0xf, true);    // row_shr:2
  AFX_DPP_ADD(0x114, 0xf, true);    // row_shr:4
  AFX_DPP_ADD(0x118, 0xf, true);    // row_shr:8  -> lane 15 of each row holds the row sum
  AFX_DPP_ADD(0x142, 0xa, false);   // row_bcast:15 into rows 1 and 3
  AFX_DPP_ADD(0x143, 0xc, false);   // row_bcast:31 into rows 2 and 3 -> lane 63 holds the total
#undef AFX_DPP_ADD
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, kBufDword3);
}
__device__ __forceinline__ u4 buf_load16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));   // nt: streamed once
}
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ u2 buf_load8(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}

// Store one row group's results (wave-uniform values, called by one lane).
template <int M, int R, int EG>
__device__ __forceinline__ void gemv_store(const GemvArgs& a, const float (&v)[M][R], int row0, const int (&e_pos)[M],
                                           const half_t (&h_res)[M][R], const half_t (&h_cs)[M][R],
                                           const half_t (&h_sn)[M][R]) {
  const int N = a.N;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    if (m >= a.M) break;
    if constexpr (EG == EG_PLAIN) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        if (row >= N) break;
        if (a.epi == EPI_F32) ((float*)a.y)[(size_t)m * a.ldy + row] = v[m][r];
        else if (a.epi == EPI_RESID)
          ((half_t*)a.y)[(size_t)m * a.ldy + row] = (half_t)((float)h_res[m][r] + (float)(half_t)v[m][r]);
        else ((half_t*)a.y)[(size_t)m * a.ldy + row] = (half_t)v[m][r];
      }
    } else if constexpr (EG == EG_SWIGLU) {
      const float g16 = (float)(half_t)v[m][0], u16 = (float)(half_t)v[m][1];
      ((half_t*)a.y)[(size_t)m * a.ldy + (row0 >> 1)] = (half_t)(glu_act(a.epi == EPI_GEGLU, g16) * u16);
    } else {
      const int p = e_pos[m];
      if (p < 0 || p >= a.kv_len) continue;
      const int dh = a.dh;
      const float v0 = (float)(half_t)v[m][0], v1 = (float)(half_t)v[m][1];
      if (row0 < a.nq + a.nk) {
        const bool isk = row0 >= a.nq;
        const int rl = isk ? row0 - a.nq : row0;
        const int head = rl / dh, i = (rl - head * dh) >> 1, half = dh >> 1;
        float o0 = v0, o1 = v1;        // row0 holds dim i, row0 + 1 holds dim i + dh/2
        if (a.rope) {
          o0 = v0 * (float)h_cs[m][0] - v1 * (float)h_sn[m][0];
          o1 = v1 * (float)h_cs[m][1] + v0 * (float)h_sn[m][1];
        }
        half_t* dst = isk ? a.kcache + (size_t)m * a.kv_seq_stride + (size_t)head * a.kv_head_stride +
                                (size_t)p * dh
                          : (half_t*)a.y + (size_t)m * a.ldy + (size_t)head * dh;
        dst[i] = (half_t)o0;
        dst[i + half] = (half_t)o1;
      } else {
        const int rl = row0 - a.nq - a.nk;
        const int head = rl / dh, dim = rl - head * dh;
        half_t* dst = a.vcache + (size_t)m * a.kv_seq_stride + (size_t)head * a.kv_head_stride +
                      (size_t)p * dh + dim;
        dst[0] = (half_t)v0;
        dst[1] = (half_t)v1;
      }
    }
  }
}

// Epilogue operands of a row group: row scales, bias, residual, and for fused QKV the RoPE
// table entries of the pair's two dims.  Unconditional loads from valid addresses (absent
// operands read a dummy element and are masked where used), so they add no branches.
template <int FMT, int M, int R, int EG>
__device__ __forceinline__ void gemv_epilogue_operands(const GemvArgs& a, int row0, const int (&e_pos)[M],
                                                       half_t (&h_scale)[R], half_t (&h_bias)[R],
                                                       half_t (&h_res)[M][R], half_t (&h_cs)[M][R],
                                                       half_t (&h_sn)[M][R]) {
  const half_t* dummy = a.x;
  const int N = a.N;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r < N ? row0 + r : N - 1;
    h_scale[r] = (half_t)1.0f;
    if constexpr (FMT == FMT_I8) h_scale[r] = a.scale[row];
    h_bias[r] = *(a.bias ? a.bias + row : dummy);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      h_res[m][r] = (half_t)0.0f;
      if constexpr (EG == EG_PLAIN)
        h_res[m][r] = *(a.epi == EPI_RESID ? a.resid + (size_t)(m < a.M ? m : 0) * a.ldy + row : dummy);
    }
  }
  if constexpr (EG == EG_QKV) {
    const int dh = a.dh, half = dh >> 1;
    const int rl = row0 >= a.nq ? row0 - a.nq : row0;
    const int i = (rl % dh) >> 1;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int p = e_pos[m] >= 0 && e_pos[m] < a.kv_len ? e_pos[m] : 0;
      const half_t* ct = a.rope ? a.cos_tab + (size_t)p * dh : dummy;
      const half_t* st = a.rope ? a.sin_tab + (size_t)p * dh : dummy;
      const int i0 = a.rope ? i : 0, i1 = a.rope ? i + half : 0;
      h_cs[m][0] = ct[i0]; h_sn[m][0] = st[i0];
      h_cs[m][1] = ct[i1]; h_sn[m][1] = st[i1];
    }
  }
}

template <int FMT, int M, int R, int XS, int EG>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int U = Units<FMT>::value;
  constexpr int XH = Fmt<FMT>::kXH2;
  static_assert(EG == EG_PLAIN || R == 2, "paired epilogues process row pairs");
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int K = a.K, N = a.N;
  const int nchunks = K / Fmt<FMT>::kWeightsPerChunk;
  const int upr = (nchunks + 64 * U - 1) / (64 * U);       // units per row
  const int rowbytes = (int)Fmt<FMT>::row_bytes(K);
  const int ngroups = (N + R - 1) / R;
  const int g = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + wave);   // this wavefront's row group
  const bool live = g < ngroups;
  const int row0 = (live ? g : ngroups - 1) * R;

  // Everything up to the staging stores is straight-line code with unconditional loads
  // (indices clamped; absent operands read from a valid dummy address and masked when used),
  // so the compiler's wait counters stay exact: the staging stores wait only for the
  // activation loads while the weights stream in.

  // ---- 1. per-sequence positions (EG_QKV) ----
  int e_pos[M];
#pragma unroll
  for (int m = 0; m < M; ++m) e_pos[m] = -1;
  if constexpr (EG == EG_QKV) {
#pragma unroll
    for (int m = 0; m < M; ++m) e_pos[m] = a.pos[m < a.M ? m : 0];
  }

  // ---- 2. activations: first staging batch (XS) ----
  half_t* xs = (half_t*)smem;
  const bool norm = XS && a.gamma != nullptr;
  const int nv = K >> 3;                        // 16-byte vectors per row
  const int nstage = (M + (norm ? 1 : 0)) * nv; // x rows, then gamma
  u4 sv[kStageUnroll];
  auto stage_load = [&](int f0) {
#pragma unroll
    for (int i = 0; i < kStageUnroll; ++i) {
      int f = f0 + 256 * i + t;
      f = f < nstage ? f : nstage - 1;
      const int m = f / nv, c = f - m * nv;
      const half_t* src = m < M ? a.x + (size_t)(m < a.M ? m : a.M - 1) * a.ldx + 8 * c : a.gamma + 8 * c;
      sv[i] = *(const u4*)src;
    }
  };
  if constexpr (XS != 0) stage_load(0);
  __builtin_amdgcn_sched_barrier(0);   // keep the activation loads ahead of the weight stream

  // ---- 3. weights: the first two units of the group's rows (a unit past K reads as zero) ----
  __amdgpu_buffer_rsrc_t wr[R], dr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r < N ? row0 + r : N - 1;   // a tail row is computed, never stored
    wr[r] = make_rsrc((const unsigned char*)a.w + (size_t)row * rowbytes, rowbytes);
    if constexpr (has_block_scales<FMT>())
      dr[r] = make_rsrc(a.scale + (size_t)row * scale_row_halves<FMT>(K), 2 * scale_row_halves<FMT>(K));
  }
  u4 wA[U][R], wB[U][R];
  using SW = typename Fmt<FMT>::S;
  SW dA[U][R], dB[U][R];
  auto load_unit = [&](u4 (&w)[U][R], SW (&d)[U][R], int j) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = j * 64 * U + 64 * u + lane;
        w[u][r] = buf_load16(wr[r], c * 16);
        if constexpr (FMT == FMT_Q4) d[u][r] = buf_load8(dr[r], (c >> 2) * 8);
        if constexpr (FMT == FMT_BW) d[u][r] = (u2){buf_load4(dr[r], (c >> 2) * 4), (uint32_t)((c >> 1) & 1)};
        if constexpr (FMT == FMT_Q4K)       // past K both read as zero: d = dmin = 0, weight 0
          d[u][r] = (u2){buf_load4(dr[r], (c >> 3) * 20), buf_load4(dr[r], (c >> 3) * 20 + 4 + 4 * ((c >> 1) & 3))};
        if constexpr (FMT == FMT_Q6K)       // past K all zero: d = 0, weight 0
          d[u][r] = (u4){buf_load4(dr[r], c * 12), buf_load4(dr[r], c * 12 + 4), buf_load4(dr[r], c * 12 + 8), 0u};
      }
    }
  };
  load_unit(wA, dA, 0);
  load_unit(wB, dB, 1);

  // ---- 4. epilogue operands of the group's rows ----
  half_t h_scale[R], h_bias[R], h_res[M][R], h_cs[M][R], h_sn[M][R];
  gemv_epilogue_operands<FMT, M, R, EG>(a, row0, e_pos, h_scale, h_bias, h_res, h_cs, h_sn);
  __builtin_amdgcn_sched_barrier(0);

  // ---- 5. finish staging x (and the norm) in LDS ----
  if constexpr (XS != 0) {
    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) ss[m] = 0.0f;
    auto stage_store = [&](int f0) {
#pragma unroll
      for (int i = 0; i < kStageUnroll; ++i) {
        const int fr = f0 + 256 * i + t;
        const int f = fr < nstage ? fr : nstage - 1;   // a clamped duplicate rewrites its own value
        *(u4*)(xs + (size_t)f * 8) = sv[i];
        const int m = f / nv;
        float q = 0.0f;
        q = dot2(as_h2(sv[i].x), as_h2(sv[i].x), q);
        q = dot2(as_h2(sv[i].y), as_h2(sv[i].y), q);
        q = dot2(as_h2(sv[i].z), as_h2(sv[i].z), q);
        q = dot2(as_h2(sv[i].w), as_h2(sv[i].w), q);
        q = fr < nstage ? q : 0.0f;
#pragma unroll
        for (int mm = 0; mm < M; ++mm) ss[mm] += m == mm ? q : 0.0f;
      }
    };
    // the first batch is straight-line code; longer rows take further batches
    stage_store(0);
    for (int f0 = 256 * kStageUnroll; f0 < nstage; f0 += 256 * kStageUnroll) {
      stage_load(f0);
      stage_store(f0);
    }
    if (norm) {
      float* red = (float*)(smem + (size_t)(M + 1) * K * 2);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float s = wave_sum_uniform(ss[m]);
        if (lane == 0) red[m * 4 + wave] = s;
      }
      __syncthreads();
      const half_t* gs = xs + (size_t)M * K;
      for (int f = t; f < M * nv; f += 256) {
        const int m = f / nv, c = f - m * nv;
        const float tot = red[m * 4 + 0] + red[m * 4 + 1] + red[m * 4 + 2] + red[m * 4 + 3];
        const float rstd = 1.0f / __builtin_sqrtf(tot / (float)K + a.eps);
        u4 xv = *(const u4*)(xs + (size_t)f * 8);
        const u4 gv = *(const u4*)(gs + 8 * c);
        uint32_t* xq = (uint32_t*)&xv;
        const uint32_t* gq = (const uint32_t*)&gv;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const h2 xx = as_h2(xq[jj]), gg = as_h2(gq[jj]);
          h2 r;
          r.x = (half_t)(((float)xx.x * rstd) * (float)gg.x);
          r.y = (half_t)(((float)xx.y * rstd) * (float)gg.y);
          xq[jj] = as_u32(r);
        }
        *(u4*)(xs + (size_t)f * 8) = xv;
        if (a.hn_out && blockIdx.x == 0 && f < nv) *(u4*)(a.hn_out + 8 * f) = xv;
      }
    }
    __syncthreads();
  }
  if (!live) return;   // no barrier follows

  // ---- 6. the K loop: compute one unit while the next is in flight ----
  const half_t* xp[M];
#pragma unroll
  for (int m = 0; m < M; ++m)
    xp[m] = XS ? xs + (size_t)m * K : a.x + (size_t)(m < a.M ? m : a.M - 1) * a.ldx;
  float acc[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;
  typename Fmt<FMT>::Ctx fctx[R];
#pragma unroll
  for (int r = 0; r < R; ++r) fctx[r] = Fmt<FMT>::Ctx::make(a.scale, row0 + r < N ? row0 + r : N - 1);
  auto compute = [&](const u4 (&w)[U][R], const SW (&d)[U][R], int j) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int craw = j * 64 * U + 64 * u + lane;
      const int c = craw < nchunks ? craw : nchunks - 1;   // x of a real chunk; the weights past K read as zero
#pragma unroll
      for (int m = 0; m < M; ++m) {
        h2 xv[XH];
        Fmt<FMT>::load_x(xp[m], c, xv);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float t = Fmt<FMT>::dot(w[u][r], xv, d[u][r], fctx[r], acc[m][r]);
          // LUT4: index 0 of a chunk past K still looks up an entry, so drop that chunk's sum
          acc[m][r] = FMT != FMT_L4 || craw < nchunks ? t : acc[m][r];
        }
      }
    }
  };
  for (int j = 0;;) {
    compute(wA, dA, j);
    if (++j >= upr) break;
    load_unit(wA, dA, j + 1);
    compute(wB, dB, j);
    if (++j >= upr) break;
    load_unit(wB, dB, j + 1);
  }

  // ---- 7. epilogue: DPP row sums (wave-uniform), one lane stores ----
  float v[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r)
      v[m][r] = wave_sum_uniform(acc[m][r]) * (float)h_scale[r] + (a.bias ? (float)h_bias[r] : 0.0f);
  if (lane == 0) gemv_store<M, R, EG>(a, v, row0, e_pos, h_res, h_cs, h_sn);
}

// Fast path for one activation row (M = 1) with K at most 64 lanes x U chunks (U a compile-time
// constant per shape family: int8 K = 4096 -> 4, 11008 -> 11; Q4_0 4096 -> 2, 11008 -> 6;
// fp16 4096 -> 8).  Each lane keeps the x values of its own U chunks in registers.  NORM = 1:
// the workgroup normalises x once (each thread a few 16-byte vectors of x and gamma), shares it
// through LDS, and every lane then reads its chunks; NORM = 2: the same staging without the
// norm; NORM = 0: every lane reads its chunks straight from global memory (no LDS, no
// barrier).  Chunks past K (the last unit of a ragged row) read a clamped address and are
// zeroed by a select.
template <int FMT, int R, int NORM, int EG, int U>
__global__ __launch_bounds__(256) void gemv_row_kernel(GemvArgs a) {
  constexpr int XH = Fmt<FMT>::kXH2;
  constexpr int KMAX = 64 * U * Fmt<FMT>::kWeightsPerChunk;
  constexpr int NVT = (KMAX / 8 + 255) / 256;          // norm vectors per thread
  static_assert(EG == EG_PLAIN || R == 2, "paired epilogues process row pairs");
  static_assert(EG != EG_HEAD || NORM == 1, "the lm_head variant has the norm prologue");
  __shared__ __align__(16) half_t xs[NORM ? KMAX : 8];
  __shared__ float red[4];
  __shared__ float xsum[4];
  // int8 with the norm prologue: the codes enter the dot products as q + 1152 (no subtraction per
  // pair) and each row's sum is corrected by 1152 * sum(x) once; sum(x) comes from the staging
  // pass.  Only there: with one row per wavefront the sum costs about what the subtractions do.
  constexpr bool kBiased = FMT == FMT_I8 && NORM == 1;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int N = a.N, K = a.K;
  const int nchunks = K / Fmt<FMT>::kWeightsPerChunk;
  const int ngroups = (N + R - 1) / R;
  const int g = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + wave);
  const bool live = g < ngroups;
  const int row0 = (live ? g : ngroups - 1) * R;

  int e_pos[1] = {-1};
  if constexpr (EG == EG_QKV) e_pos[0] = a.pos[0];

  // activations first: the lane's own chunks (no norm) or this thread's share of x and gamma
  h2 xv[U][XH];
  u4 xq[NVT], gq[NVT];
  const int nv = K >> 3;
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < NVT; ++i) {
      int f = t + 256 * i;
      f = f < nv ? f : nv - 1;
      xq[i] = *(const u4*)(a.x + 8 * f);
      if constexpr (NORM == 1) gq[i] = *(const u4*)(a.gamma + 8 * f);
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int c = 64 * u + lane;
      c = c < nchunks ? c : nchunks - 1;
      Fmt<FMT>::load_x(a.x, c, xv[u]);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // the group's weight rows, one 16-byte chunk per lane per unit
  u4 w[U][R];
  typename Fmt<FMT>::S d[U][R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r < N ? row0 + r : N - 1;
    const u4* wr = (const u4*)((const unsigned char*)a.w + (size_t)row * Fmt<FMT>::row_bytes(K));
    const half_t* dr = has_block_scales<FMT>() ? a.scale + (size_t)row * scale_row_halves<FMT>(K) : nullptr;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int c = 64 * u + lane;
      c = c < nchunks ? c : nchunks - 1;
      w[u][r] = __builtin_nontemporal_load(wr + c);
      d[u][r] = load_scales<FMT>(dr, c);
    }
  }
  half_t h_scale[R], h_bias[R], h_res[1][R], h_cs[1][R], h_sn[1][R];
  gemv_epilogue_operands<FMT, 1, R, EG>(a, row0, e_pos, h_scale, h_bias, h_res, h_cs, h_sn);
  __builtin_amdgcn_sched_barrier(0);

  if constexpr (NORM == 1) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NVT; ++i) {
      float q = dot2(as_h2(xq[i].x), as_h2(xq[i].x), 0.0f);
      q = dot2(as_h2(xq[i].y), as_h2(xq[i].y), q);
      q = dot2(as_h2(xq[i].z), as_h2(xq[i].z), q);
      q = dot2(as_h2(xq[i].w), as_h2(xq[i].w), q);
      ss += t + 256 * i < nv ? q : 0.0f;
    }
    ss = wave_sum_uniform(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const float rstd = 1.0f / __builtin_sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)K + a.eps);
#pragma unroll
    for (int i = 0; i < NVT; ++i) {
      uint32_t* xw = (uint32_t*)&xq[i];
      const uint32_t* gw = (const uint32_t*)&gq[i];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) xw[jj] = rms_pair(xw[jj], gw[jj], rstd);
    }
    if constexpr (EG == EG_HEAD) {
      if (a.hn_out && blockIdx.x == 0) {
#pragma unroll
        for (int i = 0; i < NVT; ++i)
          if (t + 256 * i < nv) *(u4*)(a.hn_out + 8 * (t + 256 * i)) = xq[i];
      }
    }
  }
  float sx = 0.0f;
  if constexpr (NORM) {
    float xp = 0.0f;
#pragma unroll
    for (int i = 0; i < NVT; ++i) {
      int f = t + 256 * i;
      if constexpr (kBiased) {
        const h2 one = {(half_t)1.0f, (half_t)1.0f};
        float q = dot2(as_h2(xq[i].x), one, 0.0f);
        q = dot2(as_h2(xq[i].y), one, q);
        q = dot2(as_h2(xq[i].z), one, q);
        q = dot2(as_h2(xq[i].w), one, q);
        xp += f < nv ? q : 0.0f;
      }
      f = f < nv ? f : nv - 1;                       // a clamped duplicate rewrites its own value
      *(u4*)(xs + 8 * f) = xq[i];
    }
    if constexpr (kBiased) {
      xp = wave_sum_uniform(xp);
      if (lane == 0) xsum[wave] = xp;
    }
    __syncthreads();
    if constexpr (kBiased) sx = (xsum[0] + xsum[1]) + (xsum[2] + xsum[3]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int c = 64 * u + lane;
      c = c < nchunks ? c : nchunks - 1;
      Fmt<FMT>::load_x(xs, c, xv[u]);
    }
  }
  typename Fmt<FMT>::Ctx fctx[R];
#pragma unroll
  for (int r = 0; r < R; ++r) fctx[r] = Fmt<FMT>::Ctx::make(a.scale, row0 + r < N ? row0 + r : N - 1);
  if (EG != EG_HEAD && !live) return;   // no barrier follows (the head variant meets one below)

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const bool ok = 64 * u + lane < nchunks;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      u4 wv = w[u][r];
      typename Fmt<FMT>::S dv = d[u][r];
      if (u == U - 1) {                              // only the last unit can hold chunks past K
        if constexpr (FMT == FMT_Q4) {
          dv.x = ok ? dv.x : 0u;
          dv.y = ok ? dv.y : 0u;
        } else if constexpr (FMT == FMT_Q4K) {
          dv.x = ok ? dv.x : 0u;                     // d = dmin = 0: weight 0 for any code
        } else if constexpr (FMT == FMT_Q6K) {
          dv.z = ok ? dv.z : 0u;                     // d = 0: weight 0 for any code
        } else if constexpr (FMT != FMT_L4 && !kBiased) {
          wv.x = ok ? wv.x : 0u; wv.y = ok ? wv.y : 0u; wv.z = ok ? wv.z : 0u; wv.w = ok ? wv.w : 0u;
        }
      }
      if constexpr (kBiased) {
        // a chunk past K: its biased codes are not zero, so its x is (clamped duplicates)
        h2 xz[Fmt<FMT>::kXH2];
#pragma unroll
        for (int j = 0; j < Fmt<FMT>::kXH2; ++j) xz[j] = u == U - 1 && !ok ? (h2){(half_t)0.0f, (half_t)0.0f} : xv[u][j];
        acc[r] = Fmt<FMT_I8>::dot_biased(wv, xz, acc[r]);
      } else {
        const float t = Fmt<FMT>::dot(wv, xv[u], dv, fctx[r], acc[r]);
        // LUT4: index 0 still looks up an entry, so a chunk past K drops its whole sum
        acc[r] = FMT == FMT_L4 && u == U - 1 && !ok ? acc[r] : t;
      }
    }
  }

  float v[1][R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float d = wave_sum_uniform(acc[r]);
    if constexpr (kBiased) d -= 1152.0f * sx;
    v[0][r] = d * (float)h_scale[r] + (a.bias ? (float)h_bias[r] : 0.0f);
  }
  if constexpr (EG == EG_HEAD) {
    __shared__ float4 part[4];
    float t1 = -INFINITY, t2 = -INFINITY, ma = 0.0f;
    int i1 = 0x7fffffff;
#pragma unroll
    for (int r = 0; r < R; ++r) {           // rows ascend, so an equal value keeps the lower row
      const int row = row0 + r;
      if (!live || row >= N) continue;
      const float y = v[0][r];
      ma = fmaxf(ma, fabsf(y));
      if (y > t1) { t2 = t1; t1 = y; i1 = row; }
      else t2 = fmaxf(t2, y);
      if (lane == 0) ((float*)a.y)[row] = y;
    }
    if (lane == 0) part[wave] = float4{t1, __int_as_float(i1), t2, ma};
    __syncthreads();
    if (t == 0) {
      float4 s = part[0];
#pragma unroll
      for (int w = 1; w < 4; ++w) s = top2_merge(s, part[w]);
      ((float4*)a.slots)[blockIdx.x] = s;
    }
  } else {
    if (lane == 0) gemv_store<1, R, EG>(a, v, row0, e_pos, h_res, h_cs, h_sn);
  }
}

typedef void (*gemv_fn)(GemvArgs);

// Kernel selection for one weight format: M tile in {1,2,4,8}, row group R = 1 (plain) or 2
// (paired epilogues, or a plain hint of 2), x in LDS (XS=1) unless it does not fit (XS=0).
template <int FMT, int M, int EG>
gemv_fn pick_gemv_r(int R, int xs) {
  if constexpr (EG == EG_PLAIN) {
    if (R == 1) return xs ? gemv_kernel<FMT, M, 1, 1, EG> : gemv_kernel<FMT, M, 1, 0, EG>;
  }
  return xs ? gemv_kernel<FMT, M, 2, 1, EG> : gemv_kernel<FMT, M, 2, 0, EG>;
}
template <int FMT, int M>
gemv_fn pick_gemv_eg(int eg, int R, int xs) {
  return eg == EG_QKV ? pick_gemv_r<FMT, M, EG_QKV>(R, xs)
       : eg == EG_SWIGLU ? pick_gemv_r<FMT, M, EG_SWIGLU>(R, xs)
                         : pick_gemv_r<FMT, M, EG_PLAIN>(R, xs);
}
template <int FMT>
gemv_fn pick_gemv(int mt, int eg, int R, int xs) {
  return mt == 1 ? pick_gemv_eg<FMT, 1>(eg, R, xs) : mt == 2 ? pick_gemv_eg<FMT, 2>(eg, R, xs)
       : mt == 4 ? pick_gemv_eg<FMT, 4>(eg, R, xs) : pick_gemv_eg<FMT, 8>(eg, R, xs);
}

template <int FMT, int U>
gemv_fn pick_gemv_row_u(int eg, int R, int norm) {
  if constexpr (FMT == FMT_F16) {
    if (eg == EG_HEAD) return norm == 1 ? gemv_row_kernel<FMT, 2, 1, EG_HEAD, U> : nullptr;
  }
  if (eg == EG_HEAD) return nullptr;
  if (norm == 2 && eg == EG_PLAIN)                 // x staged once per workgroup through LDS, no norm
    return R == 2 ? gemv_row_kernel<FMT, 2, 2, EG_PLAIN, U> : gemv_row_kernel<FMT, 1, 2, EG_PLAIN, U>;
  if (norm == 2) norm = 0;
  if (eg == EG_QKV) return norm ? gemv_row_kernel<FMT, 2, 1, EG_QKV, U> : gemv_row_kernel<FMT, 2, 0, EG_QKV, U>;
  if (eg == EG_SWIGLU) return norm ? gemv_row_kernel<FMT, 2, 1, EG_SWIGLU, U> : gemv_row_kernel<FMT, 2, 0, EG_SWIGLU, U>;
  if (R == 2) return norm ? gemv_row_kernel<FMT, 2, 1, EG_PLAIN, U> : gemv_row_kernel<FMT, 2, 0, EG_PLAIN, U>;
  return norm ? gemv_row_kernel<FMT, 1, 1, EG_PLAIN, U> : gemv_row_kernel<FMT, 1, 0, EG_PLAIN, U>;
}
// Chunks per lane the fast path is built for, per format (0: none); see gemv_row_kernel.
__host__ __device__ inline int fast_units(int fmt, int nchunks) {
  const int u = (nchunks + 63) / 64;
  if (fmt == FMT_I8 || fmt == FMT_BW) return u == 4 || u == 11 ? u : 0;
  if (fmt == FMT_Q4 || fmt == FMT_L4 || fmt == FMT_Q4K || fmt == FMT_Q6K) return u == 2 || u == 6 ? u : 0;
  return u == 8 ? u : 0;
}
template <int FMT>
gemv_fn pick_gemv_row(int eg, int R, int norm, int U) {
  if constexpr (FMT == FMT_I8 || FMT == FMT_BW)
    return U == 11 ? pick_gemv_row_u<FMT, 11>(eg, R, norm) : pick_gemv_row_u<FMT, 4>(eg, R, norm);
  else if constexpr (FMT == FMT_Q4 || FMT == FMT_L4 || FMT == FMT_Q4K || FMT == FMT_Q6K)
    return U == 6 ? pick_gemv_row_u<FMT, 6>(eg, R, norm) : pick_gemv_row_u<FMT, 2>(eg, R, norm);
  else return pick_gemv_row_u<FMT, 8>(eg, R, norm);
}

// Per-format selectors, each compiled in its own translation unit.
gemv_fn pick_gemv_i8(int mt, int eg, int R, int xs);
gemv_fn pick_gemv_q4(int mt, int eg, int R, int xs);
gemv_fn pick_gemv_f16(int mt, int eg, int R, int xs);
gemv_fn pick_gemv_bw(int mt, int eg, int R, int xs);
gemv_fn pick_gemv_l4(int mt, int eg, int R, int xs);
gemv_fn pick_gemv_q4k(int mt, int eg, int R, int xs);
gemv_fn pick_gemv_q6k(int mt, int eg, int R, int xs);
gemv_fn pick_gemv_row_i8(int eg, int R, int norm, int U);
gemv_fn pick_gemv_row_q4(int eg, int R, int norm, int U);
gemv_fn pick_gemv_row_f16(int eg, int R, int norm, int U);
gemv_fn pick_gemv_row_bw(int eg, int R, int norm, int U);
gemv_fn pick_gemv_row_l4(int eg, int R, int norm, int U);
gemv_fn pick_gemv_row_q4k(int eg, int R, int norm, int U);
gemv_fn pick_gemv_row_q6k(int eg, int R, int norm, int U);

}  // namespace afx
