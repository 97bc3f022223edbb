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
//   fp16 : a chunk = 8 weights -> one A operand;
//   blockwise int8 (one fp16 scale per 32-weight block): like int8, each operand multiplied by
//          its block's scale in fp16, i.e. the reference's reconstructed weight fp16(q * s).
// A workgroup owns 16 output rows; its NW wavefronts split K evenly and their partial 16x16
// tiles are summed through LDS by wavefront 0, which applies the epilogue.
// Weight loads are row-contiguous: a batch is 4 steps = 16 rows x 256 bytes, fetched as four
// loads in which 16 lanes read 256 contiguous bytes of one row (the MFMA layout would have 16
// lanes touch 16 rows x 16 bytes per load), then transposed into the MFMA layout through a
// wavefront-private LDS tile padded to 272 bytes per row (conflict-free 16-byte reads).  A
// wavefront issues all its batches' weight loads at once (up to four; longer rows go in
// rounds).  Activation rows of unused token columns read through a buffer resource at an
// out-of-range offset, which returns zeros without a memory access.
// MoE: the grid's y dimension is the expert; workgroups of experts with no tokens exit at once
// (fixed launch shape, so the layer stays graph-capturable).
#include <stdlib.h>
#include "afx_gemv_impl.h"
#include "afx_mfma.h"

namespace afx {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

template <int FMT> struct MfmaFmt;
template <> struct MfmaFmt<FMT_I8> { static constexpr int kK = 64, kMfma = 2; };    // k per step (64 lanes)
template <> struct MfmaFmt<FMT_Q4> { static constexpr int kK = 128, kMfma = 4; };
template <> struct MfmaFmt<FMT_F16> { static constexpr int kK = 32, kMfma = 1; };
template <> struct MfmaFmt<FMT_BW> { static constexpr int kK = 64, kMfma = 2; };

constexpr int kSPB = 4;            // steps per batch: 16 rows x 256 bytes
constexpr int kMaxSlices = 8;      // K slices of the split persistent kernel (workspace: 32 B per output)
constexpr int kPxMaxExperts = 2056; // experts the persistent kernel's LDS list holds (the reference allows 2049)
constexpr int kWRow = 256 + 16;    // LDS bytes per staged weight row
constexpr int kSRow = 40;          // LDS bytes per staged Q4_0 scale row (4 superblocks x 8 B, padded)

__device__ __forceinline__ h8 pack8(h2 a, h2 b, h2 c, h2 d) {
  h8 r;
  r[0] = a.x; r[1] = a.y; r[2] = b.x; r[3] = b.y; r[4] = c.x; r[5] = c.y; r[6] = d.x; r[7] = d.y;
  return r;
}
__device__ __forceinline__ h8 as_h8(u4 v) { return __builtin_bit_cast(h8, v); }
__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A operand of MFMA j of a step: the 8 fp16 weights (row r, k slot g) decoded from the lane's
// 16-byte chunk `w` of the step and the step's block scales `dv` of row r (Q4_0, blockwise).
template <int FMT>
__device__ __forceinline__ h8 mfma_a_operand(const u4& w, const u2& dv, int g, int j) {
  if constexpr (FMT == FMT_I8) {
    h2 q0, q1, q2, q3;
    i8x4_to_h2(j == 0 ? w.x : w.z, q0, q1);
    i8x4_to_h2(j == 0 ? w.y : w.w, q2, q3);
    return pack8(q0, q1, q2, q3);
  } else if constexpr (FMT == FMT_BW) {
    // chunk 4t + g holds k 16g .. 16g + 15 of the step: block g / 2 of its two
    const h2 sp = as_h2(dv.x);
    const half_t s = (g >> 1) ? sp.y : sp.x;
    const h2 s2 = {s, s};
    h2 q0, q1, q2, q3;
    i8x4_to_h2(j == 0 ? w.x : w.z, q0, q1);
    i8x4_to_h2(j == 0 ? w.y : w.w, q2, q3);
    return pack8(q0 * s2, q1 * s2, q2 * s2, q3 * s2);   // fp16(q * s)
  } else if constexpr (FMT == FMT_Q4) {
    const uint32_t wd = j == 0 ? w.x : j == 1 ? w.y : j == 2 ? w.z : w.w;
    const h2 dd = as_h2(j < 2 ? dv.x : dv.y);
    const half_t d = (j & 1) ? dd.y : dd.x;
    const h2 d2 = {d, d};
    h2 q[4];
    q4_word_to_h2(wd, q);
    return pack8(q[0] * d2, q[1] * d2, q[2] * d2, q[3] * d2);   // fp16((nibble - 8) * d)
  } else {
    return as_h8(w);
  }
}

// The epilogue's inputs for a lane's output rows rb .. rb + 3 (N % 4 == 0: all four exist when
// rb < N), as fp16 pairs, zeros where the epilogue has none: the int8 row scales, the bias, the
// residual of output row yr.
struct EpiOps {
  u2 sc, bi, re;
};
__device__ __forceinline__ u2 load_h4(const half_t* p) {
  h2 lo, hi;
  lo.x = p[0]; lo.y = p[1]; hi.x = p[2]; hi.y = p[3];
  return (u2){__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}
// Loaded where they are used: for the kernels whose epilogue ends the workgroup's work.  The
// persistent kernel prefetches them with each tile instead (a load issued in its epilogue would
// wait for every tile in flight before it: the memory counter retires in order).
template <int FMT>
__device__ __forceinline__ EpiOps epi_load(const MfmaArgs& a, const half_t* sbase, int rb, bool tok_ok, int yr) {
  EpiOps o = {{0u, 0u}, {0u, 0u}, {0u, 0u}};
  if (rb >= a.N) return o;
  if constexpr (FMT == FMT_I8) o.sc = *(const u2*)(sbase + rb);   // 8-byte aligned: checked at launch
  if (a.bias) o.bi = load_h4(a.bias + rb);
  if (a.epi == EPI_RESID && tok_ok) o.re = load_h4(a.resid + (size_t)yr * a.ldy + rb);
  return o;
}

// Tile epilogue of wavefront 0: v = this lane's summed tile entries, output rows rb .. rb + 3
// of one token column, stored to y row yr (tok_ok: the column is a real token) with the int8
// row scale, the bias and the epilogue, whose inputs are in `ops`.
template <int FMT, int EG>
__device__ __forceinline__ void mfma_store(const MfmaArgs& a, const EpiOps& ops, float (&v)[4], int rb, bool tok_ok,
                                           int yr) {
  const int N = a.N;
  if constexpr (FMT == FMT_I8) {
    const h2 s01 = as_h2(ops.sc.x), s23 = as_h2(ops.sc.y);
    v[0] *= (float)s01.x; v[1] *= (float)s01.y; v[2] *= (float)s23.x; v[3] *= (float)s23.y;
  }
  if (a.bias && rb < N) {
    const h2 b01 = as_h2(ops.bi.x), b23 = as_h2(ops.bi.y);
    v[0] += (float)b01.x; v[1] += (float)b01.y; v[2] += (float)b23.x; v[3] += (float)b23.y;
  }
  if (!tok_ok || rb >= N) return;
  if constexpr (EG == EG_SWIGLU) {
    half_t* yp = (half_t*)a.y + (size_t)yr * a.ldy + (rb >> 1);
    const float g0 = (float)(half_t)v[0], u0 = (float)(half_t)v[1];
    const float g1 = (float)(half_t)v[2], u1 = (float)(half_t)v[3];
    const bool gelu = a.epi == EPI_GEGLU;
    yp[0] = (half_t)(glu_act(gelu, g0) * u0);
    yp[1] = (half_t)(glu_act(gelu, g1) * u1);
  } else if (a.epi == EPI_F32) {
    float* yp = (float*)a.y + (size_t)yr * a.ldy + rb;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (rb + i < N) yp[i] = v[i];
  } else {
    half_t* yp = (half_t*)a.y + (size_t)yr * a.ldy + rb;
    const h2 r01 = as_h2(ops.re.x), r23 = as_h2(ops.re.y);
    const float res[4] = {(float)r01.x, (float)r01.y, (float)r23.x, (float)r23.y};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float o = v[i];
      if (a.epi == EPI_RESID) o = res[i] + (float)(half_t)o;
      yp[i] = (half_t)o;
    }
  }
}

template <int FMT, int EG, int NW, int NB>
__global__ __launch_bounds__(NW * 64) void mfma_kernel(MfmaArgs a) {
  constexpr int KS = MfmaFmt<FMT>::kK, NM = MfmaFmt<FMT>::kMfma;
  __shared__ __align__(16) unsigned char wl[NW][16 * kWRow];
  __shared__ __align__(16) unsigned char sl[NW][has_block_scales<FMT>() ? 16 * kSRow : 16];
  __shared__ f4 red[NW][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;          // MFMA role: A row / B column, k slot
  const int lr = lane >> 4, lc = lane & 15;        // load role: row lr + 4h, chunk lc of a batch
  const int e = blockIdx.y;
  const int N = a.N, K = a.K;
  const int n0 = blockIdx.x * 16;
  int ntok = a.M;
  const int* lst = nullptr;
  if (a.cnt) {
    ntok = a.cnt[e];
    if (ntok <= 0) return;                         // whole workgroup: no barrier reached
    lst = a.list + (size_t)e * a.T;
  }
  const unsigned char* wbase = (const unsigned char*)a.w + (size_t)e * a.w_es;
  const half_t* sbase = a.scale ? a.scale + (size_t)e * a.s_es : nullptr;
  const size_t rowbytes = Fmt<FMT>::row_bytes(K);
  const unsigned char* lrow[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const int row = n0 + 4 * h + lr < N ? n0 + 4 * h + lr : N - 1;   // tail rows computed, not stored
    lrow[h] = wbase + (size_t)row * rowbytes + lc * 16;
  }
  // block scales: lane l stages row l / 4's scales of step (batch step) l % 4 -- Q4 4 per
  // step (8 bytes), blockwise 2 per step (4 bytes)
  constexpr int kSPS = FMT == FMT_Q4 ? 4 : 2;     // block scales per step
  const half_t* srow = nullptr;
  if constexpr (has_block_scales<FMT>()) {
    const int row = n0 + (lane >> 2) < N ? n0 + (lane >> 2) : N - 1;
    srow = sbase + (size_t)row * (K >> 5) + kSPS * (lane & 3);
  }
  const int nsteps = K / KS;
  const int s0 = nsteps * wave / NW, s1 = nsteps * (wave + 1) / NW;   // this wavefront's K range
  const int nb = (s1 - s0 + kSPB - 1) / kSPB;
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, a.xbytes);
  unsigned char* wls = wl[wave];
  unsigned char* sls = sl[wave];
  constexpr int kOOB = 0x7fff0000;

  const int nsw = s1 - s0;                         // steps of this wavefront

  for (int tg = 0; tg < ntok; tg += 16) {
    const int ti = tg + r;                        // B column (token) of this lane
    const bool tok_ok = ti < ntok;
    int xr = tok_ok ? ti : 0;
    if (lst) {
      const int ent = lst[tok_ok ? ti : 0];
      xr = a.x_by_token ? ent / a.k : ent;
    }
    const int xoff = tok_ok ? xr * a.ldx * 2 : kOOB;      // out of range: reads zeros
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    // rounds of NB batches (NB = this shape's batches per wavefront when that is at most 4):
    // all of a round's weight loads are issued at once
    for (int b0 = 0; b0 < nb; b0 += NB) {
      // activations: one batch (4 steps) per load group; int8/fp16 keep two groups in flight
      // (the next batch's loads go out before this batch's math), Q4_0 one (its group is 4x larger).
      // The round's first group is issued before its weight loads: the memory counter retires in
      // order, so the first batch's math then waits only for the first batch's weights, and runs
      // while the later batches' weights are still arriving.
      constexpr int XG = NM <= 2 ? 2 : 1;
      auto load_x = [&](u4 (&xv)[kSPB][NM], int b) {
#pragma unroll
        for (int t = 0; t < kSPB; ++t) {
          const int i = (b0 + b) * kSPB + t;       // step relative to s0
          const int s = s0 + i;
          const bool in = i < nsw;
#pragma unroll
          for (int j = 0; j < NM; ++j) {
            int kx;
            if constexpr (FMT == FMT_I8 || FMT == FMT_BW) kx = s * KS + 16 * g + 8 * j;
            else if constexpr (FMT == FMT_Q4) kx = 32 * (4 * s + j) + 8 * g;
            else kx = s * KS + 8 * g;
            xv[t][j] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(xrs, in ? xoff + kx * 2 : kOOB, 0, 0));
          }
        }
      };
      u4 xv[XG][kSPB][NM];
      load_x(xv[0], 0);
      u4 wq[NB][4];
      u2 sq[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        // batch b0 + b, clamped per lane to the row (a clamped chunk is loaded but never used)
        const int sb = s0 + (b0 + b) * kSPB;
        int c = sb * 4 + lc;
        c = c < nsteps * 4 ? c : nsteps * 4 - 1;
#pragma unroll
        for (int h = 0; h < 4; ++h) wq[b][h] = __builtin_nontemporal_load((const u4*)(lrow[h] + (size_t)(c - lc) * 16));
        if constexpr (has_block_scales<FMT>()) {
          int q = sb + (lane & 3);
          q = q < nsteps ? q : nsteps - 1;
          if constexpr (FMT == FMT_Q4) sq[b] = *(const u2*)(srow + (size_t)(q - (lane & 3)) * 4);
          else sq[b] = (u2){*(const uint32_t*)(srow + (size_t)(q - (lane & 3)) * 2), 0u};
        }
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b0 + b >= nb) break;                   // wavefront-uniform
        if constexpr (XG == 2) {
          if (b + 1 < NB) load_x(xv[(b + 1) & 1], b + 1);
        } else if (b) {
          load_x(xv[0], b);
        }
        u4 (&xb)[kSPB][NM] = xv[XG == 2 ? (b & 1) : 0];
        // stage the batch, then read it back in the MFMA layout (row r, chunk 4 * step + g)
        if (b) wave_sync_lds();                    // the previous batch's reads are done
#pragma unroll
        for (int h = 0; h < 4; ++h) *(u4*)(wls + (4 * h + lr) * kWRow + lc * 16) = wq[b][h];
        if constexpr (FMT == FMT_Q4) *(u2*)(sls + (lane >> 2) * kSRow + (lane & 3) * 8) = sq[b];
        if constexpr (FMT == FMT_BW) *(uint32_t*)(sls + (lane >> 2) * kSRow + (lane & 3) * 4) = sq[b].x;
        wave_sync_lds();
        u4 wv[kSPB];
        u2 dv[kSPB];
#pragma unroll
        for (int t = 0; t < kSPB; ++t) {
          wv[t] = *(const u4*)(wls + r * kWRow + (4 * t + g) * 16);
          if constexpr (FMT == FMT_Q4) dv[t] = *(const u2*)(sls + r * kSRow + t * 8);
          if constexpr (FMT == FMT_BW) dv[t] = (u2){*(const uint32_t*)(sls + r * kSRow + t * 4), 0u};
        }
#pragma unroll
        for (int t = 0; t < kSPB; ++t) {
          if ((b0 + b) * kSPB + t >= nsw) break;   // wavefront-uniform
#pragma unroll
          for (int j = 0; j < NM; ++j)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(mfma_a_operand<FMT>(wv[t], dv[t], g, j), as_h8(xb[t][j]), acc,
                                                         0, 0, 0);
        }
      }
      wave_sync_lds();                             // the round's reads are done before the next round's writes
    }
    // sum the K ranges; wavefront 0 finishes the tile
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = acc[i];
#pragma unroll
      for (int w = 1; w < NW; ++w) {
        const f4 p = red[w][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] += p[i];
      }
      // output rows n0 + 4g .. + 3 of token ti, to its entry (MoE) or activation row (dense)
      const int yr = tok_ok ? (lst ? lst[ti] : ti) : 0;
      mfma_store<FMT, EG>(a, epi_load<FMT>(a, sbase, n0 + 4 * g, tok_ok, yr), v, n0 + 4 * g, tok_ok, yr);
    }
    __syncthreads();                               // red is reused by the next token group
  }
}

// Persistent variant for at most 16 activation rows (dense) or 16 tokens (MoE) whose K range
// per wavefront is one batch (<= kSPB steps).  One workgroup per CU walks 16-row tiles: a dense
// linear's tiles blockIdx.x, + gridDim.x, ...; MoE, a contiguous range of the active experts'
// (expert, tile) units.  Each wavefront loads its slice of x into registers once (MoE: again
// when the expert changes) and keeps it for every tile (x leaves L2 about once per workgroup
// instead of once per tile), and the weight loads of the next PD tiles are in flight while a
// tile's MFMAs run.  The cross-wavefront sums
// alternate between two LDS buffers: one barrier per tile (wavefront 0 reads tile i's buffer
// before it reaches the barrier of tile i + 1; the other wavefronts write that buffer again
// only for tile i + 2, after that barrier).
// SPLIT: K is cut into a.ks slices (long rows: the x slice of a whole row would not fit the
// registers), a unit is (expert, slice, tile), and each unit's wavefront-summed tile goes to the
// fp32 workspace a.ws[slice][row][column] (int8 row scale applied, nothing else); units of one
// (expert, slice) are contiguous, so x is reloaded only where that pair changes.  A finishing
// launch sums the slices and applies the epilogue (mfma_finish_kernel).
template <int FMT, int EG, int NW, int PD, bool MOE, bool SPLIT>
__global__ __launch_bounds__(NW * 64) void mfma_px_kernel(MfmaArgs a) {
  constexpr int KS = MfmaFmt<FMT>::kK, NM = MfmaFmt<FMT>::kMfma;
  constexpr int kSPS = FMT == FMT_Q4 ? 4 : 2;     // block scales per step (Q4_0, blockwise)
  constexpr int kOOB = 0x7fff0000;
  __shared__ __align__(16) unsigned char wl[NW][16 * kWRow];
  __shared__ __align__(16) unsigned char sl[NW][has_block_scales<FMT>() ? 16 * kSRow : 16];
  __shared__ f4 red[2][NW][64];
  // the wavefront index said to be uniform: its step range and the branches on it stay scalar
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;          // MFMA role: A row / B column (token), k slot
  const int lr = lane >> 4, lc = lane & 15;        // load role: row lr + 4h, chunk lc of the batch
  const int N = a.N, K = a.K;
  const int ntiles = (N + 15) >> 4;
  const size_t rowbytes = Fmt<FMT>::row_bytes(K);
  const unsigned char* wbase = (const unsigned char*)a.w;
  const int nsteps = K / KS;
  const int S = SPLIT ? a.ks : 1;                  // K slices
  // this wavefront's steps of slice q: [s0, s0 + nsw), 1 .. kSPB of them
  auto wrange = [&](int q, int& s0, int& nsw) {
    const int lo = nsteps * q / S, len = nsteps * (q + 1) / S - lo;
    s0 = lo + len * wave / NW;
    nsw = lo + len * (wave + 1) / NW - s0;
  };
  unsigned char* wls = wl[wave];
  unsigned char* sls = sl[wave];

  // Work units.  A dense linear walks the tiles blockIdx.x, + G, ...  MoE (cnt != null) takes a
  // contiguous, expert-major range of the active experts' (expert, tile) units, so its x (the
  // expert's routed rows) changes at most a few times per workgroup.  Every branch depends only
  // on blockIdx / gridDim and the expert counts (workgroup-uniform): all wavefronts meet every
  // barrier.
  const int G = gridDim.x;
  // MoE: the active experts, in order, compacted into LDS by the whole workgroup (a ballot prefix
  // per 64 experts), so a unit's expert is one LDS read and the expert count costs E / (64 NW)
  // rounds of loads, not E dependent ones.
  __shared__ int act_e[MOE ? kPxMaxExperts : 1];
  __shared__ int wcnt[NW];
  int v = blockIdx.x, vend = ntiles, vstep = G;
  if constexpr (SPLIT && !MOE) {                   // contiguous ranges of the (slice, tile) units
    const long long U = (long long)S * ntiles;
    v = (int)(U * blockIdx.x / G);
    vend = (int)(U * (blockIdx.x + 1) / G);
    vstep = 1;
  }
  if constexpr (MOE) {
    int nact = 0;
    for (int base = 0; base < a.E; base += NW * 64) {
      const int e = base + (int)threadIdx.x;
      const bool act = e < a.E && a.cnt[e] > 0;
      const unsigned long long m = __ballot(act);
      if (lane == 0) wcnt[wave] = __popcll(m);
      __syncthreads();
      int off = nact, tot = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        off += w < wave ? wcnt[w] : 0;
        tot += wcnt[w];
      }
      if (act) act_e[off + __popcll(m & ((1ull << lane) - 1))] = e;
      nact += tot;
      __syncthreads();                             // wcnt is rewritten next round; act_e is complete
    }
    const long long U = (long long)nact * S * ntiles;
    v = (int)(U * blockIdx.x / G);
    vend = (int)(U * (blockIdx.x + 1) / G);
    vstep = 1;
  }
  if (v >= vend) return;                           // whole workgroup, after its last barrier

  // A work unit: expert e, K slice q (this wavefront's steps [s0, s0 + nsw) of it), 16-row tile;
  // every field is workgroup-uniform.  The prefetch cursor walks the units v, v + vstep, ... by
  // increments, with a division only where the slice changes.
  struct Unit {
    int e, q, tile, s0, nsw;
  };
  // the expert is read as a uniform value, or the weight rows' buffer resource sits in vector
  // registers and every load becomes a per-lane waterfall loop
  auto expert_at = [&](int i) { return MOE ? __builtin_amdgcn_readfirstlane(act_e[i]) : 0; };
  Unit cur;
  int cei = MOE ? v / (ntiles * S) : 0;            // MoE: the cursor's expert, as an index into act_e
  cur.tile = v % ntiles;
  cur.q = SPLIT ? (v / ntiles) % S : 0;
  cur.e = expert_at(cei);
  wrange(cur.q, cur.s0, cur.nsw);
  auto advance = [&]() {                           // to the next unit of the walk (which exists)
    if (vstep != 1) {                              // dense, unsplit: tiles blockIdx.x, + G, ...
      cur.tile += vstep;
      return;
    }
    if (++cur.tile < ntiles) return;
    cur.tile = 0;
    if (++cur.q == S) {
      cur.q = 0;
      cur.e = expert_at(++cei);
    }
    wrange(cur.q, cur.s0, cur.nsw);
  };

  // this wavefront's slice of x in the B-operand layout (token column r, k slot g), for the
  // expert and slice xe (MoE: column r is entry r of the expert's list; dense: activation row r)
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, a.xbytes);
  bool tok_ok = false;
  int yr = r, xe = -1;                             // xe: expert * S + slice of the x slice held
  u4 xv[kSPB][NM];
  auto load_x = [&](const Unit& u) {
    int xr = r;
    tok_ok = r < a.M;
    if constexpr (MOE) {
      const int* lst = a.list + (size_t)u.e * a.T;
      tok_ok = r < a.cnt[u.e];
      const int ent = tok_ok ? lst[r] : 0;
      xr = a.x_by_token ? ent / a.k : ent;
      yr = ent;                                    // output row: the entry
    }
    const int xoff = tok_ok ? xr * a.ldx * 2 : kOOB;   // out of range: reads zeros
#pragma unroll
    for (int t = 0; t < kSPB; ++t) {
      const int s = u.s0 + t;
#pragma unroll
      for (int j = 0; j < NM; ++j) {
        int kx;
        if constexpr (FMT == FMT_I8 || FMT == FMT_BW) kx = s * KS + 16 * g + 8 * j;
        else if constexpr (FMT == FMT_Q4) kx = 32 * (4 * s + j) + 8 * g;
        else kx = s * KS + 8 * g;
        xv[t][j] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(xrs, t < u.nsw ? xoff + kx * 2 : kOOB, 0, 0));
      }
    }
    xe = u.e * S + u.q;
  };

  // One tile's weights for this wavefront's steps: 16 rows x 256 bytes, row-contiguous, and the
  // steps' block scales (lane l: row l / 4, step s0 + l % 4).  Each load is a buffer load at a
  // fixed per-lane offset from a workgroup-uniform base: the buffer starts at the tile's first
  // byte of this wavefront's steps and ends with the expert's matrix, so rows past N read zeros
  // (computed, never stored), and bytes past the wavefront's steps are those of the next steps
  // or row (loaded, never used).  A unit past the range (ok false) gets an empty buffer: the same
  // instructions, zeros, no memory traffic, so every path through the prefetch has the same
  // loads in flight and the compiler's wait counts for a unit's data stay exact.
  int loff[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) loff[h] = (4 * h + lr) * (int)rowbytes + lc * 16;
  const int soff = ((lane >> 2) * (K >> 5) + (lane & 3) * kSPS) * 2;
  // The epilogue's inputs (int8 row scales, bias, residual of the lane's output rows
  // tile * 16 + 4g .. + 3) come with the tile: a load issued in the epilogue would wait for every
  // tile in flight before it (the memory counter retires in order).  An absent input reads as
  // an empty buffer (zeros).
  constexpr bool kEpiIn = !MOE && !SPLIT;         // bias and residual: dense, unsplit launches only
  const long long res_halves = a.epi == EPI_RESID ? (long long)a.M * a.ldy : 0;
  auto load_tile = [&](const Unit& u, u4 (&wq)[4], u2& sq, EpiOps& eo, bool ok) {
    const int n0 = u.tile * 16;
    const long long wfirst = (long long)n0 * (long long)rowbytes + u.s0 * 64;
    const __amdgpu_buffer_rsrc_t wrs =
        make_rsrc(wbase + (size_t)u.e * a.w_es + wfirst, ok ? (int)((long long)N * (long long)rowbytes - wfirst) : 0);
#pragma unroll
    for (int h = 0; h < 4; ++h) wq[h] = buf_load16(wrs, loff[h]);
    if constexpr (has_block_scales<FMT>()) {
      const long long sfirst = (long long)n0 * (K >> 5) + u.s0 * kSPS;   // halves
      const __amdgpu_buffer_rsrc_t srs = make_rsrc(a.scale + (size_t)u.e * a.s_es + sfirst,
                                                   ok ? (int)(((long long)N * (K >> 5) - sfirst) * 2) : 0);
      if constexpr (FMT == FMT_Q4) sq = buf_load8(srs, soff);
      else sq = (u2){buf_load4(srs, soff), 0u};
    }
    if constexpr (FMT == FMT_I8) {
      const __amdgpu_buffer_rsrc_t ers = make_rsrc(a.scale + (size_t)u.e * a.s_es + n0, ok ? (N - n0) * 2 : 0);
      eo.sc = buf_load8(ers, 8 * g);
    }
    if constexpr (kEpiIn) {
      const __amdgpu_buffer_rsrc_t brs =
          make_rsrc(a.bias ? a.bias + n0 : (const half_t*)a.x, ok && a.bias ? (N - n0) * 2 : 0);
      eo.bi = buf_load8(brs, 8 * g);
      const __amdgpu_buffer_rsrc_t rrs =
          make_rsrc(res_halves ? a.resid + n0 : (const half_t*)a.x, ok && res_halves ? (int)((res_halves - n0) * 2) : 0);
      eo.re = buf_load8(rrs, (r * a.ldy + 4 * g) * 2);
    }
  };
  auto compute_tile = [&](const Unit& u, const u4 (&wq)[4], const u2& sq, const EpiOps& eo, f4 (&rd)[NW][64]) {
    if constexpr (MOE || SPLIT) {
      // the next expert's (or slice's) rows; the full wait keeps these loads from leaving the
      // compiler's wait counts (in-order, shared with the prefetched tiles) pending past the branch
      if (u.e * S + u.q != xe) {
        load_x(u);
        __builtin_amdgcn_s_waitcnt(0);
      }
    }
    wave_sync_lds();                               // the previous tile's staged reads are done
#pragma unroll
    for (int h = 0; h < 4; ++h) *(u4*)(wls + (4 * h + lr) * kWRow + lc * 16) = wq[h];
    if constexpr (FMT == FMT_Q4) *(u2*)(sls + (lane >> 2) * kSRow + (lane & 3) * 8) = sq;
    if constexpr (FMT == FMT_BW) *(uint32_t*)(sls + (lane >> 2) * kSRow + (lane & 3) * 4) = sq.x;
    wave_sync_lds();
    u4 wv[kSPB];
    u2 dv[kSPB] = {};
#pragma unroll
    for (int t = 0; t < kSPB; ++t) {
      wv[t] = *(const u4*)(wls + r * kWRow + (4 * t + g) * 16);
      if constexpr (FMT == FMT_Q4) dv[t] = *(const u2*)(sls + r * kSRow + t * 8);
      if constexpr (FMT == FMT_BW) dv[t] = (u2){*(const uint32_t*)(sls + r * kSRow + t * 4), 0u};
    }
    // every step's operands are read before the first is used: one LDS round trip, where the
    // compiler would otherwise move each step's reads into that step's branch and wait there
#pragma unroll
    for (int t = 0; t < kSPB; ++t) asm volatile("" : "+v"(wv[t]), "+v"(dv[t]));
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < kSPB; ++t) {
      if (t >= u.nsw) break;                       // wavefront-uniform
#pragma unroll
      for (int j = 0; j < NM; ++j)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(mfma_a_operand<FMT>(wv[t], dv[t], g, j), as_h8(xv[t][j]), acc,
                                                     0, 0, 0);
    }
    rd[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = acc[i];
#pragma unroll
      for (int w = 1; w < NW; ++w) {
        const f4 p = rd[w][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] += p[i];
      }
      const int rb = u.tile * 16 + 4 * g;
      if constexpr (SPLIT) {
        if constexpr (FMT == FMT_I8) {
          const h2 s01 = as_h2(eo.sc.x), s23 = as_h2(eo.sc.y);
          v[0] *= (float)s01.x; v[1] *= (float)s01.y; v[2] *= (float)s23.x; v[3] *= (float)s23.y;
        }
        if (tok_ok && rb < N)
          *(f4*)(a.ws + ((size_t)u.q * a.ws_rows + yr) * N + rb) = (f4){v[0], v[1], v[2], v[3]};
      } else {
        mfma_store<FMT, EG>(a, eo, v, rb, tok_ok, yr);
      }
    }
  };

  // PD units in flight ahead of the one being computed: unit j of the walk in buffer j % (PD + 1),
  // the buffers rotated by a fully unrolled inner loop (fixed registers).  Every pass of the loop
  // runs all PD + 1 slots (a slot past the walk's end issues out-of-range loads and skips its
  // tile), so the loop has one entry and one back edge: with early exits from the unrolled slots
  // the compiler met buffers still in flight on a back edge and waited for all of them there.
  // PD = 1 for a few units per workgroup (a deeper prefetch measured slower there: 10.7 against
  // 10.2 us for Q4_0 11008 x 4096 at 4 rows), PD = 3 for long runs of units (MoE).
  constexpr int NBUF = PD + 1;
  static_assert(NBUF % 2 == 0, "slot b of a pass is unit j0 + b with j0 a multiple of NBUF: red[b & 1] alternates");
  u4 wq[NBUF][4];
  u2 sq[NBUF];
  EpiOps eo[NBUF];
  Unit un[NBUF];
#pragma unroll
  for (int b = 0; b < NBUF; ++b) {
    sq[b] = (u2){0u, 0u};
    eo[b] = EpiOps{{0u, 0u}, {0u, 0u}, {0u, 0u}};
    un[b] = cur;
  }
  const int n = (vend - v + vstep - 1) / vstep;   // units of this workgroup, >= 1
  // unit j of the walk into buffer b: the cursor moves on while j < n, and a slot past the end
  // keeps the last unit's indices (its loads are empty either way)
  auto prefetch = [&](int j, int b) {
    if (j > 0 && j < n) advance();
    un[b] = cur;
    load_tile(un[b], wq[b], sq[b], eo[b], j < n);
  };
  load_x(cur);
#pragma unroll
  for (int b = 0; b < PD; ++b) prefetch(b, b);
  // x is complete on every path into the loop (here, and after each reload): otherwise the
  // compiler's merged wait counts keep the x slice pending and every unit's first MFMA waits for
  // the tiles prefetched before it
  __builtin_amdgcn_s_waitcnt(0);
  for (int j0 = 0; j0 < n; j0 += NBUF) {
#pragma unroll
    for (int b = 0; b < NBUF; ++b) {
      const int bp = (b + PD) % NBUF;              // unit j0 + b + PD goes to buffer bp
      prefetch(j0 + b + PD, bp);
      __builtin_amdgcn_sched_barrier(0);
      if (j0 + b < n) compute_tile(un[b], wq[b], sq[b], eo[b], red[b & 1]);   // uniform
    }
  }
}

typedef void (*mfma_fn)(MfmaArgs);

template <int FMT, int EG, int NW>
static mfma_fn pick_mfma_b(int nb) {
  switch (nb) {
    case 1: return mfma_kernel<FMT, EG, NW, 1>;
    case 2: return mfma_kernel<FMT, EG, NW, 2>;
    case 3: return mfma_kernel<FMT, EG, NW, 3>;
    default: return mfma_kernel<FMT, EG, NW, 4>;
  }
}
template <int FMT, int EG>
static mfma_fn pick_mfma_w(int nw, int nb) {
  return nw == 4 ? pick_mfma_b<FMT, EG, 4>(nb) : nw == 8 ? pick_mfma_b<FMT, EG, 8>(nb) : pick_mfma_b<FMT, EG, 16>(nb);
}
static mfma_fn pick_mfma(int fmt, bool swiglu, int nw, int nb) {
  if (fmt == FMT_I8) return swiglu ? pick_mfma_w<FMT_I8, EG_SWIGLU>(nw, nb) : pick_mfma_w<FMT_I8, EG_PLAIN>(nw, nb);
  if (fmt == FMT_BW) return swiglu ? pick_mfma_w<FMT_BW, EG_SWIGLU>(nw, nb) : pick_mfma_w<FMT_BW, EG_PLAIN>(nw, nb);
  if (fmt == FMT_Q4) return swiglu ? pick_mfma_w<FMT_Q4, EG_SWIGLU>(nw, nb) : pick_mfma_w<FMT_Q4, EG_PLAIN>(nw, nb);
  return swiglu ? pick_mfma_w<FMT_F16, EG_SWIGLU>(nw, nb) : pick_mfma_w<FMT_F16, EG_PLAIN>(nw, nb);
}

template <int FMT, int EG, int PD, bool MOE, bool SPLIT>
static mfma_fn pick_mfma_px_w(int nw) {
  if constexpr (FMT == FMT_Q4)   // Q4_0 never takes 16 wavefronts (its x slice would not fit 128 VGPRs)
    return nw == 4 ? mfma_px_kernel<FMT, EG, 4, PD, MOE, SPLIT> : mfma_px_kernel<FMT, EG, 8, PD, MOE, SPLIT>;
  else if constexpr (SPLIT)      // the split launch takes at most 8 wavefronts
    return nw == 4 ? mfma_px_kernel<FMT, EG, 4, PD, MOE, SPLIT> : mfma_px_kernel<FMT, EG, 8, PD, MOE, SPLIT>;
  else   // 16 wavefronts keep one unit of prefetch: three would spill at the 128-VGPR cap
    return nw == 4 ? mfma_px_kernel<FMT, EG, 4, PD, MOE, SPLIT>
         : nw == 8 ? mfma_px_kernel<FMT, EG, 8, PD, MOE, SPLIT> : mfma_px_kernel<FMT, EG, 16, 1, MOE, SPLIT>;
}
template <int FMT, bool MOE>
static mfma_fn pick_mfma_px_f(bool swiglu, int nw, int pd, bool split) {
  if (split)                     // the epilogue runs in the finishing launch
    return pd == 3 ? pick_mfma_px_w<FMT, EG_PLAIN, 3, MOE, true>(nw) : pick_mfma_px_w<FMT, EG_PLAIN, 1, MOE, true>(nw);
  if (pd == 3)
    return swiglu ? pick_mfma_px_w<FMT, EG_SWIGLU, 3, MOE, false>(nw) : pick_mfma_px_w<FMT, EG_PLAIN, 3, MOE, false>(nw);
  return swiglu ? pick_mfma_px_w<FMT, EG_SWIGLU, 1, MOE, false>(nw) : pick_mfma_px_w<FMT, EG_PLAIN, 1, MOE, false>(nw);
}
template <bool MOE>
static mfma_fn pick_mfma_px_m(int fmt, bool swiglu, int nw, int pd, bool split) {
  if (fmt == FMT_I8) return pick_mfma_px_f<FMT_I8, MOE>(swiglu, nw, pd, split);
  if (fmt == FMT_BW) return pick_mfma_px_f<FMT_BW, MOE>(swiglu, nw, pd, split);
  if (fmt == FMT_Q4) return pick_mfma_px_f<FMT_Q4, MOE>(swiglu, nw, pd, split);
  return pick_mfma_px_f<FMT_F16, MOE>(swiglu, nw, pd, split);
}
static mfma_fn pick_mfma_px(int fmt, bool swiglu, int nw, int pd, bool moe, bool split) {
  return moe ? pick_mfma_px_m<true>(fmt, swiglu, nw, pd, split) : pick_mfma_px_m<false>(fmt, swiglu, nw, pd, split);
}

// The K-split launch's second half: y[row][n] = epilogue(sum over the slices of ws[slice][row][n])
// (bias, residual, fp32 or fp16 store; the int8 row scale was applied per slice), four columns per
// thread.  The SwiGLU epilogue never splits (its gate/up rows are short in every model here).
__global__ __launch_bounds__(256) void mfma_finish_kernel(MfmaArgs a, int rows) {
  const int per_row = a.N >> 2;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * per_row) return;
  const int yr = idx / per_row, rb = 4 * (idx - yr * per_row);
  // every slice's load issued before the first sum (one memory round trip); slots past ks re-read
  // slice 0 and are not added
  f4 p[kMaxSlices];
#pragma unroll
  for (int q = 0; q < kMaxSlices; ++q)
    p[q] = *(const f4*)(a.ws + ((size_t)(q < a.ks ? q : 0) * a.ws_rows + yr) * a.N + rb);
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int q = 0; q < kMaxSlices; ++q)
    if (q < a.ks) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] += p[q][i];
    }
  mfma_store<FMT_F16, EG_PLAIN>(a, epi_load<FMT_F16>(a, nullptr, rb, true, yr), v, rb, true, yr);
}

static int mfma_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    hipDeviceProp_t p;
    cus = hipGetDeviceProperties(&p, dev) == hipSuccess ? p.multiProcessorCount : 256;
  }
  return cus;
}

bool mfma_supported(int fmt, int K) {
  if (fmt == FMT_L4 || fmt == FMT_Q4K || fmt == FMT_Q6K) return false;   // int4 codebook, K-quants: vector kernels
  const int ks = fmt == FMT_I8 || fmt == FMT_BW ? 64 : fmt == FMT_Q4 ? 128 : 32;
  return K % ks == 0 && K / ks >= 8;                           // at least one step per wavefront
}

int mfma_launch(int fmt, const MfmaArgs& a, int E, hipStream_t stream, const char* what, int* ks_out) {
  if (ks_out) *ks_out = 1;
  AFX_REQUIRE(fmt >= 0 && fmt <= 3, "%s: unknown weight format %d", what, fmt);
  AFX_REQUIRE(a.w && a.x && a.y, "%s: null pointer", what);
  AFX_REQUIRE(a.N >= 1 && a.N % 4 == 0, "%s: N=%d must be a multiple of 4", what, a.N);
  AFX_REQUIRE(mfma_supported(fmt, a.K), "%s: K=%d does not fit the MFMA split", what, a.K);
  AFX_REQUIRE(a.ldx % 8 == 0 && ((uintptr_t)a.x & 15) == 0 && ((uintptr_t)a.w & 15) == 0,
              "%s: x and weights must be 16-byte aligned (ldx %% 8 == 0)", what);
  AFX_REQUIRE(fmt != FMT_I8 || (a.scale && ((uintptr_t)a.scale & 7) == 0), "%s: int8 needs aligned row scales", what);
  AFX_REQUIRE(fmt != FMT_Q4 || (a.scale && ((uintptr_t)a.scale & 7) == 0), "%s: Q4_0 needs aligned block scales", what);
  AFX_REQUIRE(fmt != FMT_BW || (a.scale && ((uintptr_t)a.scale & 3) == 0), "%s: blockwise needs aligned block scales", what);
  AFX_REQUIRE(a.cnt ? (a.list && a.T >= 1 && a.k >= 1) : (a.M >= 1), "%s: bad token description", what);
  AFX_REQUIRE(a.epi != EPI_RESID || a.resid, "%s: residual pointer required", what);
  AFX_REQUIRE(!a.cnt || (!a.bias && a.epi != EPI_RESID), "%s: expert linears take no bias or residual", what);
  const long long xrows = a.cnt ? (a.x_by_token ? a.T : (long long)a.T * a.k) : a.M;
  const long long xbytes = xrows * a.ldx * 2;
  AFX_REQUIRE(xbytes < 0x7fff0000LL, "%s: activations span %lld bytes (limit 2 GiB)", what, xbytes);
  const long long rowb = fmt == FMT_I8 || fmt == FMT_BW ? a.K : fmt == FMT_Q4 ? a.K / 2 : 2LL * a.K;
  AFX_REQUIRE((long long)a.N * rowb + 65536 < 0x7fff0000LL,
              "%s: a weight matrix of %d x %d exceeds the 2 GiB buffer range", what, a.N, a.K);
  MfmaArgs b = a;
  b.xbytes = (int)xbytes;
  b.E = E;
  const bool swiglu = a.epi == EPI_SWIGLU || a.epi == EPI_GEGLU;   // gated pair epilogue
  // wavefronts per workgroup: the fewest of 4, 8, 16 that leave each wavefront at most four
  // batches; batches per round = batches per wavefront, capped at 4 (measured on MI355X);
  // AFX_MFMA_WAVES=4|8|16 overrides when that count also leaves at most four batches
  const int ks = fmt == FMT_I8 || fmt == FMT_BW ? 64 : fmt == FMT_Q4 ? 128 : 32;
  const int nsteps = a.K / ks;
  // Persistent variant (dense <= 16 rows, MoE <= 16 tokens): the most wavefronts (up to 8 for
  // Q4_0, whose x slice takes 64 VGPRs, else 16) that leave each one a single batch;
  // AFX_MFMA_PX=0 disables it, AFX_MFMA_PX_WAVES=4|8|16 caps the wavefronts.
  static int px_env = -2, px_waves = 0, px_depth = 0, px_split = 0;
  if (px_env == -2) {
    const char* s = getenv("AFX_MFMA_SPLIT");
    px_split = s ? atoi(s) : 0;
    const char* e = getenv("AFX_MFMA_PX");
    px_env = e ? atoi(e) : 1;
    const char* w = getenv("AFX_MFMA_PX_WAVES");
    px_waves = w ? atoi(w) : 0;
    const char* d = getenv("AFX_MFMA_PX_DEPTH");
    px_depth = d ? atoi(d) : 0;
  }
  // the persistent kernel reads the bias and the residual four fp16 at a time
  const bool epi_aligned =
      (!a.bias || ((uintptr_t)a.bias & 7) == 0) &&
      (a.epi != EPI_RESID || (((uintptr_t)a.resid & 7) == 0 && a.ldy % 4 == 0 && (long long)a.M * a.ldy * 2 < 0x7fff0000LL));
  if (px_env != 0 && epi_aligned && (a.cnt ? a.T <= 16 && E <= kPxMaxExperts : E == 1 && a.M <= 16)) {
    int cap = fmt == FMT_Q4 ? 8 : 16;
    if (px_waves == 4 || px_waves == 8 || px_waves == 16) cap = px_waves < cap ? px_waves : cap;
    int pw = 0;
    for (int w = cap; w >= 4; w >>= 1)
      if (nsteps >= w && (nsteps + w - 1) / w <= kSPB) { pw = w; break; }
    int S = 1;
    const long long rows = a.cnt ? (long long)a.T * a.k : a.M;
    if (!pw && a.ws && !swiglu && (fmt != FMT_Q4 || a.cnt)) {
      // K slices (2 .. 8) that leave every wavefront one batch, if the workspace holds them; at
      // most 8 wavefronts (16 would spill at their 128-VGPR cap with the slice bookkeeping).
      // Measured on MI355X against the tile kernel: int8 / blockwise 4096 x 11008..14336 at 4..16
      // rows take 17-23 us instead of 21-45, the Q4_0 experts of a 14336-long MoE down ~15%
      // less; a dense Q4_0 4096 x 11008 takes 15 us instead of 12.4, so it keeps the tile kernel.
      const int scap = cap < 8 ? cap : 8;
      for (int s = 2; s <= kMaxSlices && !pw; ++s) {
        const int lmin = nsteps / s, lmax = (nsteps + s - 1) / s;
        if ((long long)s * rows * a.N * 4 > a.ws_bytes) break;
        if (px_split >= 2 && s != px_split) continue;     // AFX_MFMA_SPLIT=2..8: tuning override
        for (int w = scap; w >= 4; w >>= 1)
          if (lmin >= w && (lmax + w - 1) / w <= kSPB) { pw = w; S = s; break; }
      }
    }
    if (pw) {
      b.ks = S;
      b.ws_rows = (int)rows;
      const int ntiles = (a.N + 15) / 16;
      const long long units = (long long)ntiles * E * S;   // MoE: units of empty experts are skipped
      const int grid = units < mfma_cus() ? (int)units : mfma_cus();
      // prefetch depth: three units ahead for long runs of units per workgroup, else one;
      // AFX_MFMA_PX_DEPTH=1|3 overrides
      int pd = (units + grid - 1) / grid >= 6 ? 3 : 1;
      if (px_depth == 1 || px_depth == 3) pd = px_depth;
      if (pw == 16) pd = 1;
      mfma_fn fn = pick_mfma_px(fmt, swiglu, pw, pd, a.cnt != nullptr, S > 1);
      hipLaunchKernelGGL(fn, dim3(grid), dim3(pw * 64), 0, stream, b);
      if (S == 1) return check_launch(what);
      int rc = check_launch(what);
      if (rc) return rc;
      if (ks_out) {                                // the caller sums the slices
        *ks_out = S;
        return 0;
      }
      const long long n = rows * (a.N / 4);
      hipLaunchKernelGGL(mfma_finish_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, b, (int)rows);
      return check_launch(what);
    }
  }
  auto batches = [&](int w) { return ((nsteps + w - 1) / w + kSPB - 1) / kSPB; };
  static int nw_env = -1;
  if (nw_env < 0) {
    const char* e = getenv("AFX_MFMA_WAVES");
    nw_env = e ? atoi(e) : 0;
  }
  int nw = batches(4) <= 4 ? 4 : batches(8) <= 4 ? 8 : 16;
  if ((nw_env == 4 || nw_env == 8 || nw_env == 16) && batches(nw_env) <= 4) nw = nw_env;   // tuning override
  const int nbw = batches(nw) < 4 ? batches(nw) : 4;
  AFX_REQUIRE(nsteps >= nw, "%s: K=%d too short for %d K ranges", what, a.K, nw);
  mfma_fn fn = pick_mfma(fmt, swiglu, nw, nbw);
  hipLaunchKernelGGL(fn, dim3((a.N + 15) / 16, E), dim3(nw * 64), 0, stream, b);
  return check_launch(what);
}

}  // namespace afx
