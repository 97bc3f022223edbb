// Tiled MFMA GEMM for many activation rows (the batched prefill's linears):
//
//   Y[m, n] = epilogue( sum_k X[m, k] * W^[n, k] ),   X fp16 [M][K] (row stride ldx),
//   W int8 codes with an fp16 row scale (W^ = q * s, the compress="int8" linear,
//   aneforge/_compile.py:171-179 and 375-385), int8 codes with an fp16 scale per 32-weight block
//   (compress="blockwise": W^ = fp16(q * s[n][k / 32]), the reference's reconstruction) or fp16 [N][K].
//
// Prefill multiplies the same weights by hundreds or thousands of token rows, so unlike the
// decode GEMV this is a dense contraction that v_mfma_f32_16x16x32_f16 bounds.  A workgroup
// computes a 128 x 128 tile of Y: four wavefronts owning 64 x 64 quarters (fp16 weights) or
// 128 x 32 column strips (int8 codes), 16 MFMA tiles of 16 x 16 each, or, for grids of at most two
// tiles per CU, eight wavefronts owning 64 x 32 (the kernel forms below).  K advances 64 at a time through two LDS
// stages: the next stage's global loads are issued before the current stage's MFMAs and land in
// the other stage afterwards, one barrier per step.  LDS rows are unpadded and XOR-swizzled (below)
// so the 16-byte / 8-byte fragment reads of 16 rows hit distinct banks.
// Fragments: A lane l = row l % 16, k 8 * (l / 16) .. + 7 (activations); B lane l = column
// l % 16 (output feature), same k (weights; int8 codes converted exactly to fp16 in
// registers, the row scale applied to the fp32 result); D lane l = rows 4 * (l / 16) + i,
// column l % 16.
// Tiles are assigned so that each XCD (dispatch is round-robin over the 8 XCDs) owns a range of
// weight tiles, walked in groups of 8 weight tiles with every row tile, weight tile fastest: the
// ~96 workgroups an XCD runs at once then share about 12 activation panels and 8 weight panels
// in its L2, instead of all the activation panels of the prompt.
#include "afx_gemv_impl.h"

namespace afx {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int kGBM = 128, kGBN = 128, kGBK = 64;
constexpr int kGAStride = kGBK * 2;                 // bytes per staged activation row (unpadded, swizzled)

template <int FMT> struct GemmW;
template <> struct GemmW<FMT_I8> { static constexpr int kRow = kGBK, kStride = kGBK, kChunks = 2; };
template <> struct GemmW<FMT_F16> { static constexpr int kRow = kGBK * 2, kStride = kGBK * 2, kChunks = 4; };
template <> struct GemmW<FMT_BW> { static constexpr int kRow = kGBK, kStride = kGBK, kChunks = 2; };

// LDS rows are stored unpadded with their 16-byte chunks (128-byte rows: activations, fp16 weights) or
// 8-byte units (64-byte rows: int8 codes) permuted by an XOR of the row, so that the fragment reads
// of 8 (16-byte) or 16 (8-byte) consecutive rows at one logical offset, and the staging writes, hit
// distinct banks.  Logical chunk c of row r sits at chunk c ^ (r & 7); logical unit u of a code row
// at unit u ^ ((r >> 2) & 7).  (Padding did the same with 144 / 72-byte rows, at 55 KB of LDS per
// workgroup for int8 against 48 KB here, which leaves room for a third workgroup per CU.)
__device__ __forceinline__ int swz16(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }
__device__ __forceinline__ int swz8(int r, int u) { return r * 64 + ((u ^ ((r >> 2) & 7)) << 3); }

struct GemmArgs {
  const void* w;          // [N][K] codes (int8) or values (fp16)
  const half_t* scale;    // int8: [N] row scales; blockwise: [N][K/32] block scales
  const half_t* bias;     // [N] or null
  const half_t* x;        // [M] rows of K, stride ldx
  void* y;                // output rows, stride ldy (fp16, or fp32 for EPI_F32)
  const half_t* resid;    // EPI_RESID: [M][ldy] fp16 (may alias y)
  int ldx, ldy, M, N, K, epi, tiles_m, tiles, per_xcd;
  int tiles_n, gn;        // grouped order (gn > 0): weight tiles per group within an XCD's range
  int x_bytes, w_bytes;   // WL 2: bytes of X and W the buffer loads may read (< 2^31)
};

__device__ __forceinline__ h8 i8x8_to_h8(u2 v) {
  h2 a, b, c, d;
  i8x4_to_h2(v.x, a, b);
  i8x4_to_h2(v.y, c, d);
  h8 r;
  r[0] = a.x; r[1] = a.y; r[2] = b.x; r[3] = b.y; r[4] = c.x; r[5] = c.y; r[6] = d.x; r[7] = d.y;
  return r;
}

// Kernel forms (WL).  0: 2 x 2 wavefronts of 64 x 64 (4 x 4 tiles of 16 x 16), pointer loads.
// 2: 1 x 4 wavefronts of 128 x 32 (8 x 2 tiles), so each weight column is read from LDS and
// converted by one wavefront only (half the int8 conversion work of form 0, more activation
// fragment reads); buffer loads with the step's K offset in a scalar register; the K loop unrolled
// by two so the LDS stage offsets are constants.  Together they cut the int8 loop's VALU from about
// 115 to 41 instructions per K step and wavefront.  (1: form 2's layout with form 0's loads.)
// 3: form 2 with the second half-step's fragments read from LDS between the first half-step's
// MFMAs (each A fragment once its two products are issued), so a K step waits on LDS once, not
// twice, at the same register count (three wavefronts per SIMD).
// 4: form 3's loop with eight wavefronts per workgroup (512 threads) in 2 x 4 tiles of 64 x 32, so a
// CU holding two workgroups (the N = 4096 shapes: 512 tiles) runs four wavefronts per SIMD, not two.
// 6: form 4 with the barrier in the middle of the K step.  The first half-step's products run; the
// next step's tiles are staged into the other stage and the step after next starts loading into the
// freed staging registers (so global loads still get a full step); one barrier publishes the stage;
// and the next step's first fragments are read between the second half-step's products.  No LDS read
// then waits at the top of a step, which pays where a CU holds a single workgroup (tiles <= CUs).
// (The same order over form 3's layout, "form 5", needed 168 VGPRs with spills and measured even with
// form 3; it is not instantiated.)
template <int WL> struct WaveLayout {
  static constexpr bool W8 = WL == 4 || WL == 6;     // eight wavefronts in 2 x 4
  static constexpr bool Q4 = WL == 0;                // four wavefronts in 2 x 2
  static constexpr int MT = W8 ? 4 : (Q4 ? 4 : 8), NT = W8 ? 2 : (Q4 ? 4 : 2);
  static constexpr int NTH = W8 ? 512 : 256;        // threads per workgroup
  static constexpr int WPE = W8 ? 4 : 3;            // wavefronts per SIMD the register budget is sized for
};
template <int V> struct Stage { static constexpr int value = V; };

// Epilogue of a wavefront tile: lane holds rows 4 * fg + i of column fr in every 16 x 16 tile.
template <int FMT, int EG, int MT, int NT>
__device__ __forceinline__ void gemm_store(const GemmArgs& a, const f4 (&acc)[MT][NT], int m0, int n0, int wm, int wn,
                                           int fr, int fg) {
  const int M = a.M, N = a.N;
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int n = n0 + wn * NT * 16 + j * 16 + fr;
    const int nc = n < N ? n : N - 1;
    const float sc = FMT == FMT_I8 ? (float)a.scale[nc] : 1.0f;
    const float bi = a.bias ? (float)a.bias[nc] : 0.0f;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * MT * 16 + i * 16 + 4 * fg + r;
        const float v = acc[i][j][r] * sc + bi;
        if constexpr (EG == EG_SWIGLU) {
          // gate row n (even) and up row n + 1 sit in lanes l and l ^ 1
          const float pv = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false));
          if ((fr & 1) == 0 && m < M && n < N) {
            const float g = (float)(half_t)v, u = (float)(half_t)pv;
            ((half_t*)a.y)[(size_t)m * a.ldy + (n >> 1)] = (half_t)(glu_act(a.epi == EPI_GEGLU, g) * u);
          }
        } else {
          if (m < M && n < N) {
            if (a.epi == EPI_F32) ((float*)a.y)[(size_t)m * a.ldy + n] = v;
            else if (a.epi == EPI_RESID)
              ((half_t*)a.y)[(size_t)m * a.ldy + n] = (half_t)((float)a.resid[(size_t)m * a.ldy + n] + (float)(half_t)v);
            else ((half_t*)a.y)[(size_t)m * a.ldy + n] = (half_t)v;
          }
        }
      }
    }
  }
}

template <int FMT, int EG, int WL>
__global__ __launch_bounds__(WaveLayout<WL>::NTH)
__attribute__((amdgpu_waves_per_eu(WaveLayout<WL>::WPE, WaveLayout<WL>::WPE))) void gemm_kernel(GemmArgs a) {
  constexpr int MT = WaveLayout<WL>::MT, NT = WaveLayout<WL>::NT, NTH = WaveLayout<WL>::NTH;
  constexpr int WS = GemmW<FMT>::kStride, WR = GemmW<FMT>::kRow, WC = GemmW<FMT>::kChunks * 256 / NTH;
  constexpr int AC = 4 * 256 / NTH;                 // 16-byte activation chunks per thread and stage
  constexpr bool kCodes = FMT == FMT_I8 || FMT == FMT_BW;   // one byte per weight
  __shared__ __align__(16) unsigned char As[2][kGBM * kGAStride];
  __shared__ __align__(16) unsigned char Bs[2][kGBN * WS];
  __shared__ uint32_t Ss[2][FMT == FMT_BW ? kGBN : 1];    // blockwise: the 2 block scales of each row's step
  const int id = blockIdx.x;
  int n0, m0;
  if (a.gn > 0) {
    // grouped order: XCD x (id % 8) owns weight tiles [nb, ne), walked in groups of gn weight tiles
    // with every row tile; inside a group the weight tile is fastest, so the workgroups an XCD runs
    // at once cover about (concurrent / gn) row tiles x gn weight tiles of L2-resident operands
    const int x = id & 7, l = id >> 3;
    const int nb = (a.tiles_n * x) >> 3, ne = (a.tiles_n * (x + 1)) >> 3;
    if (l >= (ne - nb) * a.tiles_m) return;         // whole workgroup: no barrier reached
    const int span = a.gn * a.tiles_m;
    const int g = l / span, r = l - g * span;
    const int gs = ne - nb - g * a.gn < a.gn ? ne - nb - g * a.gn : a.gn;
    n0 = (nb + g * a.gn + r % gs) * kGBN;
    m0 = (r / gs) * kGBM;
  } else {
    // tile: the XCD (id % 8) gets a contiguous range of logical tiles, row tiles fastest
    const int logical = (id & 7) * a.per_xcd + (id >> 3);
    if (logical >= a.tiles) return;                 // whole workgroup: no barrier reached
    n0 = (logical / a.tiles_m) * kGBN;
    m0 = (logical % a.tiles_m) * kGBM;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr bool W8 = WaveLayout<WL>::W8, Q4 = WaveLayout<WL>::Q4;
  const int wm = W8 ? wave >> 2 : (Q4 ? wave >> 1 : 0), wn = W8 ? wave & 3 : (Q4 ? wave & 1 : wave);
  const int M = a.M, N = a.N, K = a.K;
  const int nk = K / kGBK;

  // global-load roles: activations 4 x 16 B per thread (row c / 8, chunk c % 8), weights WC x 16 B
  const half_t* xp[AC];
  int aoff[AC];
#pragma unroll
  for (int i = 0; i < AC; ++i) {
    const int c = tid + NTH * i, r = c >> 3, ch = c & 7;
    const int m = m0 + r < M ? m0 + r : M - 1;     // clamped rows are computed, not stored
    xp[i] = a.x + (size_t)m * a.ldx + ch * 8;
    aoff[i] = swz16(r, ch);
  }
  const unsigned char* wp[WC];
  int boff[WC], boff2[WC];
#pragma unroll
  for (int i = 0; i < WC; ++i) {
    const int c = tid + NTH * i;
    const int r = kCodes ? c >> 2 : c >> 3, ch = kCodes ? c & 3 : c & 7;
    const int n = n0 + r < N ? n0 + r : N - 1;
    wp[i] = (const unsigned char*)a.w + (size_t)n * (kCodes ? K : 2 * K) + ch * 16;
    boff[i] = kCodes ? swz8(r, 2 * ch) : swz16(r, ch);   // codes: the chunk's two 8-byte units
    boff2[i] = kCodes ? swz8(r, 2 * ch + 1) : 0;
  }
  const half_t* sp = nullptr;                       // blockwise: thread t < 128 carries row n0 + t's scales
  if constexpr (FMT == FMT_BW) {
    const int n = n0 + (tid & 127) < N ? n0 + (tid & 127) : N - 1;
    sp = a.scale + (size_t)n * (K >> 5);
  }
  u4 ra[AC], rb[WC];
  uint32_t rs = 0;
  // WL 2: buffer loads over the whole X and W (byte offsets fit 31 bits, checked by the host), the
  // per-lane offset fixed and the step's K offset a scalar, so a step's loads take no address VALU
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, a.x_bytes), wr = make_rsrc(a.w, a.w_bytes);
  int xo[AC], wo[WC];
  if constexpr (WL >= 2) {
#pragma unroll
    for (int i = 0; i < AC; ++i) xo[i] = (int)((const unsigned char*)xp[i] - (const unsigned char*)a.x);
#pragma unroll
    for (int i = 0; i < WC; ++i) wo[i] = (int)(wp[i] - (const unsigned char*)a.w);
  }
  auto load = [&](int kt) {
    if constexpr (WL >= 2) {
#pragma unroll
      for (int i = 0; i < AC; ++i)
        ra[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(xr, xo[i], kt * (kGBK * 2), 0));
#pragma unroll
      for (int i = 0; i < WC; ++i)
        rb[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wr, wo[i], kt * WR, 0));
    } else {
#pragma unroll
      for (int i = 0; i < AC; ++i) ra[i] = *(const u4*)(xp[i] + (size_t)kt * kGBK);
#pragma unroll
      for (int i = 0; i < WC; ++i) rb[i] = *(const u4*)(wp[i] + (size_t)kt * WR);
    }
    if constexpr (FMT == FMT_BW) rs = *(const uint32_t*)(sp + 2 * kt);
  };
  auto stage = [&](int s) {
    if constexpr (FMT == FMT_BW) {
      if (tid < kGBN) Ss[s][tid] = rs;
    }
#pragma unroll
    for (int i = 0; i < AC; ++i) *(u4*)(As[s] + aoff[i]) = ra[i];
#pragma unroll
    for (int i = 0; i < WC; ++i) {
      if constexpr (kCodes) {                      // the two 8-byte units land apart after the swizzle
        *(u2*)(Bs[s] + boff[i]) = (u2){rb[i].x, rb[i].y};
        *(u2*)(Bs[s] + boff2[i]) = (u2){rb[i].z, rb[i].w};
      } else {
        *(u4*)(Bs[s] + boff[i]) = rb[i];
      }
    }
  };

  f4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

  load(0);
  stage(0);
  if constexpr (WL == 6) {
    if (nk > 1) load(1);                           // the mid-step form keeps one step of loads in flight
  }
  __syncthreads();
  const int fr = lane & 15, fg = lane >> 4;
  // one K step on stage s: the next stage's loads, this stage's MFMAs, then the next stage staged
  auto kstep = [&](int kt, auto st) {
    const int s = decltype(st)::value >= 0 ? decltype(st)::value : (kt & 1);
    if (kt + 1 < nk) load(kt + 1);                 // next stage streams during this stage's MFMAs
    if constexpr (WL >= 3) {
      // the second half-step's fragments are read between the first half-step's MFMAs, each A fragment
      // as soon as its two products have been issued, so only the first half-step waits on LDS
      typedef typename std::conditional<kCodes, u2, u4>::type Raw;
      auto read_a = [&](int kk, int i) {
        return __builtin_bit_cast(h8, *(const u4*)(As[s] + swz16(wm * MT * 16 + i * 16 + fr, kk * 4 + fg)));
      };
      auto read_b = [&](int kk, int j) -> Raw {
        const int br = wn * NT * 16 + j * 16 + fr;
        if constexpr (kCodes) return *(const u2*)(Bs[s] + swz8(br, kk * 4 + fg));
        else return *(const u4*)(Bs[s] + swz16(br, kk * 4 + fg));
      };
      auto conv_b = [&](int kk, int j, Raw r) -> h8 {
        if constexpr (FMT == FMT_I8) {
          return i8x8_to_h8(r);
        } else if constexpr (FMT == FMT_BW) {
          const h2 sp2 = as_h2(Ss[s][wn * NT * 16 + j * 16 + fr]);
          const half_t sc = kk ? sp2.y : sp2.x;
          const h8 s8 = {sc, sc, sc, sc, sc, sc, sc, sc};
          return i8x8_to_h8(r) * s8;
        } else {
          return __builtin_bit_cast(h8, r);
        }
      };
      h8 af[MT];
      Raw bq[NT];
#pragma unroll
      for (int i = 0; i < MT; ++i) af[i] = read_a(0, i);
#pragma unroll
      for (int j = 0; j < NT; ++j) bq[j] = read_b(0, j);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        h8 bf[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) bf[j] = conv_b(kk, j, bq[j]);
        if (kk == 0)
#pragma unroll
          for (int j = 0; j < NT; ++j) bq[j] = read_b(1, j);
        if constexpr (FMT != FMT_BW) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
#pragma unroll
          for (int j = 0; j < NT; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
          if (kk == 0) af[i] = read_a(1, i);
        }
        if constexpr (FMT != FMT_BW) __builtin_amdgcn_s_setprio(0);
      }
    } else {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      h8 af[MT], bf[NT];
#pragma unroll
      for (int i = 0; i < MT; ++i)
        af[i] = __builtin_bit_cast(h8, *(const u4*)(As[s] + swz16(wm * MT * 16 + i * 16 + fr, kk * 4 + fg)));
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int br = wn * NT * 16 + j * 16 + fr;
        if constexpr (FMT == FMT_I8) {
          bf[j] = i8x8_to_h8(*(const u2*)(Bs[s] + swz8(br, kk * 4 + fg)));
        } else if constexpr (FMT == FMT_BW) {       // k 32kk .. 32kk + 31 is block kk of the step
          const h2 sp2 = as_h2(Ss[s][br]);
          const half_t sc = kk ? sp2.y : sp2.x;
          const h8 s8 = {sc, sc, sc, sc, sc, sc, sc, sc};
          bf[j] = i8x8_to_h8(*(const u2*)(Bs[s] + swz8(br, kk * 4 + fg))) * s8;   // fp16(q * s)
        } else {
          bf[j] = __builtin_bit_cast(h8, *(const u4*)(Bs[s] + swz16(br, kk * 4 + fg)));
        }
      }
      // raised wave priority over the MFMA cluster: a wavefront that has its fragments keeps the matrix
      // pipe fed ahead of the others' loads and conversions (int8: +0.5-1.9% on the 7B prefill shapes,
      // +0.7% on the whole cfg3 prefill, MI355X); blockwise, whose fragments take a scale multiply
      // each, measured 0.5% slower with it and keeps the default priority
      if constexpr (FMT != FMT_BW) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
      if constexpr (FMT != FMT_BW) __builtin_amdgcn_s_setprio(0);
    }
    }
    if (kt + 1 < nk) stage(s ^ 1);                 // the other stage was last read before the previous barrier
    __syncthreads();
  };
  if constexpr (WL == 6) {
    typedef typename std::conditional<kCodes, u2, u4>::type Raw;
    auto read_a = [&](int s, int kk, int i) {
      return __builtin_bit_cast(h8, *(const u4*)(As[s] + swz16(wm * MT * 16 + i * 16 + fr, kk * 4 + fg)));
    };
    auto read_b = [&](int s, int kk, int j) -> Raw {
      const int br = wn * NT * 16 + j * 16 + fr;
      if constexpr (kCodes) return *(const u2*)(Bs[s] + swz8(br, kk * 4 + fg));
      else return *(const u4*)(Bs[s] + swz16(br, kk * 4 + fg));
    };
    auto conv_b = [&](int s, int kk, int j, Raw r) -> h8 {
      if constexpr (FMT == FMT_I8) {
        return i8x8_to_h8(r);
      } else if constexpr (FMT == FMT_BW) {
        const h2 sp2 = as_h2(Ss[s][wn * NT * 16 + j * 16 + fr]);
        const half_t sc = kk ? sp2.y : sp2.x;
        const h8 s8 = {sc, sc, sc, sc, sc, sc, sc, sc};
        return i8x8_to_h8(r) * s8;
      } else {
        return __builtin_bit_cast(h8, r);
      }
    };
    h8 af[MT];
    Raw bq[NT];
#pragma unroll
    for (int i = 0; i < MT; ++i) af[i] = read_a(0, 0, i);
#pragma unroll
    for (int j = 0; j < NT; ++j) bq[j] = read_b(0, 0, j);
    auto mstep = [&](int kt, auto st) {
      constexpr int s = decltype(st)::value;
      const bool more = kt + 1 < nk;               // uniform over the workgroup
      h8 bf[NT];
      // first half-step: kk 0's products, kk 1's fragments read between them
#pragma unroll
      for (int j = 0; j < NT; ++j) bf[j] = conv_b(s, 0, j, bq[j]);
#pragma unroll
      for (int j = 0; j < NT; ++j) bq[j] = read_b(s, 1, j);
      if constexpr (FMT != FMT_BW) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        af[i] = read_a(s, 1, i);
      }
      if constexpr (FMT != FMT_BW) __builtin_amdgcn_s_setprio(0);
      // the next step's tiles into the other stage (last read before the previous barrier), the step
      // after next loading into the freed registers, one barrier
      if (more) stage(s ^ 1);
      if (kt + 2 < nk) load(kt + 2);
      if (more) __syncthreads();
      // second half-step: kk 1's products, the next step's kk 0 fragments read between them
#pragma unroll
      for (int j = 0; j < NT; ++j) bf[j] = conv_b(s, 1, j, bq[j]);
      if (more)
#pragma unroll
        for (int j = 0; j < NT; ++j) bq[j] = read_b(s ^ 1, 0, j);
      if constexpr (FMT != FMT_BW) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        if (more) af[i] = read_a(s ^ 1, 0, i);
      }
      if constexpr (FMT != FMT_BW) __builtin_amdgcn_s_setprio(0);
    };
    for (int kt = 0; kt < nk; kt += 2) {           // unrolled by two: the stage offsets are constants
      mstep(kt, Stage<0>{});
      if (kt + 1 < nk) mstep(kt + 1, Stage<1>{});
    }
  } else if constexpr (WL >= 2) {                  // unrolled by two: the stage offsets are constants
    for (int kt = 0; kt < nk; kt += 2) {
      kstep(kt, Stage<0>{});
      if (kt + 1 < nk) kstep(kt + 1, Stage<1>{});
    }
  } else {
    for (int kt = 0; kt < nk; ++kt) kstep(kt, Stage<-1>{});
  }

  gemm_store<FMT, EG, MT, NT>(a, acc, m0, n0, wm, wn, fr, fg);
}

typedef void (*gemm_fn)(GemmArgs);

}  // namespace afx

using namespace afx;

extern "C" {

// Y = epilogue(X @ W^T) for M activation rows (batched prefill).  fmt: 0 = int8 + row scale,
// 2 = fp16, 3 = int8 + fp16 scale per 32-weight block.  epi: 0 fp16, 1 fp16 + residual (resid [M][ldy], may alias y), 2 fp32, 3 SwiGLU
// over interleaved gate/up rows (y[m][n/2] = silu(g) * u, ldy >= N/2), 5 GeGLU (the same with gelu_tanh(g)).
int afx_gemm(int fmt, const void* w, const void* scale, const void* x, int ldx, void* y, int ldy, int M, int N,
             int K, const void* bias, const void* residual, int epi, void* stream) {
  AFX_REQUIRE(fmt == FMT_I8 || fmt == FMT_F16 || fmt == FMT_BW,
              "afx_gemm: format %d not supported (int8 = 0, fp16 = 2, blockwise = 3)", fmt);
  AFX_REQUIRE(w && x && y, "afx_gemm: null pointer");
  AFX_REQUIRE(M >= 1 && N >= 16 && N % 16 == 0 && K >= kGBK && K % kGBK == 0,
              "afx_gemm: need M >= 1, N %% 16 == 0, K %% 64 == 0 (M=%d N=%d K=%d)", M, N, K);
  AFX_REQUIRE(ldx >= K && ldx % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0,
              "afx_gemm: x and weights must be 16-byte aligned rows (ldx %% 8 == 0)");
  AFX_REQUIRE((epi >= 0 && epi <= 3) || epi == EPI_GEGLU, "afx_gemm: unknown epilogue %d", epi);
  const bool glu = epi == EPI_SWIGLU || epi == EPI_GEGLU;
  AFX_REQUIRE(fmt != FMT_I8 || scale, "afx_gemm: int8 weights need row scales");
  AFX_REQUIRE(fmt != FMT_BW || (scale && ((uintptr_t)scale & 3) == 0), "afx_gemm: blockwise weights need aligned block scales");
  AFX_REQUIRE(epi != EPI_RESID || residual, "afx_gemm: residual pointer required");
  AFX_REQUIRE(glu ? ldy >= N / 2 : ldy >= N, "afx_gemm: ldy=%d too small", ldy);
  GemmArgs a = {};
  a.w = w; a.scale = (const half_t*)scale; a.bias = (const half_t*)bias; a.x = (const half_t*)x; a.y = y;
  a.resid = (const half_t*)residual; a.ldx = ldx; a.ldy = ldy; a.M = M; a.N = N; a.K = K; a.epi = epi;
  a.tiles_m = (M + kGBM - 1) / kGBM;
  a.tiles = a.tiles_m * ((N + kGBN - 1) / kGBN);
  a.per_xcd = (a.tiles + 7) / 8;
  a.tiles_n = (N + kGBN - 1) / kGBN;
  // tile order: groups of 8 weight tiles per XCD (AFX_GEMM_GN overrides; 0 = the row-tiles-fastest
  // contiguous order).  At M = 2048 on the 7B shapes, against the contiguous order: gate/up 900 -> 947,
  // down 798 -> 815 TFLOP/s, o-proj and QKV within noise; outputs bit-identical.
  const char* ge = getenv("AFX_GEMM_GN");            // read per call: tests compare the orders in one process
  const int gn_env = ge ? atoi(ge) : 8;
  a.gn = gn_env > 0 ? gn_env : 0;
  if (a.gn > 0) a.per_xcd = ((a.tiles_n + 7) / 8) * a.tiles_m;   // the largest XCD range
  // kernel form (outputs are bit-identical across forms): int8 codes take form 6 when the tiles fit one
  // workgroup per CU (N = 4096 at M = 1000: o-proj 57.2 -> 53.3 us, down 130.3 -> 120.9 us against form
  // 4), form 4 when they fit two (the N = 4096 shapes at M = 2048: o-proj 95.5 -> 85.9 us, down 208.6 ->
  // 201.2 us against form 3) and form 3 otherwise (gate/up, QKV at M = 2048; form 2 -> 3 there: QKV 874 ->
  // 930, gate/up 966 -> 994 TFLOP/s); blockwise takes form 2 (form 3 even, form 4 slower); fp16 weights
  // take form 6 (eight wavefronts without the AGPR spill-over of the four-wavefront fp16 forms, which
  // leaves them at one or two wavefronts per SIMD: at M = 2048 against form 0, QKV 137.7 -> 125.3,
  // gate/up 470.0 -> 422.6, down 234.8 -> 214.1 us).  AFX_GEMM_WL=0|2|3|4|6 overrides.  Forms 2-6 address
  // X and W with 31-bit buffer offsets, so larger operands take form 0.
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
  }
  const char* we = getenv("AFX_GEMM_WL");           // read per call, like AFX_GEMM_GN
  const int wl_env = we ? atoi(we) : -1;
  const int wl = wl_env >= 0 ? wl_env : (fmt == FMT_I8 ? (a.tiles <= cus ? 6 : a.tiles <= 2 * cus ? 4 : 3) : fmt == FMT_BW ? 2 : 6);
  const long long xb = ((long long)(M - 1) * ldx + K) * 2;
  const long long wb = (long long)N * K * (fmt == FMT_F16 ? 2 : 1);
  const bool form2 = (wl == 2 || wl == 3 || wl == 4 || wl == 6) && xb < (1ll << 31) && wb < (1ll << 31);
  gemm_fn fn;
  int nth = 256;
  if (form2 && wl == 6) {
    a.x_bytes = (int)xb;
    a.w_bytes = (int)wb;
    nth = 512;
    if (fmt == FMT_I8) fn = glu ? gemm_kernel<FMT_I8, EG_SWIGLU, 6> : gemm_kernel<FMT_I8, EG_PLAIN, 6>;
    else if (fmt == FMT_BW) fn = glu ? gemm_kernel<FMT_BW, EG_SWIGLU, 6> : gemm_kernel<FMT_BW, EG_PLAIN, 6>;
    else fn = glu ? gemm_kernel<FMT_F16, EG_SWIGLU, 6> : gemm_kernel<FMT_F16, EG_PLAIN, 6>;
  } else if (form2 && wl == 4) {
    a.x_bytes = (int)xb;
    a.w_bytes = (int)wb;
    nth = 512;
    if (fmt == FMT_I8) fn = glu ? gemm_kernel<FMT_I8, EG_SWIGLU, 4> : gemm_kernel<FMT_I8, EG_PLAIN, 4>;
    else if (fmt == FMT_BW) fn = glu ? gemm_kernel<FMT_BW, EG_SWIGLU, 4> : gemm_kernel<FMT_BW, EG_PLAIN, 4>;
    else fn = glu ? gemm_kernel<FMT_F16, EG_SWIGLU, 4> : gemm_kernel<FMT_F16, EG_PLAIN, 4>;
  } else if (form2 && wl == 3) {
    a.x_bytes = (int)xb;
    a.w_bytes = (int)wb;
    if (fmt == FMT_I8) fn = glu ? gemm_kernel<FMT_I8, EG_SWIGLU, 3> : gemm_kernel<FMT_I8, EG_PLAIN, 3>;
    else if (fmt == FMT_BW) fn = glu ? gemm_kernel<FMT_BW, EG_SWIGLU, 3> : gemm_kernel<FMT_BW, EG_PLAIN, 3>;
    else fn = glu ? gemm_kernel<FMT_F16, EG_SWIGLU, 3> : gemm_kernel<FMT_F16, EG_PLAIN, 3>;
  } else if (form2) {
    a.x_bytes = (int)xb;
    a.w_bytes = (int)wb;
    if (fmt == FMT_I8) fn = glu ? gemm_kernel<FMT_I8, EG_SWIGLU, 2> : gemm_kernel<FMT_I8, EG_PLAIN, 2>;
    else if (fmt == FMT_BW) fn = glu ? gemm_kernel<FMT_BW, EG_SWIGLU, 2> : gemm_kernel<FMT_BW, EG_PLAIN, 2>;
    else fn = glu ? gemm_kernel<FMT_F16, EG_SWIGLU, 2> : gemm_kernel<FMT_F16, EG_PLAIN, 2>;
  } else {
    if (fmt == FMT_I8) fn = glu ? gemm_kernel<FMT_I8, EG_SWIGLU, 0> : gemm_kernel<FMT_I8, EG_PLAIN, 0>;
    else if (fmt == FMT_BW) fn = glu ? gemm_kernel<FMT_BW, EG_SWIGLU, 0> : gemm_kernel<FMT_BW, EG_PLAIN, 0>;
    else fn = glu ? gemm_kernel<FMT_F16, EG_SWIGLU, 0> : gemm_kernel<FMT_F16, EG_PLAIN, 0>;
  }
  hipLaunchKernelGGL(fn, dim3(8 * a.per_xcd), dim3(nth), 0, (hipStream_t)stream, a);
  return check_launch("afx_gemm");
}

}  // extern "C"
