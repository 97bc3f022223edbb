// Weight codecs on the device: GGUF Q4_0 <-> the superblock layout the GEMV streams, and
// "debug" dequantisers that run the exact same in-register unpack as the GEMV kernels and
// write the dequantised weights as fp32, so the host can check them bit-for-bit.
//
// GGUF Q4_0 block (ggml block_q4_0; decoded on the host by the reference through the
// third-party `gguf` package, aneforge/_gguf.py:34-39): 18 bytes = fp16 d + 16 bytes qs;
// element i (i < 16) is (qs[i] & 15) - 8, element i+16 is (qs[i] >> 4) - 8, value = elem * d.
//
// Superblock layout (this library): per row, K/128 superblocks of 64 bytes.  The 32-bit word
// at index (row*(K/128) + sb)*16 + g*4 + j holds elements 8g..8g+7 of block 4*sb+j, with
// the even elements' nibbles in bits 0,4,8,12 and the odd elements' in bits 16,20,24,28
// (see q4_word_to_h2).  A 16-byte load at offset 16g of a superblock therefore yields word g
// of four consecutive blocks - exactly one MFMA B-operand slot per block, and 32 weights for
// the dot2 GEMV.  Block scales stay row-major: d[row][K/32].
#include "afx_gemv_core.h"

namespace afx {

__global__ void q4_repack_kernel(const uint8_t* __restrict__ blocks, uint32_t* __restrict__ qs,
                                 half_t* __restrict__ d, int N, int K) {
  const int nb = K >> 5;
  const long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= (long long)N * nb) return;
  const int row = (int)(b / nb), blk = (int)(b - (long long)row * nb);
  const uint8_t* src = blocks + b * 18;
  uint16_t dbits = (uint16_t)src[0] | ((uint16_t)src[1] << 8);
  d[(size_t)row * nb + blk] = __builtin_bit_cast(half_t, dbits);
  uint8_t e[32];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    e[i] = src[2 + i] & 15;
    e[i + 16] = src[2 + i] >> 4;
  }
  const int sb = blk >> 2, j = blk & 3;
  uint32_t* dst = qs + ((size_t)row * (K >> 7) + sb) * 16;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    uint32_t w = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      w |= (uint32_t)e[8 * g + 2 * t] << (4 * t);
      w |= (uint32_t)e[8 * g + 2 * t + 1] << (16 + 4 * t);
    }
    dst[g * 4 + j] = w;
  }
}

__global__ void q4_unpack_kernel(const uint32_t* __restrict__ qs, const half_t* __restrict__ d,
                                 uint8_t* __restrict__ blocks, int N, int K) {
  const int nb = K >> 5;
  const long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= (long long)N * nb) return;
  const int row = (int)(b / nb), blk = (int)(b - (long long)row * nb);
  const int sb = blk >> 2, j = blk & 3;
  const uint32_t* src = qs + ((size_t)row * (K >> 7) + sb) * 16;
  uint8_t e[32];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t w = src[g * 4 + j];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      e[8 * g + 2 * t] = (w >> (4 * t)) & 15;
      e[8 * g + 2 * t + 1] = (w >> (16 + 4 * t)) & 15;
    }
  }
  uint8_t* dst = blocks + b * 18;
  const uint16_t dbits = __builtin_bit_cast(uint16_t, d[(size_t)row * nb + blk]);
  dst[0] = dbits & 255;
  dst[1] = dbits >> 8;
#pragma unroll
  for (int i = 0; i < 16; ++i) dst[2 + i] = (uint8_t)(e[i] | (e[i + 16] << 4));
}

// GGUF Q4_K super-block (ggml block_q4_K, 144 B: fp16 d, fp16 dmin, 12 bytes of 6-bit scales and
// mins, 128 code bytes) -> codes [N][K/2] (the 128 code bytes as they are) + 5 dwords per
// super-block in hdr [N][K/256][5]: {d | dmin << 16}, then {sc(2p), sc(2p+1), m(2p), m(2p+1)} for
// pairs p = 0..3.  The 12-byte field: j < 4: sc = b[j] & 63, m = b[j + 4] & 63; j >= 4: sc =
// (b[j + 4] & 15) | (b[j - 4] >> 6) << 4, m = (b[j + 4] >> 4) | (b[j] >> 6) << 4.
__device__ __forceinline__ void k4_scale_min(const uint8_t* b, int j, uint32_t& sc, uint32_t& m) {
  if (j < 4) {
    sc = b[j] & 63;
    m = b[j + 4] & 63;
  } else {
    sc = (b[j + 4] & 15) | ((b[j - 4] >> 6) << 4);
    m = (b[j + 4] >> 4) | ((b[j] >> 6) << 4);
  }
}

__global__ void q4k_repack_kernel(const uint8_t* __restrict__ blocks, uint8_t* __restrict__ qs,
                                  uint32_t* __restrict__ hdr, int N, int K) {
  const int nb = K >> 8;
  const long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= (long long)N * nb) return;
  const uint8_t* src = blocks + b * 144;
  uint32_t* h = hdr + b * 5;                     // row-major over (row, super-block)
  h[0] = (uint32_t)src[0] | ((uint32_t)src[1] << 8) | ((uint32_t)src[2] << 16) | ((uint32_t)src[3] << 24);
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    uint32_t s0, m0, s1, m1;
    k4_scale_min(src + 4, 2 * p, s0, m0);
    k4_scale_min(src + 4, 2 * p + 1, s1, m1);
    h[1 + p] = s0 | (s1 << 8) | (m0 << 16) | (m1 << 24);
  }
  uint8_t* dst = qs + b * 128;
#pragma unroll
  for (int i = 0; i < 128; ++i) dst[i] = src[16 + i];
}

// Q4_K weights as T rows out[n * ldo + k]: one thread per code dword (elements 4 apart in two
// runs 32 apart), through the GEMV's own Fmt<FMT_Q4K> arithmetic.
template <typename T>
__global__ void dequant_q4k_kernel(const uint32_t* __restrict__ qs, const uint32_t* __restrict__ hdr,
                                   T* __restrict__ out, long long ldo, int N, int K) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const int per = K >> 3;                        // code dwords per row
  if (i >= (long long)N * per) return;
  const int row = (int)(i / per), w = (int)(i - (long long)row * per);
  const int sb = w >> 5, b0 = 4 * (w & 31), p = b0 >> 5, l0 = b0 & 31;
  const uint32_t* h = hdr + ((size_t)row * (K >> 8) + sb) * 5;
  const h2 dd = as_h2(h[0]);
  const uint32_t sm = h[1 + p];
  const float dsa = (float)dd.x * ubyte_f32(sm, 0), dsb = (float)dd.x * ubyte_f32(sm, 1);
  const float dma = (float)dd.y * ubyte_f32(sm, 2), dmb = (float)dd.y * ubyte_f32(sm, 3);
  const uint32_t q = qs[i], lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
  T* o = out + (size_t)row * ldo + 256 * sb + 64 * p + l0;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    o[t] = (T)(half_t)__builtin_fmaf(dsa, ubyte_f32(lo, t), -dma);
    o[32 + t] = (T)(half_t)__builtin_fmaf(dsb, ubyte_f32(hi, t), -dmb);
  }
}

// GGUF Q6_K super-block (ggml block_q6_K, 210 B: ql[128], qh[64], int8 scales[16], fp16 d) -> the
// chunked layout of Fmt<FMT_Q6K>: codes [N][K/2] (per 32-weight chunk, code dword k byte j = low
// nibbles of elements 8k + j and 8k + 4 + j) + 3 side dwords per chunk in sw [N][K/32][3].  In the
// ggml block, element e = 128h + 32s + l takes its low 4 bits from nibble s >> 1 of ql[64h + 32(s & 1)
// + l], its high 2 bits from bits 2s..2s+1 of qh[32h + l], and scale e / 16.
__global__ void q6k_repack_kernel(const uint8_t* __restrict__ blocks, uint32_t* __restrict__ qs,
                                  uint32_t* __restrict__ sw, int N, int K) {
  const long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= (long long)N * (K >> 8)) return;
  const uint8_t* src = blocks + b * 210;
  auto lo4 = [&](int e) -> uint32_t {
    const int h = e >> 7, s = (e >> 5) & 3, l = e & 31;
    return (src[64 * h + 32 * (s & 1) + l] >> (4 * (s >> 1))) & 15u;
  };
  auto hi2 = [&](int e) -> uint32_t {
    const int h = e >> 7, s = (e >> 5) & 3, l = e & 31;
    return (src[128 + 32 * h + l] >> (2 * s)) & 3u;
  };
  const uint32_t dbits = (uint32_t)src[208] | ((uint32_t)src[209] << 8);
  uint32_t* q = qs + b * 32;                       // 8 chunks x 4 dwords
  uint32_t* w = sw + b * 24;                       // 8 chunks x 3 dwords
  for (int c = 0; c < 8; ++c) {
    const int e0 = 32 * c;
    for (int k = 0; k < 4; ++k) {
      uint32_t v = 0;
      for (int j = 0; j < 4; ++j) v |= (lo4(e0 + 8 * k + j) | (lo4(e0 + 8 * k + 4 + j) << 4)) << (8 * j);
      q[4 * c + k] = v;
    }
    for (int p = 0; p < 2; ++p) {
      uint32_t v = 0;
      for (int j = 0; j < 4; ++j) {
        const int f = e0 + 16 * p + j;
        v |= (hi2(f) | (hi2(f + 4) << 2) | (hi2(f + 8) << 4) | (hi2(f + 12) << 6)) << (8 * j);
      }
      w[3 * c + p] = v;
    }
    w[3 * c + 2] = (uint32_t)src[192 + (e0 >> 4)] | ((uint32_t)src[192 + (e0 >> 4) + 1] << 8) | (dbits << 16);
  }
}

// Q6_K weights as T rows out[n * ldo + k]: one thread per code dword, the Fmt<FMT_Q6K> arithmetic.
template <typename T>
__global__ void dequant_q6k_kernel(const uint32_t* __restrict__ qs, const uint32_t* __restrict__ sw,
                                   T* __restrict__ out, long long ldo, int N, int K) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const int per = K >> 3;
  if (i >= (long long)N * per) return;
  const int row = (int)(i / per), w = (int)(i - (long long)row * per);
  const int c = w >> 2, k = w & 3;
  const uint32_t* s3 = sw + ((size_t)row * (K >> 5) + c) * 3;
  const float dsup = (float)as_h2(s3[2]).y;
  const float ds = dsup * (float)(int8_t)((s3[2] >> (k < 2 ? 0 : 8)) & 0xFFu);
  const uint32_t H = s3[k >> 1], q = qs[i];
  const uint32_t lo = (q & 0x0F0F0F0Fu) | ((k & 1 ? H : H << 4) & 0x30303030u);
  const uint32_t hi = ((q >> 4) & 0x0F0F0F0Fu) | ((k & 1 ? H >> 2 : H << 2) & 0x30303030u);
  T* o = out + (size_t)row * ldo + 32 * c + 8 * k;
  // gguf-py's product (d*sc) * (q - 32), bit for bit including the sign of a zero weight (the GEMV's
  // fma form gives +0 where this gives -0, which changes no product with x).  The empty asm keeps
  // the product a v_mul_f32: fused into a v_fma_mix with a +0 addend it would turn -0 into +0.
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    float a = ds * (ubyte_f32(lo, t) - 32.0f), b = ds * (ubyte_f32(hi, t) - 32.0f);
    asm("" : "+v"(a), "+v"(b));
    o[t] = (T)(half_t)a;
    o[4 + t] = (T)(half_t)b;
  }
}

// out[n][k] = code * scale as fp32, through the GEMV's own unpack helpers.
__global__ void dequant_i8_kernel(const uint32_t* __restrict__ q, const half_t* __restrict__ s,
                                  float* __restrict__ out, int N, int K) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;   // one dword = 4 codes
  const long long nw = (long long)N * (K >> 2);
  if (i >= nw) return;
  const int row = (int)(i / (K >> 2));
  h2 lo, hi;
  i8x4_to_h2(q[i], lo, hi);
  const float sc = (float)s[row];
  float4 o = {(float)lo.x * sc, (float)lo.y * sc, (float)hi.x * sc, (float)hi.y * sc};
  *(float4*)(out + 4 * i) = o;
}

// compress="blockwise": fp16(q * s[row][k / 32]) -- the reference's reconstructed weight.
__global__ void dequant_bw_kernel(const uint32_t* __restrict__ q, const half_t* __restrict__ s,
                                  float* __restrict__ out, int N, int K) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;   // one dword = 4 codes
  const long long nw = (long long)N * (K >> 2);
  if (i >= nw) return;
  const int row = (int)(i / (K >> 2)), k0 = (int)(i - (long long)row * (K >> 2)) * 4;
  h2 lo, hi;
  i8x4_to_h2(q[i], lo, hi);
  const half_t sc = s[(size_t)row * (K >> 5) + (k0 >> 5)];
  const h2 s2 = {sc, sc};
  lo = lo * s2;
  hi = hi * s2;
  float4 o = {(float)lo.x, (float)lo.y, (float)hi.x, (float)hi.y};
  *(float4*)(out + 4 * i) = o;
}

__global__ void dequant_q4_kernel(const uint32_t* __restrict__ qs, const half_t* __restrict__ d,
                                  float* __restrict__ out, int N, int K) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;   // one word = 8 elements
  const long long nw = (long long)N * (K >> 3);
  if (i >= nw) return;
  const int wpr = K >> 3;
  const int row = (int)(i / wpr), w = (int)(i - (long long)row * wpr);
  const int sb = w >> 4, g = (w >> 2) & 3, j = w & 3;
  const int blk = 4 * sb + j;
  h2 v[4];
  q4_word_to_h2(qs[i], v);
  const float sc = (float)d[(size_t)row * (K >> 5) + blk];
  float* o = out + (size_t)row * K + 32 * blk + 8 * g;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    o[2 * t] = (float)v[t].x * sc;
    o[2 * t + 1] = (float)v[t].y * sc;
  }
}

// Weights as fp16 rows out[n * ldo + k], the values the GEMV / MFMA kernels multiply with:
// int8 fp16(q * s[n]); Q4_0 fp16((nibble - 8) * d) (the reference's GGUF fp16 weights);
// blockwise fp16(q * s[n][k / 32]).  One thread per 8 weights, one 16-byte store.
// compress="int4": codebook[row][index]; one thread per 8 columns (4 bytes of indices).
template <typename T>
__global__ void dequant_l4_kernel(const uint32_t* __restrict__ idx, const half_t* __restrict__ cb,
                                  T* __restrict__ out, long long ldo, int N, int K) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const int per = K >> 3;
  if (i >= (long long)N * per) return;
  const int row = (int)(i / per), c = (int)(i - (long long)row * per);
  const uint32_t w = idx[i];
  cb += 16 * (size_t)row;
  T* o = out + (size_t)row * ldo + 8 * c;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    o[2 * b] = (T)cb[(w >> (8 * b)) & 15];
    o[2 * b + 1] = (T)cb[(w >> (8 * b + 4)) & 15];
  }
}

template <int FMT>
__global__ void dequant_f16_kernel(const void* __restrict__ w, const half_t* __restrict__ s,
                                   half_t* __restrict__ out, long long ldo, int N, int K) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const int per = K >> 3;
  if (i >= (long long)N * per) return;
  const int row = (int)(i / per), c = (int)(i - (long long)row * per);
  h2 v[4];
  int k0;
  half_t sc;
  if constexpr (FMT == FMT_Q4) {
    // superblock word c: elements 8g .. 8g + 7 of block 4 * (c / 16) + c % 4, g = (c / 4) % 4
    const int blk = 4 * (c >> 4) + (c & 3);
    k0 = 32 * blk + 8 * ((c >> 2) & 3);
    q4_word_to_h2(((const uint32_t*)w)[i], v);
    sc = s[(size_t)row * (K >> 5) + blk];
  } else {
    const u2 q = ((const u2*)w)[i];
    i8x4_to_h2(q.x, v[0], v[1]);
    i8x4_to_h2(q.y, v[2], v[3]);
    k0 = 8 * c;
    sc = FMT == FMT_BW ? s[(size_t)row * (K >> 5) + (k0 >> 5)] : s[row];
  }
  const h2 s2 = {sc, sc};
  u4 o;
  o.x = as_u32(v[0] * s2); o.y = as_u32(v[1] * s2); o.z = as_u32(v[2] * s2); o.w = as_u32(v[3] * s2);
  *(u4*)(out + (size_t)row * ldo + k0) = o;
}

}  // namespace afx

using namespace afx;

extern "C" {

// GGUF Q4_0 blocks [N][K/32] (18 B each) -> superblock codes qs [N][K/2] + scales d [N][K/32].
int afx_q4_0_repack(const void* blocks, void* qs, void* d, int N, int K, void* stream) {
  AFX_REQUIRE(blocks && qs && d, "afx_q4_0_repack: null pointer");
  AFX_REQUIRE(N >= 1 && K >= 128 && K % 128 == 0, "afx_q4_0_repack: K=%d must be a positive multiple of 128", K);
  const long long nblk = (long long)N * (K / 32);
  hipLaunchKernelGGL(q4_repack_kernel, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)blocks, (uint32_t*)qs, (half_t*)d, N, K);
  return check_launch("afx_q4_0_repack");
}

// GGUF Q4_K super-blocks [N][K/256] (144 B each) -> codes qs [N][K/2] + headers hdr [N][K/256][5] u32.
int afx_q4_k_repack(const void* blocks, void* qs, void* hdr, int N, int K, void* stream) {
  AFX_REQUIRE(blocks && qs && hdr, "afx_q4_k_repack: null pointer");
  AFX_REQUIRE(N >= 1 && K >= 256 && K % 256 == 0, "afx_q4_k_repack: K=%d must be a positive multiple of 256", K);
  AFX_REQUIRE(((uintptr_t)hdr & 3) == 0, "afx_q4_k_repack: hdr must be 4-byte aligned");
  const long long nblk = (long long)N * (K / 256);
  hipLaunchKernelGGL(q4k_repack_kernel, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)blocks, (uint8_t*)qs, (uint32_t*)hdr, N, K);
  return check_launch("afx_q4_k_repack");
}

// GGUF Q6_K super-blocks [N][K/256] (210 B each) -> codes qs [N][K/2] + side words sw [N][K/32][3] u32.
int afx_q6_k_repack(const void* blocks, void* qs, void* sw, int N, int K, void* stream) {
  AFX_REQUIRE(blocks && qs && sw, "afx_q6_k_repack: null pointer");
  AFX_REQUIRE(N >= 1 && K >= 256 && K % 256 == 0, "afx_q6_k_repack: K=%d must be a positive multiple of 256", K);
  AFX_REQUIRE(((uintptr_t)qs & 3) == 0 && ((uintptr_t)sw & 3) == 0, "afx_q6_k_repack: outputs must be 4-byte aligned");
  const long long nblk = (long long)N * (K / 256);
  hipLaunchKernelGGL(q6k_repack_kernel, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)blocks, (uint32_t*)qs, (uint32_t*)sw, N, K);
  return check_launch("afx_q6_k_repack");
}

// Inverse of afx_q4_0_repack (round-trip check back to GGUF bytes).
int afx_q4_0_unpack(const void* qs, const void* d, void* blocks, int N, int K, void* stream) {
  AFX_REQUIRE(blocks && qs && d, "afx_q4_0_unpack: null pointer");
  AFX_REQUIRE(N >= 1 && K >= 128 && K % 128 == 0, "afx_q4_0_unpack: K=%d must be a positive multiple of 128", K);
  const long long nblk = (long long)N * (K / 32);
  hipLaunchKernelGGL(q4_unpack_kernel, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint32_t*)qs, (const half_t*)d, (uint8_t*)blocks, N, K);
  return check_launch("afx_q4_0_unpack");
}

// Dequantise through the GEMV unpack path: fmt 0 = int8 [N][K] + s[N]; fmt 1 = Q4_0 superblock.
// fmt 0 int8, 1 Q4_0 (superblock layout), 3 blockwise, 4 int4 codebook, 5 Q4_K, 6 Q6_K -> fp16 rows of stride ldo.
int afx_dequant_f16(int fmt, const void* w, const void* scale, void* out, long long ldo, int N, int K,
                    void* stream) {
  AFX_REQUIRE(w && scale && out, "afx_dequant_f16: null pointer");
  AFX_REQUIRE(fmt == 0 || fmt == 1 || fmt == 3 || fmt == 4 || fmt == 5 || fmt == 6,
              "afx_dequant_f16: format %d has no scales to apply", fmt);
  const int kq = fmt == 1 ? 128 : fmt == 3 ? 32 : fmt == 5 || fmt == 6 ? 256 : 8;
  AFX_REQUIRE(N >= 1 && K >= kq && K % kq == 0, "afx_dequant_f16: K=%d must be a multiple of %d", K, kq);
  AFX_REQUIRE(ldo >= K && ldo % 8 == 0 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)w & 7) == 0,
              "afx_dequant_f16: out rows must be 16-byte aligned (ldo %% 8 == 0) and ldo >= K");
  const long long n8 = (long long)N * (K / 8);
  const dim3 grid((unsigned)((n8 + 255) / 256));
  if (fmt == 4)
    hipLaunchKernelGGL(dequant_l4_kernel<half_t>, grid, dim3(256), 0, (hipStream_t)stream, (const uint32_t*)w,
                       (const half_t*)scale, (half_t*)out, ldo, N, K);
  else if (fmt == 5)
    hipLaunchKernelGGL(dequant_q4k_kernel<half_t>, grid, dim3(256), 0, (hipStream_t)stream, (const uint32_t*)w,
                       (const uint32_t*)scale, (half_t*)out, ldo, N, K);
  else if (fmt == 6)
    hipLaunchKernelGGL(dequant_q6k_kernel<half_t>, grid, dim3(256), 0, (hipStream_t)stream, (const uint32_t*)w,
                       (const uint32_t*)scale, (half_t*)out, ldo, N, K);
  else if (fmt == 0)
    hipLaunchKernelGGL(dequant_f16_kernel<FMT_I8>, grid, dim3(256), 0, (hipStream_t)stream, w,
                       (const half_t*)scale, (half_t*)out, ldo, N, K);
  else if (fmt == 1)
    hipLaunchKernelGGL(dequant_f16_kernel<FMT_Q4>, grid, dim3(256), 0, (hipStream_t)stream, w,
                       (const half_t*)scale, (half_t*)out, ldo, N, K);
  else
    hipLaunchKernelGGL(dequant_f16_kernel<FMT_BW>, grid, dim3(256), 0, (hipStream_t)stream, w,
                       (const half_t*)scale, (half_t*)out, ldo, N, K);
  return check_launch("afx_dequant_f16");
}

int afx_dequant(int fmt, const void* w, const void* scale, float* out, int N, int K, void* stream) {
  AFX_REQUIRE(w && scale && out, "afx_dequant: null pointer");
  if (fmt == 0) {
    AFX_REQUIRE(K % 4 == 0 && ((uintptr_t)w & 3) == 0, "afx_dequant: int8 K must be a multiple of 4");
    const long long nw = (long long)N * (K / 4);
    hipLaunchKernelGGL(dequant_i8_kernel, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (const uint32_t*)w, (const half_t*)scale, out, N, K);
  } else if (fmt == 1) {
    AFX_REQUIRE(K % 128 == 0, "afx_dequant: Q4_0 K must be a multiple of 128");
    const long long nw = (long long)N * (K / 8);
    hipLaunchKernelGGL(dequant_q4_kernel, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (const uint32_t*)w, (const half_t*)scale, out, N, K);
  } else if (fmt == 4) {
    AFX_REQUIRE(K % 8 == 0 && ((uintptr_t)w & 3) == 0, "afx_dequant: int4 K must be a multiple of 8");
    const long long n8 = (long long)N * (K / 8);
    hipLaunchKernelGGL(dequant_l4_kernel<float>, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (const uint32_t*)w, (const half_t*)scale, out, (long long)K, N, K);
  } else if (fmt == 5) {
    AFX_REQUIRE(K % 256 == 0 && ((uintptr_t)w & 3) == 0 && ((uintptr_t)scale & 3) == 0,
                "afx_dequant: Q4_K K must be a multiple of 256");
    const long long n8 = (long long)N * (K / 8);
    hipLaunchKernelGGL(dequant_q4k_kernel<float>, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (const uint32_t*)w, (const uint32_t*)scale, out, (long long)K, N, K);
  } else if (fmt == 6) {
    AFX_REQUIRE(K % 32 == 0 && ((uintptr_t)w & 3) == 0 && ((uintptr_t)scale & 3) == 0,
                "afx_dequant: Q6_K K must be a multiple of 32");
    const long long n8 = (long long)N * (K / 8);
    hipLaunchKernelGGL(dequant_q6k_kernel<float>, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (const uint32_t*)w, (const uint32_t*)scale, out, (long long)K, N, K);
  } else if (fmt == 3) {
    AFX_REQUIRE(K % 32 == 0 && ((uintptr_t)w & 3) == 0, "afx_dequant: blockwise K must be a multiple of 32");
    const long long nw = (long long)N * (K / 4);
    hipLaunchKernelGGL(dequant_bw_kernel, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (const uint32_t*)w, (const half_t*)scale, out, N, K);
  } else {
    return set_error("afx_dequant: unknown format %d", fmt);
  }
  return check_launch("afx_dequant");
}

}  // extern "C"
