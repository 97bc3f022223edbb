// Shared device helpers for the aneforge_amd HIP kernels (gfx950 / CDNA4 only).
//
// Conventions used by every kernel in this library:
//  * fp16 tensors travel as raw IEEE half bits; on the device they are `_Float16`.
//  * All accumulation is fp32.  Integer codes are turned into fp16 values EXACTLY
//    (magic-number construction, see i8x4_to_h2 / q4_word_to_h2), so a dequantised
//    weight q*s is bit-identical to the fp32 product of the code and the fp32 scale.
//  * Wavefronts are 64 lanes; every reduction below is written for wave64.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace afx {

typedef _Float16 half_t;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// RMSNorm output of an fp16 pair: fp16((x * rstd) * g), each product rounded to fp32 as written.
// Each product is one v_fma_mix_f32 reading its fp16 operand in place, with a -0 addend:
// a*b + (-0) rounds exactly as a*b, signed zeros included, so the result is the plain
// convert-and-multiply form's bit for bit at half its instructions.
__device__ __forceinline__ uint32_t rms_pair(uint32_t x2, uint32_t g2, float rstd) {
  const float mz = -0.0f;
  float a0, a1, b0, b1;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(a0) : "v"(x2), "v"(rstd), "v"(mz));
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(a1) : "v"(x2), "v"(rstd), "v"(mz));
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(b0) : "v"(a0), "v"(g2), "v"(mz));
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(b1) : "v"(a1), "v"(g2), "v"(mz));
  h2 o;
  o.x = (half_t)b0;
  o.y = (half_t)b1;
  return as_u32(o);
}

// c + a.x*b.x + a.y*b.y in fp32 (v_dot2_f32_f16).
__device__ __forceinline__ float dot2(h2 a, h2 b, float c) {
  return __builtin_amdgcn_fdot2(a, b, c, false);
}

// Four signed int8 codes (one dword, byte i = code i) -> two exact fp16 pairs.
// (b ^ 0x80) = b + 128 is placed in the low mantissa byte of 0x64xx (= 1024 + byte),
// then 1152 = 1024 + 128 is subtracted; every step is exact in fp16.
__device__ __forceinline__ void i8x4_to_h2(uint32_t w, h2& lo, h2& hi) {
  const uint32_t u = w ^ 0x80808080u;
  const h2 off = {(half_t)1152.0f, (half_t)1152.0f};
  lo = as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - off;   // codes 0,1
  hi = as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - off;   // codes 2,3
}

// One 32-bit word of the repacked Q4_0 layout holds 8 consecutive elements e0..e7 of a
// 32-element block: low half-word = e0,e2,e4,e6 (bits 0,4,8,12), high half-word =
// e1,e3,e5,e7 (bits 16,20,24,28).  Output: exact fp16 pairs (e0-8,e1-8) .. (e6-8,e7-8).
// Nibble n in bits 0..3 of a half gives 0x6400|n = 1024+n; in bits 4..7 it gives
// 1024+16n, and (1024+16n)/16 - 72 = n-8 exactly.
// The constant in a vector register.  gfx9 VALU instructions read at most one scalar operand and
// a VOP3 encoding takes no literal, so with both the mask and 0x64006400 as constants the
// compiler splits (w & mask) | 0x64006400 into v_and + v_or; with 0x64006400 in a vector
// register (the mask in a scalar one) it is a single v_and_or_b32.
__device__ __forceinline__ uint32_t vreg_u32(uint32_t c) {
  uint32_t r;
  asm("v_mov_b32 %0, %1" : "=v"(r) : "n"(c));
  return r;
}
__device__ __forceinline__ void q4_word_to_h2(uint32_t w, h2 out[4]) {
  const h2 off_lo = {(half_t)-1032.0f, (half_t)-1032.0f};
  const h2 sc_hi = {(half_t)0.0625f, (half_t)0.0625f};
  const h2 off_hi = {(half_t)-72.0f, (half_t)-72.0f};
  const uint32_t magic = vreg_u32(0x64006400u);
  const uint32_t w8 = w >> 8;
  out[0] = as_h2((w & 0x000F000Fu) | magic) + off_lo;
  out[1] = as_h2((w & 0x00F000F0u) | magic) * sc_hi + off_hi;
  out[2] = as_h2((w8 & 0x000F000Fu) | magic) + off_lo;
  out[3] = as_h2((w8 & 0x00F000F0u) | magic) * sc_hi + off_hi;
}

__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor(v, m));
  return v;
}

// Reductions over the 16 lanes of each DPP row (xor 1, xor 2, then the half-row and row mirrors,
// which pair the two halves of an 8 / 16 lane group): every lane of a row gets its row's result.
// Four dependent VALU operations instead of six LDS-routed shuffles.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);     // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);     // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);    // row_half_mirror
  return v + dpp_f<0x140>(v);   // row_mirror
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  return fmaxf(v, dpp_f<0x140>(v));
}
__device__ __forceinline__ float lane0(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
}

// Transposed butterfly: each lane holds v[R] (R row partials); afterwards lane l holds the
// full 64-lane sum of row (l >> (6 - log2 R)) in v[0].  Costs R-1 + log2(64/R) shuffles
// instead of R*6.
template <int R>
__device__ __forceinline__ float wave_reduce_rows(float (&v)[R], int lane) {
  static_assert(R == 1 || R == 2 || R == 4 || R == 8 || R == 16, "R must be a power of two <= 16");
  if constexpr (R >= 16) {
    const bool hi = lane & 32;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float keep = hi ? v[i + 8] : v[i], send = hi ? v[i] : v[i + 8];
      v[i] = keep + shfl_xor(send, 32);
    }
  }
  if constexpr (R >= 8) {
    constexpr int B = (R >= 16) ? 16 : 32;
    const bool hi = lane & B;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float keep = hi ? v[i + 4] : v[i], send = hi ? v[i] : v[i + 4];
      v[i] = keep + shfl_xor(send, B);
    }
  }
  if constexpr (R >= 4) {
    constexpr int B = (R >= 16) ? 8 : (R >= 8) ? 16 : 32;
    const bool hi = lane & B;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float keep = hi ? v[i + 2] : v[i], send = hi ? v[i] : v[i + 2];
      v[i] = keep + shfl_xor(send, B);
    }
  }
  if constexpr (R >= 2) {
    constexpr int B = (R >= 16) ? 4 : (R >= 8) ? 8 : (R >= 4) ? 16 : 32;
    const bool hi = lane & B;
    float keep = hi ? v[1] : v[0], send = hi ? v[0] : v[1];
    v[0] = keep + shfl_xor(send, B);
  }
  constexpr int start = 32 / R;  // remaining butterfly over the low bits
  float s = v[0];
#pragma unroll
  for (int m = start; m >= 1; m >>= 1) s += shfl_xor(s, m);
  return s;
}

// Row owned by `lane` after wave_reduce_rows<R>.
template <int R>
__device__ __forceinline__ int reduced_row_of_lane(int lane) {
  if constexpr (R == 1) return 0;
  else if constexpr (R == 2) return lane >> 5;
  else if constexpr (R == 4) return ((lane >> 5) << 1) | ((lane >> 4) & 1);
  else if constexpr (R == 8) return ((lane >> 5) << 2) | (((lane >> 4) & 1) << 1) | ((lane >> 3) & 1);
  else return ((lane >> 5) << 3) | (((lane >> 4) & 1) << 2) | (((lane >> 3) & 1) << 1) | ((lane >> 2) & 1);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }
// tanh-approximated GELU (the "gelu_pytorch_tanh" of Gemma's GeGLU), 0.5 g (1 + tanh(z)) with
// z = sqrt(2/pi) (g + 0.044715 g^3); since 0.5 (1 + tanh(z)) = 1 / (1 + exp(-2z)), this is
// g / (1 + exp(-2z)): the same form as silu with a different argument.
__device__ __forceinline__ float gelu_tanh(float g) {
  const float two_z = 1.5957691216057308f * (g + 0.044715f * g * g * g);   // 2 * sqrt(2/pi) * (...)
  return g / (1.0f + __expf(-two_z));
}
// The gated MLP activation of an interleaved (gate, up) row pair: silu for SwiGLU, tanh-GELU for
// GeGLU (gelu = 1; a uniform flag, so the two share every kernel instance).
__device__ __forceinline__ float glu_act(bool gelu, float g) { return gelu ? gelu_tanh(g) : silu(g); }

// v_permlane16_swap(a, b) exchanges the odd 16-lane rows of a with the even rows of b, and
// v_permlane32_swap the upper 32 lanes of a with the lower 32 lanes of b.  With b a copy of a,
// afterwards a and b hold each row (half) and its partner row (half), so op(a, b) reduces over
// lane pairs 16 (32) apart in every lane.  Issued as inline assembly on two distinct registers
// (the s_nop covers the VALU-write-then-permlane hazard): this compiler's builtin returns the
// same half twice when its two results are combined.
__device__ __forceinline__ void swap16(float v, float& r0, float& r1) {
  unsigned a = __builtin_bit_cast(unsigned, v), b;
  asm volatile("v_mov_b32 %1, %0\n\ts_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "=&v"(b));
  r0 = __builtin_bit_cast(float, a);
  r1 = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ void swap32(float v, float& r0, float& r1) {
  unsigned a = __builtin_bit_cast(unsigned, v), b;
  asm volatile("v_mov_b32 %1, %0\n\ts_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "=&v"(b));
  r0 = __builtin_bit_cast(float, a);
  r1 = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float swap16_sum(float v) { float a, b; swap16(v, a, b); return a + b; }
__device__ __forceinline__ float swap32_sum(float v) { float a, b; swap32(v, a, b); return a + b; }
__device__ __forceinline__ float swap16_max(float v) { float a, b; swap16(v, a, b); return fmaxf(a, b); }
__device__ __forceinline__ float swap32_max(float v) { float a, b; swap32(v, a, b); return fmaxf(a, b); }

// Greedy-pick summaries {largest value, its index (int bits), second largest, largest magnitude}
// of two disjoint index ranges, merged: the larger first value wins, the lower index on an exact
// tie, and the loser's first value competes for second place (an exact tie makes them equal).
__device__ __forceinline__ float4 top2_merge(float4 a, float4 b) {
  const int ia = __float_as_int(a.y), ib = __float_as_int(b.y);
  // non-short-circuit operators: three compares combined in lane masks, no branch
  const bool a_first = (a.x > b.x) | ((a.x == b.x) & (ia < ib));
  const float4 f = a_first ? a : b, o = a_first ? b : a;
  return float4{f.x, f.y, fmaxf(f.z, o.x), fmaxf(a.w, b.w)};
}

}  // namespace afx

// ---- host-side error plumbing shared by all entry points (defined in afx_capi.hip) ----
extern "C" const char* afx_last_error(void);
namespace afx {
int set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));   // the compiler checks every message
int check_launch(const char* what);
}  // namespace afx

#define AFX_REQUIRE(cond, ...) \
  do { if (!(cond)) return ::afx::set_error(__VA_ARGS__); } while (0)
