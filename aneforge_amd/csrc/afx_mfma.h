// MFMA skinny GEMM for 2..16 activation rows ("tokens") against streamed quantized weights:
// the batched linears (cfg1 B = 4 / 8) and the grouped MoE experts.  See afx_mfma.hip.
#pragma once
#include "afx_gemv_core.h"

namespace afx {

struct MfmaArgs {
  const void* w;           // weights [E][N][row bytes] (format FMT)
  const half_t* scale;     // I8: [E][N] row scales; Q4: [E][N][K/32] block scales; F16: unused
  long long w_es, s_es;    // per-expert strides (bytes of w, elements of scale); 0 for a dense linear
  const half_t* x;         // activations, row r at x + r * ldx
  int ldx;
  void* y;                 // output rows at y + row * ldy (fp16, or fp32 for EPI_F32)
  int ldy;
  const half_t* bias;      // [N] or null (dense)
  const half_t* resid;     // [M][ldy] or null (EPI_RESID, dense; may alias y)
  const int* cnt;          // MoE: tokens per expert [E]; null for a dense linear
  const int* list;         // MoE: entry lists [E][T] (entry = token * k + slot)
  int T, k;                // MoE: tokens and top-k
  int x_by_token;          // MoE: x row of an entry = entry / k (1) or the entry itself (0)
  int M;                   // dense: activation rows (<= 16 per token group; any count, in groups)
  int N, K;
  int epi;                 // EPI_F16 / EPI_RESID / EPI_F32 / EPI_SWIGLU / EPI_GEGLU (gemv epilogue codes)
  int xbytes;              // set by mfma_launch: bytes of the activation rows the kernel may read
  int E;                   // set by mfma_launch: experts (1 for a dense linear)
  float* ws;               // optional fp32 workspace for K-split partials (null: no split)
  long long ws_bytes;
  int ks, ws_rows;         // set by mfma_launch: K slices, output rows per slice in ws
};

// Launch the MFMA kernel over E experts (1 for a dense linear).  Returns 0 or a negative code.
// ks_out (optional): a K-split launch then leaves its slices in a.ws without the finishing sum
// and reports their count there (1: no split, y was written).
int mfma_launch(int fmt, const MfmaArgs& a, int E, hipStream_t stream, const char* what, int* ks_out = nullptr);
// Whether the MFMA path supports this shape (K divisible into steps, one or more per wavefront).
bool mfma_supported(int fmt, int K);

}  // namespace afx
