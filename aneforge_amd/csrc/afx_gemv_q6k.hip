// Instantiations of the weight-streaming GEMV for FMT_Q6K (GGUF Q6_K super-blocks repacked by
// afx_q6_k_repack; one translation unit per format keeps the build parallel).
#include "afx_gemv_impl.h"

namespace afx {
gemv_fn pick_gemv_q6k(int mt, int eg, int R, int xs) { return pick_gemv<FMT_Q6K>(mt, eg, R, xs); }
gemv_fn pick_gemv_row_q6k(int eg, int R, int norm, int U) { return pick_gemv_row<FMT_Q6K>(eg, R, norm, U); }
}  // namespace afx
