// Instantiations of the weight-streaming GEMV for FMT_Q4K (GGUF Q4_K super-blocks repacked by
// afx_q4_k_repack; one translation unit per format keeps the build parallel).
#include "afx_gemv_impl.h"

namespace afx {
gemv_fn pick_gemv_q4k(int mt, int eg, int R, int xs) { return pick_gemv<FMT_Q4K>(mt, eg, R, xs); }
gemv_fn pick_gemv_row_q4k(int eg, int R, int norm, int U) { return pick_gemv_row<FMT_Q4K>(eg, R, norm, U); }
}  // namespace afx
