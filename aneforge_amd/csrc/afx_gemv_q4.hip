// Instantiations of the weight-streaming GEMV for FMT_Q4 (one translation unit per format keeps
// the build parallel).
#include "afx_gemv_impl.h"

namespace afx {
gemv_fn pick_gemv_q4(int mt, int eg, int R, int xs) { return pick_gemv<FMT_Q4>(mt, eg, R, xs); }
gemv_fn pick_gemv_row_q4(int eg, int R, int norm, int U) { return pick_gemv_row<FMT_Q4>(eg, R, norm, U); }
}  // namespace afx
