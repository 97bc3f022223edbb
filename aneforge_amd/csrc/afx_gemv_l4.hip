// Instantiations of the weight-streaming GEMV for FMT_L4 (compress="int4": 4-bit indices into a
// per-tensor 16-entry codebook; one translation unit per format keeps the build parallel).
#include "afx_gemv_impl.h"

namespace afx {
gemv_fn pick_gemv_l4(int mt, int eg, int R, int xs) { return pick_gemv<FMT_L4>(mt, eg, R, xs); }
gemv_fn pick_gemv_row_l4(int eg, int R, int norm, int U) { return pick_gemv_row<FMT_L4>(eg, R, norm, U); }
}  // namespace afx
