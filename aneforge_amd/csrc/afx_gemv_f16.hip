// Instantiations of the weight-streaming GEMV for FMT_F16 (one translation unit per format keeps
// the build parallel).
#include "afx_gemv_impl.h"

namespace afx {
gemv_fn pick_gemv_f16(int mt, int eg, int R, int xs) { return pick_gemv<FMT_F16>(mt, eg, R, xs); }
gemv_fn pick_gemv_row_f16(int eg, int R, int norm, int U) { return pick_gemv_row<FMT_F16>(eg, R, norm, U); }
}  // namespace afx
