// Instantiations of the weight-streaming GEMV for FMT_I8 (one translation unit per format keeps
// the build parallel).
#include "afx_gemv_impl.h"

namespace afx {
gemv_fn pick_gemv_i8(int mt, int eg, int R, int xs) { return pick_gemv<FMT_I8>(mt, eg, R, xs); }
gemv_fn pick_gemv_row_i8(int eg, int R, int norm, int U) { return pick_gemv_row<FMT_I8>(eg, R, norm, U); }
}  // namespace afx
