// Instantiations of the weight-streaming GEMV for FMT_BW (compress="blockwise": int8 codes with
// one fp16 scale per 32-weight block; one translation unit per format keeps the build parallel).
#include "afx_gemv_impl.h"

namespace afx {
gemv_fn pick_gemv_bw(int mt, int eg, int R, int xs) { return pick_gemv<FMT_BW>(mt, eg, R, xs); }
gemv_fn pick_gemv_row_bw(int eg, int R, int norm, int U) { return pick_gemv_row<FMT_BW>(eg, R, norm, U); }
}  // namespace afx
