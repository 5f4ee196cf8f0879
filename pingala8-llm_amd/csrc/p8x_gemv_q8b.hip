// p8x_gemv_q8b.hip -- GEMV instantiations, 8-bit-per-128 activations, 5..8 columns
#include "p8x_gemv.h"

namespace p8x {

template <int NCOL>
static int q8_cm(int cm, const GemvJob &job0, int tasks, const uint32_t *a2, hipStream_t st) {
    if (cm == kCmC3) return launch_gemv_t<NCOL, P8X_ACT_Q8_128, false, kCmC3>(job0, tasks, a2, st);
    if (cm == kCmC6) return launch_gemv_t<NCOL, P8X_ACT_Q8_128, false, kCmC6>(job0, tasks, a2, st);
    if (cm == kCmC234) return launch_gemv_t<NCOL, P8X_ACT_Q8_128, false, kCmC234>(job0, tasks, a2, st);
    if (cm == kCmC2346) return launch_gemv_t<NCOL, P8X_ACT_Q8_128, false, kCmC2346>(job0, tasks, a2, st);
    return launch_gemv_t<NCOL, P8X_ACT_Q8_128, false, kCmAll>(job0, tasks, a2, st);
}

int launch_gemv_q8_lo(int ncols, int cm, const GemvJob &job0, int tasks, const uint32_t *a2, hipStream_t st);

int launch_gemv_q8(int ncols, int cm, const GemvJob &job0, int tasks, const uint32_t *a2, hipStream_t st) {
    switch (ncols) {
        case 5: return q8_cm<5>(cm, job0, tasks, a2, st);
        case 6: return q8_cm<6>(cm, job0, tasks, a2, st);
        case 7: return q8_cm<7>(cm, job0, tasks, a2, st);
        case 8: return q8_cm<8>(cm, job0, tasks, a2, st);
        default: return launch_gemv_q8_lo(ncols, cm, job0, tasks, a2, st);
    }
}

}  // namespace p8x
