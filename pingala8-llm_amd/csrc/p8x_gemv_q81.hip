// p8x_gemv_q81.hip -- GEMV instantiations: ggml block_q8_1 activations, and the integer-partials variant
#include "p8x_gemv.h"

namespace p8x {

int launch_gemv_q81(int ncols, int cm, const GemvJob &job0, int tasks, const uint32_t *a2, hipStream_t st) {
    if (ncols == 1 && cm == kCmC3) return launch_gemv_t<1, P8X_ACT_Q8_1, false, kCmC3>(job0, tasks, a2, st);
    switch (ncols) {
        case 1: return launch_gemv_t<1, P8X_ACT_Q8_1, false, kCmAll>(job0, tasks, a2, st);
        case 2: return launch_gemv_t<2, P8X_ACT_Q8_1, false, kCmAll>(job0, tasks, a2, st);
        case 3: return launch_gemv_t<3, P8X_ACT_Q8_1, false, kCmAll>(job0, tasks, a2, st);
        case 4: return launch_gemv_t<4, P8X_ACT_Q8_1, false, kCmAll>(job0, tasks, a2, st);
        case 5: return launch_gemv_t<5, P8X_ACT_Q8_1, false, kCmAll>(job0, tasks, a2, st);
        case 6: return launch_gemv_t<6, P8X_ACT_Q8_1, false, kCmAll>(job0, tasks, a2, st);
        case 7: return launch_gemv_t<7, P8X_ACT_Q8_1, false, kCmAll>(job0, tasks, a2, st);
        default: return launch_gemv_t<8, P8X_ACT_Q8_1, false, kCmAll>(job0, tasks, a2, st);
    }
}

int launch_gemv_partials(int act, const GemvJob &job0, const uint32_t *a2, hipStream_t st) {
    if (act == P8X_ACT_Q8_128) return launch_gemv_t<1, P8X_ACT_Q8_128, true, kCmAll>(job0, job0.ntasks, a2, st);
    return launch_gemv_t<1, P8X_ACT_Q8_1, true, kCmAll>(job0, job0.ntasks, a2, st);
}

}  // namespace p8x
