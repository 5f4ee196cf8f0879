// p8x_gemv_wm.hip -- wave-independent GEMV instantiations, 2..8 columns of 8-bit-per-128 activations (v_dot4 and
// matrix-core kernels)
#include "p8x_gemv.h"

namespace p8x {

template <int NCOL>
static int wave_cm(int cm, const GemvJob *jobs, const uint32_t *ujob, int units, unsigned *ctr, const uint32_t *a2, hipStream_t st,
                   hipEvent_t e0, hipEvent_t e1) {
    if (cm == kCmC3) return launch_gemv_wave_t<kCmC3, NCOL>(jobs, ujob, units, ctr, a2, st, e0, e1);
    if (cm == kCmC6) return launch_gemv_wave_t<kCmC6, NCOL>(jobs, ujob, units, ctr, a2, st, e0, e1);
    if (cm == kCmC234) return launch_gemv_wave_t<kCmC234, NCOL>(jobs, ujob, units, ctr, a2, st, e0, e1);
    if (cm == kCmC2346) return launch_gemv_wave_t<kCmC2346, NCOL>(jobs, ujob, units, ctr, a2, st, e0, e1);
    return launch_gemv_wave_t<kCmAll, NCOL>(jobs, ujob, units, ctr, a2, st, e0, e1);
}

int launch_gemv_wave_mc(int ncols, int cm, const GemvJob *jobs, const uint32_t *ujob, int units, unsigned *ctr, const uint32_t *a2, hipStream_t st,
                        hipEvent_t e0, hipEvent_t e1) {
    switch (ncols) {
        case 2: return wave_cm<2>(cm, jobs, ujob, units, ctr, a2, st, e0, e1);
        case 3: return wave_cm<3>(cm, jobs, ujob, units, ctr, a2, st, e0, e1);
        case 4: return wave_cm<4>(cm, jobs, ujob, units, ctr, a2, st, e0, e1);
        case 5: return wave_cm<5>(cm, jobs, ujob, units, ctr, a2, st, e0, e1);
        case 6: return wave_cm<6>(cm, jobs, ujob, units, ctr, a2, st, e0, e1);
        case 7: return wave_cm<7>(cm, jobs, ujob, units, ctr, a2, st, e0, e1);
        case 8: return wave_cm<8>(cm, jobs, ujob, units, ctr, a2, st, e0, e1);
        default: return set_error(P8X_ERR_ARG, "k_gemv_wave: %d columns", ncols);
    }
}

int launch_gemv_wave_mx(int ncols, const GemvJob *jobs, const uint32_t *ujob, int units, unsigned *ctr, const uint32_t *a2, hipStream_t st,
                        hipEvent_t e0, hipEvent_t e1) {
    switch (ncols) {
        case 2: return launch_gemv_wave_mx_t<2>(jobs, ujob, units, ctr, a2, st, e0, e1);
        case 3: return launch_gemv_wave_mx_t<3>(jobs, ujob, units, ctr, a2, st, e0, e1);
        case 4: return launch_gemv_wave_mx_t<4>(jobs, ujob, units, ctr, a2, st, e0, e1);
        case 5: return launch_gemv_wave_mx_t<5>(jobs, ujob, units, ctr, a2, st, e0, e1);
        case 6: return launch_gemv_wave_mx_t<6>(jobs, ujob, units, ctr, a2, st, e0, e1);
        case 7: return launch_gemv_wave_mx_t<7>(jobs, ujob, units, ctr, a2, st, e0, e1);
        case 8: return launch_gemv_wave_mx_t<8>(jobs, ujob, units, ctr, a2, st, e0, e1);
        default: return set_error(P8X_ERR_ARG, "k_gemv_wave_mx: %d columns", ncols);
    }
}

}  // namespace p8x
