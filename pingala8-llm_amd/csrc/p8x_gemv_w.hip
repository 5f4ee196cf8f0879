// p8x_gemv_w.hip -- wave-independent GEMV instantiations (one column, 8-bit-per-128 activations)
#include "p8x_gemv.h"

namespace p8x {

int launch_gemv_wave_mc(int ncols, int cm, const GemvJob *jobs, const uint32_t *ujob, int units, unsigned *ctr, const uint32_t *a2, hipStream_t st,
                        hipEvent_t e0, hipEvent_t e1);

int launch_gemv_wave(int ncols, int cm, const GemvJob *jobs, const uint32_t *ujob, int units, unsigned *ctr, const uint32_t *a2, hipStream_t st,
                     hipEvent_t e0, hipEvent_t e1) {
    if (ncols != 1) return launch_gemv_wave_mc(ncols, cm, jobs, ujob, units, ctr, a2, st, e0, e1);
    if (cm == kCmC3) return launch_gemv_wave_t<kCmC3, 1>(jobs, ujob, units, ctr, a2, st, e0, e1);
    if (cm == kCmC6) return launch_gemv_wave_t<kCmC6, 1>(jobs, ujob, units, ctr, a2, st, e0, e1);
    if (cm == kCmC234) return launch_gemv_wave_t<kCmC234, 1>(jobs, ujob, units, ctr, a2, st, e0, e1);
    if (cm == kCmC2346) return launch_gemv_wave_t<kCmC2346, 1>(jobs, ujob, units, ctr, a2, st, e0, e1);
    return launch_gemv_wave_t<kCmAll, 1>(jobs, ujob, units, ctr, a2, st, e0, e1);
}

}  // namespace p8x
