// p8x_gemv_w.hip -- wave-independent GEMV instantiations (one column, 8-bit-per-128 activations)
#include "p8x_gemv.h"

namespace p8x {

int launch_gemv_wave(int cm, const GemvJob *jobs, const GemvJob &job0, const uint32_t *ujob, int units, unsigned *ctr, const uint32_t *a2,
                     hipStream_t st) {
    if (cm == kCmC3) return launch_gemv_wave_t<kCmC3>(jobs, job0, ujob, units, ctr, a2, st);
    if (cm == kCmC6) return launch_gemv_wave_t<kCmC6>(jobs, job0, ujob, units, ctr, a2, st);
    if (cm == kCmC234) return launch_gemv_wave_t<kCmC234>(jobs, job0, ujob, units, ctr, a2, st);
    return launch_gemv_wave_t<kCmAll>(jobs, job0, ujob, units, ctr, a2, st);
}

int launch_gemv_rg(int cm, const GemvJob &job, int ng, const uint32_t *a2, hipStream_t st) {
    if (cm == kCmC3) return launch_gemv_rg_t<kCmC3>(job, ng, a2, st);
    if (cm == kCmC6) return launch_gemv_rg_t<kCmC6>(job, ng, a2, st);
    if (cm == kCmC234) return launch_gemv_rg_t<kCmC234>(job, ng, a2, st);
    return launch_gemv_rg_t<kCmAll>(job, ng, a2, st);
}

}  // namespace p8x
