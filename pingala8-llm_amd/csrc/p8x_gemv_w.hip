// p8x_gemv_w.hip -- wave-independent GEMV instantiations (one column, 8-bit-per-128 activations) and the
// single-GEMV row-group kernel
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

int launch_gemv_rg_mc(int ncols, int cm, const RgJobs &job, int ng, const uint32_t *a2, hipStream_t st);

int launch_gemv_rg(int ncols, int cm, const RgJobs &job, int ng, const uint32_t *a2, hipStream_t st) {
    if (ncols != 1) return launch_gemv_rg_mc(ncols, cm, job, ng, a2, st);
    if (cm == kCmC3) return launch_gemv_rg_t<kCmC3, 1, false>(job, ng, a2, st);
    if (cm == kCmC6) return launch_gemv_rg_t<kCmC6, 1, false>(job, ng, a2, st);
    if (cm == kCmC234) return launch_gemv_rg_t<kCmC234, 1, false>(job, ng, a2, st);
    if (cm == kCmC2346) return launch_gemv_rg_t<kCmC2346, 1, false>(job, ng, a2, st);
    return launch_gemv_rg_t<kCmAll, 1, false>(job, ng, a2, st);
}

}  // namespace p8x
