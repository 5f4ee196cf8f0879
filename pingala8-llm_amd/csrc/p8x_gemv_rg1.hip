// p8x_gemv_rg1.hip -- single-GEMV row-group kernel instantiations, one column (the drop-in p8x_mul_mat_vec).
// Built with kernel-argument preloading (see the Makefile): the activation pointers, the rotation and the K plan
// reach the waves in SGPRs, so the first loads do not wait for the kernel-argument segment.
#include "p8x_gemv.h"

namespace p8x {

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
