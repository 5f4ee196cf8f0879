// p8x_gemv_rgm.hip -- single-GEMV row-group kernel instantiations: two columns of one-class tensors (class 3 or 6),
// and one column over several linears that share their input (p8x_mul_mat_vec_multi / _glu).
// (More columns measured slower than the multi-column task kernel on the Llama shapes: 8-wave workgroups at
// 256 VGPRs, and K-chunks whose fix-ups cost more than they save.)
#include "p8x_gemv.h"

namespace p8x {

template <int NCOL>
static int rg_cm(int cm, const RgJobs &job, int ng, const uint32_t *a2, hipStream_t st) {
    if (cm == kCmC3) return launch_gemv_rg_t<kCmC3, NCOL, false>(job, ng, a2, st);
    if (cm == kCmC6) return launch_gemv_rg_t<kCmC6, NCOL, false>(job, ng, a2, st);
    return set_error(P8X_ERR_UNSUPPORTED, "k_gemv_rg: %d columns need a one-class tensor", NCOL);
}

// several linears on one activation vector (one column): the MULTI instantiations
int launch_gemv_rg_multi(int cm, const RgJobs &jobs, int ng, const uint32_t *a2, hipStream_t st) {
    if (cm == kCmC3) return launch_gemv_rg_t<kCmC3, 1, true>(jobs, ng, a2, st);
    if (cm == kCmC6) return launch_gemv_rg_t<kCmC6, 1, true>(jobs, ng, a2, st);
    if (cm == kCmC234) return launch_gemv_rg_t<kCmC234, 1, true>(jobs, ng, a2, st);
    if (cm == kCmC2346) return launch_gemv_rg_t<kCmC2346, 1, true>(jobs, ng, a2, st);
    return launch_gemv_rg_t<kCmAll, 1, true>(jobs, ng, a2, st);
}

int launch_gemv_rg_mc(int ncols, int cm, const RgJobs &job, int ng, const uint32_t *a2, hipStream_t st) {
    if (ncols == 2) return rg_cm<2>(cm, job, ng, a2, st);
    return set_error(P8X_ERR_UNSUPPORTED, "k_gemv_rg: %d columns", ncols);
}

}  // namespace p8x
