// p8x_gemm.hip -- prompt-processing GEMM (weight tiles decoded to fp16 in LDS, MFMA, fp32 accumulation).
#include <hip/hip_runtime.h>

#include "p8x_internal.h"
#include "p8x_lane.h"

namespace p8x {

int launch_mul_mat(const p8x_tensor *t, const void *x, int x_dtype, int N, size_t ldx, float *y, size_t ldy, hipStream_t st) {
    (void)t; (void)x; (void)x_dtype; (void)N; (void)ldx; (void)y; (void)ldy; (void)st;
    return set_error(P8X_ERR_UNSUPPORTED, "p8x_mul_mat: not built yet");
}

}  // namespace p8x
