// p8x_internal.h -- library-internal types shared by the host code and the kernel launchers.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <vector>

#include "../../include/p8x.h"
#include "p8x_format.h"

namespace p8x {
struct GemvJob;
}

struct p8x_tensor {
    int rows = 0, K = 0, nb = 0, ng = 0, nsl = 0, nd = 0;
    size_t n = 0, nt = 0, kbytes = 0, stream_bytes = 0;
    size_t class_tiles[8] = {0};
    int device = 0;
    const uint8_t *base = nullptr;   // device slot bytes
    uint8_t *owned = nullptr;        // set when the library copied host bytes (the slot sits past a pad that puts
                                     // the payload on a 256-byte boundary)
    // views into the slot (device)
    const uint32_t *M = nullptr;
    const uint16_t *S = nullptr;
    const uint32_t *D = nullptr;     // payload in the device layout (dev_word): in the slot copy, or Dl
    uint32_t *Dl = nullptr;          // the library's re-laid payload copy when the caller owns the device slot
    const int16_t *prm = nullptr;
    uint16_t *Sg = nullptr;          // row scales regrouped [ng][nb][32]: a row group's scales in one run
    int16_t *pinv = nullptr;         // original row -> sorted row (built at prepare)
    std::vector<int16_t> pinv_host;  // the same on the host (row-range requests find their row groups)
    uint16_t *prmd = nullptr;        // sorted row -> original row, bit 15 set when that row carries clamp-delta entries
    bool prm_identity = false;
    // device metadata built at prepare
    uint32_t *a2 = nullptr;          // [2][256]: A[f] + h c (bytewise), h-major; then the same as fp16 [256][2][4]
    float *ic = nullptr;             // sg / c per column [K]
    int *cp = nullptr;               // delta CSR by original row [rows + 1]
    uint16_t *cc = nullptr;          // [nd]
    float *cv = nullptr;             // [nd]
    // workspace (stream-ordered use)
    int8_t *wq = nullptr;            // q8_128 activations [P8X_MAX_COLS][K]
    float *wd = nullptr;             // [P8X_MAX_COLS][nsl]
    int32_t *wsum = nullptr;         // [P8X_MAX_COLS][nsl]
    uint8_t *wq81 = nullptr;         // block_q8_1 [P8X_MAX_COLS][K / 32]
    float *wy = nullptr;             // x16 products: plane rows [2 x 4][rows]
    unsigned lin_words = 0;               // one class, tiles in order: payload words per tile (else 0)
    unsigned long long *wglu = nullptr;   // gate / up meeting slots (this tensor as the gate) [rows], 0 between calls
    unsigned long long *wslot = nullptr;  // K-half meeting slots of one-column two-chunk plans [rows], 0 between calls
    uint64_t ic_hash = 0;            // hash of the rotation sg / c (tensors with equal hashes share quantized inputs)
    std::vector<float> ic_host;      // the rotation sg / c on the host (several-tensor launches compare it bit for bit)
    p8x::GemvJob *djob = nullptr;    // the tensor's metadata as a device-side GEMV job (launches over several tensors)
    float *wpart = nullptr;          // K-chunk partial rows [nks][ncols][rows], sized for the largest plan
    size_t wpart_floats = 0;
    unsigned *wcnt = nullptr;        // split-K arrival counters [ng]
    int *drows = nullptr;            // original rows that carry clamp-delta entries [ndrows]
    std::vector<int> dorig;          // host: those original rows
    int ndrows = 0;
    uint16_t *wx16 = nullptr;        // prompt GEMM: rotated fp16 activations [N][K] (grown on demand)
    size_t wx16_elems = 0;           // capacity in bytes
    float *wmm = nullptr;            // prompt GEMM: K-split partial planes (grown on demand)
    size_t wmm_bytes = 0;
    uint32_t a2_host[512];           // host copy of a2 (batches check that tensors share the tables)
};

namespace p8x {

int set_error(int code, const char *fmt, ...);
int hip_check(hipError_t e, const char *what);

struct GemvPlan {
    int bpk, nks, grid, items, gpt;   // gpt: row groups per task (waves per workgroup)
};
GemvPlan gemv_plan(const p8x_tensor *t, int ncols, int act, bool partials);
// K-chunks of the single-call row-group kernel (8-bit-per-128 activations); *kc = blocks per chunk
int rg_plan(const p8x_tensor *t, int ncols, int *kc);

// launchers (p8x_gemv.hip, p8x_decode.hip, p8x_gemm.hip)
int launch_act_q8_128(const p8x_tensor *t, const float *x, int ncols, size_t ldx, int8_t *q, float *d, int32_t *sum, hipStream_t st);
int launch_act_q8_1(const p8x_tensor *t, const float *x, int ncols, size_t ldx, void *blocks, hipStream_t st);
// x16 planes: column n's hi plane at qh + n qstride, lo plane at ql + n qstride (scales and sums at n qstride / 128)
int launch_act_x16(const p8x_tensor *t, const float *x, int ncols, size_t ldx, int8_t *qh, float *dh, int32_t *sh, int8_t *ql, float *dl,
                   int32_t *sl, int qstride, hipStream_t st);
int launch_gemv_x16(const p8x_tensor *t, const float *x, int ncols, size_t ldx, float *y, size_t ldy, hipStream_t st);
int launch_gemv_x16_on(const p8x_tensor *t, const float *x, int ncols, size_t ldx, float *y, size_t ldy, int8_t *q, float *d, bool have,
                       hipStream_t st);
// Prepared-activation reuse within one graph evaluation (p8x_graph_begin): a device array of kActCacheBytes per GPU
// holds the activation the last x16 / block_q8_1 call prepared; act_reuse returns it (nullptr: no reuse, use the
// tensor's workspace) and whether it already holds this call's activation (same evaluation, input, stride, columns,
// mode, K, rotation and stream), and records this call's key.
constexpr size_t kActCacheBytes = 320 << 10;   // x16 and block_q8_1 activations of up to 4 / 8 columns of K <= 32768
constexpr int kMaxActDevices = 64;
int act_cache_resolve(int device);
void act_epoch_advance();
uint8_t *act_reuse(const p8x_tensor *t, int act, const float *x, int ncols, size_t ldx, size_t bytes, hipStream_t st, bool *have);
int launch_gemv_multi(const p8x_tensor *const *ts, int n, const float *x, size_t ldx, float *const *y, const size_t *ldy, float *out,
                      hipStream_t st);
int launch_gemv(const p8x_tensor *t, int act, const void *q, const float *d, int ncols, const float *x, size_t ldx,
                float *y, size_t ldy, int32_t *partials, hipStream_t st);
int launch_gemv_range(const p8x_tensor *t, int act, const void *q, const float *d, int ncols, const float *x, size_t ldx,
                      float *y, size_t ldy, int32_t *partials, int g0, int ng, hipStream_t st);
// window of row groups g0 .. g0 + gn - 1 and blocks b0 .. b0 + bn - 1; out relative to it
int launch_decode_rotated(const p8x_tensor *t, int dtype, int g0, int gn, int b0, int bn, void *out, size_t ld, hipStream_t st);
// original rows row0 .. row0 + nrows - 1 to out rows 0 .. nrows - 1
int launch_dequant(const p8x_tensor *t, int dtype, int row0, int nrows, void *out, size_t ld, hipStream_t st);
int launch_mul_mat(const p8x_tensor *t, const void *x, int x_dtype, int N, size_t ldx, float *y, size_t ldy, hipStream_t st);
int reserve_mul_mat(const p8x_tensor *t, int n_max);
// the tensor's GemvJob in device memory (t->djob), at prepare
int upload_job(p8x_tensor *t);
// device address of the no-allocation scratch array on `device` (hipGetSymbolAddress, once per device)
int scratch_resolve(int device);

int num_cus();
// offsets of the side regions of an n-byte slot, top-down from its end (vrn_offsets, CPU.patch:33-40):
// delta, c16, prm, pinv, signs, trailer
void side_offsets(size_t n, size_t rows, size_t K, size_t nd, size_t off[6]);

#ifdef P8X_TIMELINE
// Timeline build only (make timeline): per-workgroup / per-wave s_memrealtime records written by the instrumented
// kernels, [kTimelineRecords][8] words followed by the record counter.
constexpr unsigned kTimelineRecords = 65536;
unsigned long long *timeline_buf();
#endif

}  // namespace p8x
