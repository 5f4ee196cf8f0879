/*
 * p8x.h -- C ABI of the MI355X (gfx950) Pingala-8 hot path: block decode of the 2-bit coset-trellis
 * weight tiles and the fused decode x activation products that consume them.
 *
 * Reference interfaces replaced (patches/llama_cpu_vs_7ac59a6.patch, "CPU.patch"):
 *   tensor contract ......... ggml/include/ggml-vr-native.h (CPU.patch:1-51)
 *   probe / prepare ......... vrc_probe, vrc_init (CPU.patch:234-275); vr_native_probe,
 *                             vr_prepare_native (CPU.patch:1955-1965, :4335-4390)
 *   dequantize_row .......... vrc_dequant_f32 (CPU.patch:1012-1027), vrc_decode_tile_int (:992-1010)
 *   dequant to fp16 ......... ggml_cuda_f44_to_fp16/_fp32 hooks (CPU.patch:1351-1365); for VR tensors
 *                             the role of k_r51_k1 (CPU.patch:2176-2235)
 *   activation quantization . vrc_prep_block (CPU.patch:559-571), k_vr_qx_real (:4292-4307);
 *                             ggml quantize_q8_1 (stock llama.cpp, called at CPU.patch:1576)
 *   vec_dot ................. vrc_tile / vrc_dot128 (CPU.patch:617-668)
 *   mul_mat_vec ............. vr_mul_mat_vec + k_vr (CPU.patch:4466-4521, :3951-4016), vrc_tg (:1161-1199),
 *                             ggml_cuda_f44_mul_mat_vec (:2615-2631)
 *   mul_mat (prompt) ........ ggml_cuda_f44_mul_mat_q8 (CPU.patch:2303-2343)
 *
 * Conventions (as the reference): weights W are [rows][K] (ggml ne0 = K); y[rows] = W x. Tiles are
 * 32 sorted rows x 256 columns; outputs are written in ORIGINAL row order (prm un-permute) and the sparse
 * clamp delta is applied on the original activations. Differences: status codes instead of aborts,
 * explicit handles instead of a global registry, deterministic reductions instead of float atomics.
 *
 * Every function returns P8X_OK (0) or a P8X_ERR_* code; p8x_last_error() gives a thread-local message.
 * Device entry points take device pointers and a hipStream_t passed as void* (NULL = null stream); they
 * are asynchronous. Calls that share one p8x_tensor use its workspace and must be ordered on one stream.
 */
#ifndef P8X_H
#define P8X_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    P8X_OK = 0,
    P8X_ERR_ARG = 1,          /* bad argument (null pointer, shape, out of range) */
    P8X_ERR_FORMAT = 2,       /* slot bytes fail the tensor contract checks */
    P8X_ERR_HIP = 3,          /* a HIP runtime call failed */
    P8X_ERR_UNSUPPORTED = 4,  /* valid request this build does not serve */
    P8X_ERR_NOMEM = 5
};

enum { P8X_F32 = 0, P8X_F16 = 1, P8X_BF16 = 2, P8X_I16 = 3 };
enum { P8X_DOMAIN_ORIGINAL = 0, P8X_DOMAIN_ROTATED = 1 };
enum { P8X_ACT_Q8_128 = 0, P8X_ACT_Q8_1 = 1, P8X_ACT_X16 = 2 };

#define P8X_MAX_COLS 8

typedef struct p8x_tensor p8x_tensor;

typedef struct p8x_info {
    int rows, K, nd, ng, nb;
    size_t n;               /* slot bytes */
    size_t kbytes;          /* kernel bytes (header + M + S + D) */
    size_t stream_bytes;    /* packed weight stream read by a GEMV: M words + S + D payload */
    size_t class_tiles[8];  /* tiles per class 0..7 */
    const void *dev_base;   /* device address of the slot bytes (on_device = 0: the library's copy, whose payload
                               region is re-laid for 16-byte loads; on_device = 1: the caller's bytes, unchanged) */
} p8x_info;

const char *p8x_version(void);
const char *p8x_error_string(int code);
const char *p8x_last_error(void);

/* ---- tensor contract (CPU.patch:25-51) ------------------------------------------------------------ */
/* bytes a slot needs: vrn_need (CPU.patch:27-29) */
size_t p8x_need(size_t kbytes, int rows, int K, int nd);
/* 1 if the host bytes carry a native trailer for this shape, else 0: vrc_probe (CPU.patch:234-238) */
int p8x_probe(const void *slot, size_t n, int rows, int K);

/* Validate a slot and build its device-side metadata: vrc_init + vr_prepare_native (CPU.patch:240-275,
 * :4335-4390). on_device = 0: `slot` is host memory and is copied to a device allocation the handle owns;
 * on_device = 1: `slot` is device memory that must outlive the handle; it is only read, and the handle keeps a
 * copy of the payload re-laid for 16-byte loads (the device then holds the payload twice). Allocates everything the GEMV,
 * decode and activation entry points use; only p8x_mul_mat (see p8x_mul_mat_reserve) and
 * p8x_gemv_batch_create allocate later. */
int p8x_prepare(const void *slot, size_t n, int rows, int K, int on_device, p8x_tensor **out);
void p8x_release(p8x_tensor *t);
int p8x_tensor_info(const p8x_tensor *t, p8x_info *out);

/* ---- decode / dequantize_row ---------------------------------------------------------------------- */
/* Original-domain weights of the whole tensor, row r of `out` = ORIGINAL row r, row stride `ld` elements,
 * dtype P8X_F32 | P8X_F16 | P8X_BF16. F32 is bit-exact to vrc_dequant_f32 (CPU.patch:1012-1027); F16/BF16
 * are that F32 rounded to nearest even. */
int p8x_dequantize(const p8x_tensor *t, int dtype, void *out, size_t ld, void *stream);
/* Rotated-domain sorted-row weights: P8X_I16 = exact tile ints (vrc_decode_tile_int, CPU.patch:992-1010),
 * P8X_F32 = int * S (vr_wint * vr_wscale, CPU.patch:4030-4071). out is [rows][ld]. */
int p8x_decode_rotated(const p8x_tensor *t, int dtype, void *out, size_t ld, void *stream);

/* The same on part of a tensor (the reference's per-tile and per-row-group core functions): p8x_decode_tiles = the
 * tiles of row groups g0 .. g0 + ng - 1 and blocks b0 .. b0 + nb - 1 (vrc_decode_tile_int for one tile,
 * CPU.patch:992-1010), out [32 ng][ld >= 256 nb] relative to the window; p8x_dequantize_rows = ORIGINAL rows
 * row0 .. row0 + nrows - 1 of dequantize_row, out [nrows][ld >= K], the same bits as the whole-tensor call. */
int p8x_decode_tiles(const p8x_tensor *t, int dtype, int g0, int ng, int b0, int nb, void *out, size_t ld, void *stream);
int p8x_dequantize_rows(const p8x_tensor *t, int dtype, int row0, int nrows, void *out, size_t ld, void *stream);

/* ---- activations ------------------------------------------------------------------------------------ */
/* x' = FWHT256(x * sg / c) / 16, 8-bit per 128-column half-slice: q [ncols][K] int8, d [ncols][K/128]
 * (d = amax/127), sum [ncols][K/128] (sum of q; may be NULL). Bit-exact to vrc_prep_block / k_vr_qx_real. */
int p8x_quantize_q8_128(const p8x_tensor *t, const float *x, int ncols, size_t ldx,
                        int8_t *q, float *d, int32_t *sum, void *stream);
/* x16 precision mode (the reference CPU path's default, vrc_prep_block16, CPU.patch:575-616): per 128-column half,
 * d = max|x'| / 8191 and q = round-half-even(x' / d) (14 bits), split into two 8-bit planes q = 128 hi + lo:
 * qh/ql [ncols][K] int8, dh = 128 d and dl = d [ncols][K/128], sh/sl sums (may be NULL). Bit-exact to the reference.
 * The planes are two virtual 8-bit-per-128 columns: p8x_vec_dot(P8X_ACT_Q8_128) takes them as such. */
int p8x_quantize_x16(const p8x_tensor *t, const float *x, int ncols, size_t ldx, int8_t *qh, float *dh, int32_t *sh,
                     int8_t *ql, float *dl, int32_t *sl, void *stream);
/* x' quantized to ggml block_q8_1 (36 B: fp16 d, fp16 s, 32 x int8), [ncols][K/32] blocks, with ggml's
 * quantize_row_q8_1_ref convention: d = amax/127, q = roundf(x' * (1/d)) (ties away from zero), s = fp16(d * sum q).
 * The products read d and q only, so blocks from another q8_1 producer (ggml's CUDA kernel, say) are accepted. */
int p8x_quantize_q8_1(const p8x_tensor *t, const float *x, int ncols, size_t ldx, void *blocks, void *stream);

/* ---- products --------------------------------------------------------------------------------------- */
/* vec_dot against pre-quantized activations (vrc_tile, CPU.patch:617-668): act = P8X_ACT_Q8_128 (q, d from
 * p8x_quantize_q8_128, `d` required) or P8X_ACT_Q8_1 (q = block_q8_1 array, d ignored). Writes y [ncols][ldy]
 * in ORIGINAL rows. The clamp delta needs the unquantized activations: it is added when x ([ncols][ldx] f32)
 * is given and skipped when x is NULL. partials (optional, sorted rows): int32 [ncols][rows][K/128] for
 * Q8_128 or [ncols][rows][K/32] for Q8_1, the exact integer dot of each row with each quantization block. */
int p8x_vec_dot(const p8x_tensor *t, int act, const void *q, const float *d, int ncols, const float *x, size_t ldx,
                float *y, size_t ldy, int32_t *partials, void *stream);
/* p8x_vec_dot on the sorted row groups g0 .. g0 + ng - 1 (vrc_tile's per-tile products summed over K, CPU.patch:617-
 * 668; the reference's CPU GEMV hands such row groups to its threads): y is written at those groups' ORIGINAL rows
 * only (same values as the whole-tensor call), partials are [ncols][32 ng][blocks] for those sorted rows. */
int p8x_vec_dot_rows(const p8x_tensor *t, int act, const void *q, const float *d, int ncols, int g0, int ng, const float *x, size_t ldx,
                     float *y, size_t ldy, int32_t *partials, void *stream);
/* y = W x for 1..8 columns (vr_mul_mat_vec, CPU.patch:4466-4521): activation prep + fused decode-GEMV +
 * un-permute + clamp delta. x [ncols][ldx] f32, y [ncols][ldy] f32, original rows. One launch for one column
 * (and two columns of short K), deterministic. The K-chunk partial rows, arrival counters and meeting slots live
 * in the tensor's handle: calls on one tensor from different streams must not overlap (on one stream they are
 * ordered); counters and slots are put back by each call. Records kernel launches only (capture-safe). */
int p8x_mul_mat_vec(const p8x_tensor *t, const float *x, int ncols, size_t ldx, float *y, size_t ldy, void *stream);
/* the same with the activation mode chosen: P8X_ACT_Q8_128 (as p8x_mul_mat_vec), P8X_ACT_Q8_1 (ggml block_q8_1 of x',
 * quantized inside the GEMV's launch, or by a prep launch within a graph evaluation, below), or P8X_ACT_X16 (1..4
 * columns: both planes of each column through one GEMV, summed, then the clamp delta; the reference's CPU default) */
int p8x_mul_mat_vec_act(const p8x_tensor *t, int act, const float *x, int ncols, size_t ldx, float *y, size_t ldy, void *stream);
/* Marks the start of a graph evaluation (ggml_vr_cpu_graph_begin, CPU.patch:1148). After the first call, a
 * p8x_mul_mat_vec_act call in P8X_ACT_X16 or P8X_ACT_Q8_1 mode reuses the activation that the previous such call on
 * the same device prepared when the input pointer, stride, column count, mode, K, input rotation and stream are the
 * same and no p8x_graph_begin came between them (the reference's cache across consecutive mul_mats on one input,
 * CPU.patch:1142-1143, :1171-1180). The caller keeps x unchanged between such calls, as within one graph evaluation;
 * with reuse on, calls in these modes on one device are ordered on one stream (they share a per-GPU buffer, a fixed
 * device array: nothing is allocated). Without any p8x_graph_begin call nothing is reused. */
void p8x_graph_begin(void);
/* Several linears on the same activation vector in one launch, batch 1 (the q/k/v or gate/up of a layer; ggml issues
 * one mul_mat per linear): y_i = W_i x for n = 1..4 tensors with the same K, codebook and input rotation (column
 * scales c and signs; a file encodes the linears that share an input with one c). Same arithmetic and results as n
 * p8x_mul_mat_vec calls; no counterpart in the reference. */
int p8x_mul_mat_vec_multi(const p8x_tensor *const *tensors, int n, const float *x, size_t ldx, float *const *y, const size_t *ldy,
                          void *stream);
/* The gated FFN input in one launch, batch 1: out[r] = silu(gate x)[r] * (up x)[r], silu(g) = g / (1 + e^-g) (ggml's
 * swiglu, the fusion ggml applies to mul_mat_vec + glu and the reference switches off for its tensors, CPU.patch:2608-
 * 2610). gate and up: same rows, K, codebook and input rotation; the two products are p8x_mul_mat_vec's (with their
 * clamp deltas), each row's pair meets through the gate tensor's workspace (calls with one gate tensor are ordered
 * on one stream). */
int p8x_mul_mat_vec_glu(const p8x_tensor *gate, const p8x_tensor *up, const float *x, size_t ldx, float *out, void *stream);
/* The two calls above with the activation mode chosen, as p8x_mul_mat_vec_act (the reference's CPU path defaults to
 * x16, CPU.patch:1157-1160, and prepares the activation once for consecutive mul_mats on the same input and c,
 * CPU.patch:1142-1143, :1171-1180): P8X_ACT_Q8_128 runs the one-launch forms above; P8X_ACT_X16 prepares x once in
 * tensor 0's (the gate's) workspace and runs each tensor's GEMV on it (both planes as two columns, summed, then the
 * clamp delta); P8X_ACT_Q8_1 runs each tensor's block_q8_1 GEMV with x quantized in its launch; then for the GLU
 * silu(gate) * up. Same values as p8x_mul_mat_vec_act per tensor. Calls sharing a tensor are ordered on one stream. */
int p8x_mul_mat_vec_multi_act(const p8x_tensor *const *tensors, int n, int act, const float *x, size_t ldx, float *const *y,
                              const size_t *ldy, void *stream);
int p8x_mul_mat_vec_glu_act(const p8x_tensor *gate, const p8x_tensor *up, int act, const float *x, size_t ldx, float *out, void *stream);

/* ---- a decode step's chain of linears in one launch ----
 * The graph-level form of the per-node calls above: where the reference walks the graph's MUL_MAT nodes once
 * (ggml_cuda_f44_prepare_graph, CPU.patch:1955-2004) and then launches one kernel per node (CPU.patch:2615-2631),
 * a step object takes the chain of a batch-1 step's linears once and runs it as one cooperative launch: stage s
 * computes p8x_mul_mat_vec_multi (or, with glu_out, p8x_mul_mat_vec_glu) of its tensors on its input x, and reads
 * x only after every earlier stage has finished (a grid barrier between stages), so a stage's input may be an
 * earlier stage's output. Results equal those per-node calls bit for bit. Stage tensors share one codebook; each
 * stage's tensors share K and the input rotation; x and outputs are device vectors (x 16-byte aligned). The step
 * keeps pointers: the tensors and buffers must outlive it. Calls of one step object are ordered on one stream. */
typedef struct p8x_step_stage {
    int n;                               /* 1..4 tensors on the same input */
    const p8x_tensor *tensors[4];
    const float *x;                      /* input, K floats */
    float *y[4];                         /* outputs, rows floats each (unused with glu_out) */
    float *glu_out;                      /* non-NULL: n == 2, glu_out = silu(tensors[0] x) * (tensors[1] x) */
} p8x_step_stage;
typedef struct p8x_step p8x_step;
int p8x_step_create(const p8x_step_stage *stages, int n, p8x_step **out);
int p8x_step_run(p8x_step *step, void *stream);
/* Synchronizes the device and reports whether every barrier of the launches so far completed (P8X_ERR_HIP if a
 * barrier wait gave up; the step then refuses further runs). */
int p8x_step_check(p8x_step *step);
int p8x_step_info(const p8x_step *step, int *grid, int *stages, int *class_set);
void p8x_step_release(p8x_step *step);
/* The step with the activation mode chosen (the reference CPU path's modes, CPU.patch:1157-1160): P8X_ACT_Q8_128
 * is p8x_step_create; P8X_ACT_Q8_1 and P8X_ACT_X16 make a step whose p8x_step_run enqueues each stage as its
 * per-node call (p8x_mul_mat_vec_multi_act, or p8x_mul_mat_vec_glu_act for a swiglu pair) in stage order on the
 * stream, the same bits as those calls; p8x_step_info reports grid 0 (no cooperative launch), and the step can be
 * captured in a HIP graph. Same stage checks as p8x_step_create. */
int p8x_step_create_act(const p8x_step_stage *stages, int n, int act, p8x_step **out);
/* Prompt GEMM (ggml_cuda_f44_mul_mat_q8, CPU.patch:2303-2343): Y [N][ldy] = X [N][ldx] W^T in ORIGINAL rows,
 * X in P8X_F32 or P8X_BF16 (16-byte aligned, ldx % 8 == 0). The Hadamard rotation is applied to X (fp16 x'),
 * weight tiles are decoded from the LDS coset table straight into fp16 MFMA operands (v S), fp32 accumulation,
 * clamp delta on the original X. Uses the handle's workspace (x' and output planes, N-dependent): a call with
 * a larger N than any before allocates it (synchronizing the device) unless p8x_mul_mat_reserve covered N. */
int p8x_mul_mat(const p8x_tensor *t, const void *x, int x_dtype, int N, size_t ldx, float *y, size_t ldy, void *stream);
/* No counterpart in the reference (ggml's pool allocator serves its temporaries): allocate the p8x_mul_mat
 * workspace for up to n_max tokens at set-up, so later calls with N <= n_max allocate nothing. */
int p8x_mul_mat_reserve(const p8x_tensor *t, int n_max);
/* No counterpart in the reference; for callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): p8x_mul_mat with its workspace (fp16 x' and K-split output planes) in a
 * fixed device array of P8X_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends. Allocates nothing and never
 * synchronizes; rejects (P8X_ERR_UNSUPPORTED) a call whose workspace exceeds the array (512 tokens of the Llama-3.1-8B
 * FFN shapes fit). Every call on one GPU shares that GPU's array: calls that overlap on one GPU (other streams, other
 * threads) race; calls ordered on one stream do not. Results equal p8x_mul_mat's. */
#define P8X_NOALLOC_SCRATCH_BYTES (96 << 20)
int p8x_mul_mat_noalloc(const p8x_tensor *t, const void *x, int x_dtype, int N, size_t ldx, float *y, size_t ldy, void *stream);

/* ---- grouped GEMV ------------------------------------------------------------------------------------- */
/* No counterpart in the reference (ggml issues one mul_mat per graph node). A fixed list of independent
 * GEMVs y_i = W_i x_i (8-bit-per-128 activations, the same ncols 1..8 for all) run as one batched
 * activation-prep launch plus one fused decode + GEMV launch, so the packed weights of many linears stream
 * through a single persistent grid (e.g. q/k/v, or gate/up, of a layer). All tensors must share the codebook
 * and coset vector. x/y are device pointers fixed at creation; create allocates the batch's workspace. */
typedef struct p8x_gemv_batch p8x_gemv_batch;
int p8x_gemv_batch_create(const p8x_tensor *const *tensors, const float *const *x, const size_t *ldx,
                          float *const *y, const size_t *ldy, int njobs, int ncols, p8x_gemv_batch **out);
/* the same with the activation mode: P8X_ACT_Q8_128 (as above) or P8X_ACT_X16 (1..4 columns; the prep writes both
 * planes of each column, the fused launch multiplies them as 2 ncols columns, the finishing launch sums each
 * column's planes and then adds the clamp delta: p8x_mul_mat_vec_act's x16 values) */
int p8x_gemv_batch_create_act(const p8x_tensor *const *tensors, const float *const *x, const size_t *ldx,
                              float *const *y, const size_t *ldy, int njobs, int ncols, int act, p8x_gemv_batch **out);
/* No counterpart in the reference: the same with the fused launch's kernel chosen by the caller (for comparisons):
 * P8X_GEMV_KERNEL_AUTO (the plan's choice, as p8x_gemv_batch_create_act), P8X_GEMV_KERNEL_DOT4 (v_dot4 products) or
 * P8X_GEMV_KERNEL_MFMA (the matrix-core kernel: class-3 batches of 2..8 multiplied columns, else P8X_ERR_UNSUPPORTED).
 * Both kernels give the same bits. */
#define P8X_GEMV_KERNEL_AUTO 0
#define P8X_GEMV_KERNEL_DOT4 1
#define P8X_GEMV_KERNEL_MFMA 2
int p8x_gemv_batch_create_ex(const p8x_tensor *const *tensors, const float *const *x, const size_t *ldx,
                             float *const *y, const size_t *ldy, int njobs, int ncols, int act, int kernel, p8x_gemv_batch **out);
int p8x_gemv_batch_run(const p8x_gemv_batch *b, void *stream);
/* the launches of p8x_gemv_batch_run separately: stage 0 = activation prep, 1 = fused decode + GEMV (sorted-row
 * partials per K-chunk and column), 2 = partials to original rows with the clamp delta */
int p8x_gemv_batch_run_stage(const p8x_gemv_batch *b, int stage, void *stream);
/* No counterpart in the reference; for callers that time the batch's kernels themselves: the same, with hipEvent_t
 * ev_start / ev_stop (either may be NULL) recorded by the runtime at the stage kernel's own start and end
 * (hipExtLaunchKernel), so their elapsed time is the kernel's duration without the queue work around it. */
int p8x_gemv_batch_run_stage_timed(const p8x_gemv_batch *b, int stage, void *stream, void *ev_start, void *ev_stop);
void p8x_gemv_batch_release(p8x_gemv_batch *b);
/* The launch plan of a batch: work units (a 32-row group over a K-chunk), jobs cut along K, waves of the launch,
 * class_set (bit c: tile class c is decoded), small_launch = 1 when the batch had fewer whole-K units than two
 * rounds of the launch's waves and every job was cut into units of two or more blocks, matrix_cores = 1 when the
 * fused launch computes the tile products on the matrix cores (the plan's choice: class-3 batches of 4..8 q8/128
 * columns or 2..4 x16 columns, whose planes count as two; p8x_gemv_batch_create_ex chooses explicitly). */
typedef struct p8x_batch_info { int njobs, ncols, class_set, units, split_jobs, small_launch, waves, matrix_cores; } p8x_batch_info;
int p8x_gemv_batch_info(const p8x_gemv_batch *b, p8x_batch_info *out);

/* ---- native model files (GGUF): slot bytes for p8x_prepare ----------------------------------------------- */
/* The host side of the reference's model loader for VR tensors (llama_model_loader::vr_native_init and
 * vr_native_load, CPU.patch:4700-4869): p8x_vr_open parses one GGUF file (or the shards of one model, metadata from
 * the first) and checks its VR metadata (vr.format, vr.ns = 108, vr.trl = 2, vr.n_linear = 7 x block_count,
 * vr.layout 2 or 3), finds every linear by its ".vr_c" side tensor and checks the side tensors (vr_c F16 [K], vr_prm
 * I16 [rows] in layout 2 and none in layout 3, optional vr_didx I16 [nd, 2] + vr_dval F32 [nd], vr.had_signs I8
 * [256]). p8x_vr_load assembles linear i's in-memory slot exactly as the reference's loader does (kernel bytes, VR3
 * expanded; c16, prm or identity, pinv, delta, signs, trailer at the top-down offsets of a slot of slot_bytes, the
 * size of the smallest of the reference's six quant slot types that holds it), with its checks (header NS / TRL,
 * tables equal across tensors, kbytes against the M words, prm a permutation, delta indices, signs +-1). Failures
 * return P8X_ERR_FORMAT with the reason in p8x_last_error(). Loads of one file may run on several threads. */
typedef struct p8x_vr_file p8x_vr_file;
typedef struct p8x_vr_desc {
    const char *name;       /* "<base>.weight" (valid while the file is open) */
    int rows, K, nd;
    int layout;             /* 2: sorted rows + vr_prm; 3: VR3 file bytes, natural rows */
    size_t fbytes;          /* bytes of the weight tensor in the file */
    size_t kbytes;          /* kernel bytes in memory (header, M, S, D) */
    size_t slot_bytes;      /* bytes p8x_vr_load writes (pass them to p8x_prepare as n) */
    int slot_type;          /* the ggml quant type of that slot (IQ2_XXS = 16, Q2_K = 10 .. Q6_K = 14) */
} p8x_vr_desc;
int p8x_vr_open(const char *const *paths, int npaths, p8x_vr_file **out);
int p8x_vr_count(const p8x_vr_file *f);
int p8x_vr_find(const p8x_vr_file *f, const char *name);   /* index of "<base>.weight", or -1 */
int p8x_vr_describe(const p8x_vr_file *f, int i, p8x_vr_desc *out);
int p8x_vr_load(p8x_vr_file *f, int i, void *slot, size_t cap);
void p8x_vr_close(p8x_vr_file *f);
/* The VR3 file layout (llama-vr3.h vrn3_rows / vrn3_expand, CPU.patch:4916-4950): one class per tensor, natural
 * rows, no M words; word 515 = P8X_VR3_TAG | class. p8x_vr3_rows: rows from the file size, K and word 515 (0 when
 * inconsistent), *kbytes = the expanded kernel bytes. p8x_vr3_expand writes those kbytes (arithmetic M words, word
 * 515 = 0, zero pad before the payload). */
#define P8X_VR3_TAG 0x56523300u
size_t p8x_vr3_rows(size_t fbytes, size_t K, uint32_t w515, size_t *kbytes);
int p8x_vr3_expand(const void *file_bytes, size_t fbytes, size_t rows, size_t K, void *dst, size_t cap);

/* ---- host-side producers (not on the hot path) -------------------------------------------------------- */
/* Random valid tensor slot (the reference's random-valid timing arm, CPU.patch:4391-4458). class_p[8] are
 * tile-class probabilities; codebook 0 = the shipped table (research/work/r48k3/tables_vrc.pt), 1 = random
 * A in [-64,64], c in [-16,16]. Writes at most cap bytes into out; *n_out = slot size. */
int p8x_synth_random(uint64_t seed, int rows, int K, const double *class_p, int codebook, int nd,
                     int permute_rows, void *out, size_t cap, size_t *n_out);
/* Quantize f32 weights W [rows][K] to a class-3 slot with the plain-MSE 8-state Viterbi (the identity-Hessian
 * case of the reference encoder, research/detail/r59_sourcecoding.py:39-98, r48k.py:213-239): S = fp16(1.05
 * rms/23.557) per 256 block of the rotated row, c16 per column, seeded Hadamard signs, clamp delta for
 * |W| > fp16(1.001 max|W|). c16 may be NULL (all ones). */
int p8x_quantize_tensor(const float *W, int rows, int K, const uint16_t *c16, uint64_t sign_seed,
                        void *out, size_t cap, size_t *n_out);

/* ---- encoder of real weights: every class, LDLQ error feedback, class allocation ----
 * Restates the reference's offline tensor encoder (research/detail/r48k.py:213-239 k_tensor, :104-118 encode,
 * :57-95 vit_k, :33-55 best_cw, :97-102 zero_ldlq, :121-141 alloc), which is Python (torch) there; this is its
 * native host form, behind the same inputs: weights W [rows][K], column scales c, the layer input's second moment H,
 * a bit budget. Every choice is a deterministic function of the inputs (fixed operation order, ties to the lower
 * index). */
typedef struct p8x_encode_params {
    const uint16_t *c16;     /* K fp16 column scales c (the decoder divides column k by c[k]); NULL: all 1 */
    const int8_t *signs;     /* 256 Hadamard signs (+1/-1); NULL: drawn from sign_seed */
    uint64_t sign_seed;
    const float *H;          /* K x K row-major symmetric second moment of the layer input (original columns); NULL:
                              * identity (plain MSE, no feedback) */
    const double *U;         /* K x K row-major upper factor in the rotated domain (p8x_encode_factor); overrides H */
    double damp;             /* diagonal damping of the rotated H, relative to its mean diagonal (0.1) */
    const uint8_t *classes;  /* (rows/32) x (K/256) class per tile, sorted-row order; NULL: allocated */
    double bits_per_weight;  /* index-stream budget of the allocation (2.0) */
    int n_salient;           /* the tiles that hold the n largest |W| are allocated class >= 6 (4) */
    const int16_t *prm;      /* sorted row -> original row; NULL: ascending mean log block energy */
    double alpha;            /* S = fp16(alpha * rms / gain[class]) per row and 256 columns (1.05) */
    const double *gain;      /* 8 class gains; NULL: those of the shipped codebook */
    const double *dist;      /* 8 class distortion factors of the allocation; NULL: those of the shipped codebook */
    const uint32_t *A;       /* 256-entry int8x4 codebook; NULL: the shipped one (then cs is ignored) */
    uint32_t cs;             /* coset int8x4 of a caller codebook; A[f] + cs must stay in int8 */
    int threads;             /* host worker threads; 0: hardware concurrency, at most 16 */
} p8x_encode_params;
void p8x_encode_defaults(p8x_encode_params *p);
/* Encodes W into a new slot (malloc'd; release with p8x_encode_free). P8X_ERR_ARG for bad shapes or inputs
 * (non-finite W, zero/non-finite c, H not positive definite, prm not a permutation, class > 7),
 * P8X_ERR_UNSUPPORTED when the payload or the delta list exceed the format or A + cs wraps. */
int p8x_encode_tensor(const float *W, int rows, int K, const p8x_encode_params *p, void **out, size_t *n_out);
void p8x_encode_free(void *slot);
/* U (K x K, upper, U^T U = Hq^-1) with Hq = R diag(1/c) H diag(1/c) R^T + damp * mean(diag) * I and R the per-256
 * block rotation FWHT(sg * .)/16 (research/detail/r48k.py:215-218). */
int p8x_encode_factor(const float *H, const uint16_t *c16, const int8_t *signs, uint64_t sign_seed, int K,
                      double damp, int threads, double *U);
/* Class per tile from per-tile distortion weights E (sum over the tile's 32 rows of block energy times the block's
 * mean U_ii^-2 share) within budget_bits for the whole tensor; floor_ (or NULL) marks tiles held at class >= 6
 * (research/detail/r48k.py:121-141). */
int p8x_encode_alloc(const double *E, int n_tiles, double budget_bits, const double *dist, const uint8_t *floor_,
                     uint8_t *classes);
/* bytes the two producers need */
size_t p8x_slot_bytes(int rows, int K, const size_t class_tiles[8], int nd);

#ifdef __cplusplus
}
#endif
#endif
