/*
 * p8x_oracle.h -- CPU restatement of the Pingala-8 native tensor hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library (libp8x) links, loads or
 * calls this code. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg use it, and only as the checker.
 *
 * Every function restates the algorithm of the reference CPU core
 * (patches/llama_cpu_vs_7ac59a6.patch, "CPU.patch" below) in plain scalar C.
 * Citations point at the hunk line in the patch file.
 *
 * Pinning (what checks each function, see tests/test_oracle.py):
 *   orc_open / layout       : reference-compiled fixtures (tests/golden) + vrn_* layout formulas
 *   orc_trellis_word        : exhaustive 2^16 + random u32 vs orc_trellis_serial (bit-serial recurrence)
 *   orc_decode_tile         : golden fixtures from the compiled reference core, plus the bit-by-bit
 *                             per-weight decoder orc_weight_int (independent path)
 *   orc_dequant_f32         : golden fixtures (f32 bit patterns) from the compiled reference core
 *   orc_fwht256             : H*H = 256 I (involution up to 1/256), golden prep fixtures
 *   orc_prep_q8_128         : golden fixtures (ints, scales, sums) from the compiled reference core
 *   orc_prep_x16            : golden fixtures from the compiled reference core
 *   orc_partials_q8_128     : numpy int64 matmul of decoded ints x activation ints
 *   orc_gemv_q8_128_f64     : the reference's per-(row, half-slice) formula in fp64 (CPU.patch:3951-4016);
 *                             cross-checked against the compiled reference vrc_tile within fp32 rounding
 *   orc_quantize_q8_1       : ggml block_q8_1 (third-party, llama.cpp @7ac59a6, not vendored):
 *                             parity unpinned beyond its published definition; closed-form checks only
 */
#ifndef P8X_ORACLE_H
#define P8X_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* class tables, CPU.patch:188-195 */
int orc_w1(int c);
int orc_w2(int c);
int orc_w3(int c);
int orc_sh1(int c);
int orc_sh2(int c);
int orc_nw(int c);
int orc_nstage(int c);
int orc_mc(int c);

float    orc_h2f(uint16_t h);
uint16_t orc_f2h(float f);

/* Parsed view of one native tensor slot (CPU.patch:25-51, :234-275). Owns ic and the delta CSR. */
typedef struct orc_tensor {
    const uint8_t *base;
    size_t n;
    int rows, K, nb, ng, nsl, nd;
    size_t nt, kbytes;
    const uint32_t *A;      /* 256 codebook words (int8 x4) */
    uint32_t cs;            /* coset vector c (int8 x4) */
    const uint32_t *M;      /* tile words: payload word offset | class << 29 */
    const uint16_t *S;      /* fp16 scales [nb][rows] (sorted rows) */
    const uint32_t *D;      /* payload */
    const uint16_t *c16;    /* per-column scale c, fp16 [K] */
    const int16_t *prm;     /* sorted row -> original row */
    const int16_t *pinv;    /* original row -> sorted row */
    const int8_t *sg;       /* Hadamard signs [256] */
    const uint16_t *drow, *dcol; const float *dval;  /* clamp delta (original indices) */
    float *ic;              /* sg / c per column [K] */
    int *cp; uint16_t *cc; float *cv;                /* delta CSR by original row */
} orc_tensor;

/* 0 = ok; 1 = trailer/shape mismatch; 2 = header NS/TRL; 3 = kbytes beyond side data; 4 = kbytes != M-implied size */
int  orc_open(orc_tensor *t, const uint8_t *base, size_t n, int rows, int K);
void orc_close(orc_tensor *t);
size_t orc_need(size_t kbytes, size_t rows, size_t K, size_t nd);
void orc_offsets(size_t n, size_t rows, size_t K, size_t nd, size_t off[6]);  /* E, C, P, Q, SG, T */

/* trellis: chunk-order stage-1 MSB word -> chunk-order coset word (bit t = h_t) */
uint32_t orc_trellis_word(uint32_t z);
uint32_t orc_trellis_serial(uint32_t z);

/* bit-by-bit per-weight integer (independent of the word-parallel decoder) */
int orc_weight_int(const orc_tensor *t, int r_sorted, int col);

/* block decode of tile (g, b): exact ints, [32 lanes][256 natural columns] */
void orc_decode_tile(const orc_tensor *t, int g, int b, int16_t *out);
/* whole tensor ints, sorted rows, natural columns: [rows][K] */
void orc_decode_all(const orc_tensor *t, int16_t *out);
/* original-domain f32 weights, [rows][K] by ORIGINAL row (dequantize_row) */
void orc_dequant_f32(const orc_tensor *t, float *W);

void orc_fwht256(float *v);
/* x' = FWHT256(x * ic)/16, q8 per 128 (reference layout: q[K], d[K/128], sx[K/128]) */
void orc_prep_q8_128(const orc_tensor *t, const float *x, int8_t *q, float *d, int32_t *sx);
/* x16 precision mode: q = 128 hi + lo per 128, d = amax/8191 (hi plane scale 128 d, lo plane d) */
void orc_prep_x16(const orc_tensor *t, const float *x, int8_t *qh, float *dh, int32_t *sh, int8_t *ql, float *dl, int32_t *sl);
/* x' quantized to ggml block_q8_1 (36 B blocks: fp16 d, fp16 s, 32 x int8) */
void orc_quantize_q8_1(const orc_tensor *t, const float *x, uint8_t *blocks);
/* rotated activation x' in f32 */
void orc_rotate_act(const orc_tensor *t, const float *x, float *xr);

/* integer partial per (sorted row, half-slice): sum over the 128 columns of v * q */
void orc_partials_q8_128(const orc_tensor *t, const int8_t *q, int32_t *isum /* [rows][K/128] */);
/* integer partial per (sorted row, 32-col block) against q8_1 blocks */
void orc_partials_q8_1(const orc_tensor *t, const uint8_t *blocks, int32_t *isum /* [rows][K/32] */);
/* fp64 GEMV: y[prm[r]] = sum_s S*XS*isum + delta . x (original rows) */
void orc_gemv_q8_128_f64(const orc_tensor *t, const float *x, double *y);
void orc_gemv_q8_1_f64(const orc_tensor *t, const float *x, double *y);
/* fp64 GEMV on the x16 planes (hi scaled 128 d, lo scaled d), planes summed before the clamp delta */
void orc_gemv_x16_f64(const orc_tensor *t, const float *x, double *y);
/* orc_gemv_q8_128_f64 for ncols columns x [ncols][ldx] -> y [ncols][rows] (each tile decoded once) */
void orc_gemv_q8_128_f64_cols(const orc_tensor *t, const float *x, int ncols, size_t ldx, double *y);
/* fp64 dense product with the f32-dequantized weights (prompt GEMM reference): y[n][r] = W[r] . x[n] */
void orc_dense_f64(const float *W, int rows, int K, const float *x, int N, double *y);

#ifdef __cplusplus
}
#endif
#endif
