/*
 * ref_driver.c -- C entry points around the reference's own CPU core (vr-native-cpu-core.h),
 * which oracle/Makefile extracts from patches/llama_cpu_vs_7ac59a6.patch into oracle/_ref/src/.
 *
 * TEST INFRASTRUCTURE ONLY: used to write the golden fixtures in tests/golden/ and as the
 * CPU baseline of bench.py. The multi-threaded GEMV driver restates the reference's ggml glue
 * (CPU.patch:1161-1199 vrc_tg, :1201-1262 ggml_vr_cpu_mul_mat): phase 1 prepares the activation
 * per 256-block over the threads, a barrier, then phase 2 hands out 32-row groups from an
 * atomic counter; each group is un-permuted and gets its clamp delta. The ggml threadpool it
 * used is replaced by a small pthread pool.
 */
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "vr-native-cpu-core.h"

const char *ref_isa(void) {
#if defined(__AVXVNNI__)
    return "avx2+avx-vnni (v4 tg path)";
#elif defined(__AVX2__)
    return "avx2 (lane-SIMD v2 path)";
#else
    return "scalar";
#endif
}

void *ref_open(const uint8_t *base, size_t n, int rows, int K, int *rc) {
    vrc_meta *m = (vrc_meta *)malloc(sizeof(vrc_meta));
    *rc = vrc_init(m, base, n, rows, K);
    if (*rc) { free(m); return NULL; }
    return m;
}

void ref_close(void *h) { vrc_meta *m = (vrc_meta *)h; vrc_free(m); free(m); }

void ref_decode_tile(void *h, int g, int b, int16_t *out) { vrc_decode_tile_int((const vrc_meta *)h, g, b, out); }

void ref_dequant(void *h, float *W) { vrc_dequant_f32((const vrc_meta *)h, W); }

void ref_prep_block(void *h, const float *x, int b, int8_t *X2, float *XS, int32_t *SX) {
    vrc_prep_block((const vrc_meta *)h, x, b, X2, XS, SX);
}

void ref_prep_block16(void *h, const float *x, int b, int8_t *Xh, float *XSh, int32_t *SXh, int8_t *Xl, float *XSl, int32_t *SXl) {
    vrc_prep_block16((const vrc_meta *)h, x, b, Xh, XSh, SXh, Xl, XSl, SXl);
}

void ref_tile(void *h, int g, int b, int ncol, const int8_t *X2, const float *XS, const int32_t *SX, float *accY) {
    static _Thread_local uint8_t tb[64 * 3 * 128];
    vrc_tile((const vrc_meta *)h, g, b, ncol, X2, XS, SX, accY, tb);
}

/* ------------------------------------------------------------------------------------------ thread pool */
typedef struct job {
    vrc_meta *m; const float *x; float *y; int np;
    int8_t *X; float *XS; int32_t *SX; uint32_t *LH;   /* plane p at p * nsl (contiguous planes) */
} job;

typedef struct pool {
    int nth;
    pthread_t *tid;
    pthread_barrier_t start, mid, done;
    job *jobs; int njobs; int quit;
    atomic_int cnt;
} pool;

typedef struct { pool *p; int ith; } warg;

static void run_job(pool *p, int ith, job *J) {
    const int nth = p->nth;
    vrc_meta *m = J->m;
    const int nb = m->nb, np = J->np;
    const size_t xps = (size_t)m->nsl * 256, sps = (size_t)m->nsl, lhs = (size_t)m->nsl * 16;
    for (int b = ith; b < nb; b += nth) {            /* phase 1 (CPU.patch:1170-1176) */
        if (np == 2)
            vrc_prep_block16(m, J->x, b, J->X + (size_t)2 * b * 256, J->XS + 2 * b, J->SX + 2 * b,
                             J->X + xps + (size_t)2 * b * 256, J->XS + sps + 2 * b, J->SX + sps + 2 * b);
        else
            vrc_prep_block(m, J->x, b, J->X + (size_t)2 * b * 256, J->XS + 2 * b, J->SX + 2 * b);
        for (int q = 0; q < np; ++q)
            for (int hs = 0; hs < 2; ++hs)
                vrc_prep_cx(m->cs, J->X + q * xps + (size_t)(2 * b + hs) * 256, J->LH + q * lhs + (size_t)(2 * b + hs) * 16);
    }
    if (ith == 0) atomic_store(&p->cnt, 0);
    pthread_barrier_wait(&p->mid);
    float accY[64 * 32] __attribute__((aligned(64)));
    for (int g = atomic_fetch_add(&p->cnt, 1); g < m->ng; g = atomic_fetch_add(&p->cnt, 1)) {   /* phase 2 */
        memset(accY, 0, sizeof(float) * 64);
#if defined(VRC_V4)
        if (np == 2) for (int b = 0; b < nb; ++b) vrc_tile_v4x(m, g, b, J->X, xps, J->XS, J->SX, sps, J->LH, lhs, accY);
        else for (int b = 0; b < nb; ++b) vrc_tile_v4(m, g, b, J->X, J->XS, J->SX, J->LH, accY);
#elif defined(__AVX2__)
        {
            __m256i tbv[96], acci[2];
            /* planes are virtual columns of the batch path (CPU.patch:1232-1244) */
            for (int b = 0; b < nb; ++b) vrc_tile_ls(m, g, b, np, J->X, J->XS, J->SX, accY, tbv, acci);
        }
#else
        {
            static _Thread_local uint8_t tb[64 * 3 * 128];
            for (int b = 0; b < nb; ++b) vrc_tile(m, g, b, np, J->X, J->XS, J->SX, accY, tb);
        }
#endif
        for (int j = 0; j < 32; ++j) {
            const int ro = m->prm[g * 32 + j];
#if defined(VRC_V4)
            float a = accY[j];
#else
            float a = np == 2 ? accY[j] + accY[32 + j] : accY[j];
#endif
            for (int e = m->cp[ro]; e < m->cp[ro + 1]; ++e) a += m->cv[e] * J->x[m->cc[e]];
            J->y[ro] = a;
        }
    }
}

static void *worker(void *arg) {
    warg *w = (warg *)arg;
    pool *p = w->p;
    for (;;) {
        pthread_barrier_wait(&p->start);
        if (p->quit) break;
        for (int i = 0; i < p->njobs; ++i) {
            run_job(p, w->ith, &p->jobs[i]);
            pthread_barrier_wait(&p->done);
        }
    }
    free(w);
    return NULL;
}

void *ref_pool_create(int nth) {
    pool *p = (pool *)calloc(1, sizeof(pool));
    p->nth = nth;
    p->tid = (pthread_t *)calloc((size_t)nth, sizeof(pthread_t));
    pthread_barrier_init(&p->start, NULL, (unsigned)nth + 1);
    pthread_barrier_init(&p->mid, NULL, (unsigned)nth);
    pthread_barrier_init(&p->done, NULL, (unsigned)nth + 1);
    for (int i = 0; i < nth; ++i) {
        warg *w = (warg *)malloc(sizeof(warg));
        w->p = p; w->ith = i;
        pthread_create(&p->tid[i], NULL, worker, w);
    }
    return p;
}

void ref_pool_destroy(void *hp) {
    pool *p = (pool *)hp;
    p->quit = 1;
    pthread_barrier_wait(&p->start);
    for (int i = 0; i < p->nth; ++i) pthread_join(p->tid[i], NULL);
    pthread_barrier_destroy(&p->start); pthread_barrier_destroy(&p->mid); pthread_barrier_destroy(&p->done);
    free(p->tid); free(p);
}

/* Run a sequence of GEMVs y_i = W_i x_i (np = 1: q8 activations, np = 2: x16 planes). Returns 0. */
int ref_gemv_seq(void *hp, void **metas, const float **xs, float **ys, int njobs, int np) {
    pool *p = (pool *)hp;
    int kmax = 0;
    for (int i = 0; i < njobs; ++i) if (((vrc_meta *)metas[i])->K > kmax) kmax = ((vrc_meta *)metas[i])->K;
    const size_t nsl = (size_t)kmax / 128;
    int8_t *X = (int8_t *)aligned_alloc(64, 2 * nsl * 256);
    float *XS = (float *)malloc(sizeof(float) * 2 * nsl);
    int32_t *SX = (int32_t *)malloc(sizeof(int32_t) * 2 * nsl);
    uint32_t *LH = (uint32_t *)aligned_alloc(64, sizeof(uint32_t) * 2 * nsl * 16);
    job *jobs = (job *)calloc((size_t)njobs, sizeof(job));
    for (int i = 0; i < njobs; ++i) {
        jobs[i].m = (vrc_meta *)metas[i]; jobs[i].x = xs[i]; jobs[i].y = ys[i]; jobs[i].np = np;
        jobs[i].X = X; jobs[i].XS = XS; jobs[i].SX = SX; jobs[i].LH = LH;
    }
    p->jobs = jobs; p->njobs = njobs;
    pthread_barrier_wait(&p->start);
    for (int i = 0; i < njobs; ++i) pthread_barrier_wait(&p->done);
    free(jobs); free(X); free(XS); free(SX); free(LH);
    return 0;
}
