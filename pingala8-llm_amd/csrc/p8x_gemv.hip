// p8x_gemv.hip -- activation prep and the fused decode + GEMV (batch 1..8) for gfx950.
//
// Activation prep restates k_vr_qx_real / vrc_prep_block (CPU.patch:4292-4307, :559-571): per 256-block
// x' = FWHT256(x * ic) / 16 with the reference's butterfly operands, then 8-bit per 128-column half-slice
// (d = amax / 127, q = round-half-even(x' / d)). One wave per 256-block: lane l holds x'[4l .. 4l+3];
// butterflies h = 1, 2 are in registers, h = 4 .. 128 cross lanes (l ^ h/4).
//
// GEMV: persistent workgroups of 8 waves build the 64 KB replicated coset table once, then walk work
// items (row group g, K-chunk of `bpk` 256-blocks). A wave decodes one tile per step (p8x_lane.h) and
// takes v_dot4 products of the looked-up int8x4 codewords (coset already folded in) with the activation
// chunk, which is an LDS broadcast because chunk order is the same in every lane. Per lane-slice:
// isum = sum_s dot_s << SH_s (CPU.patch:646-662); y_row += float(isum) * d * S. The two half-slices of a
// row meet through one cross-lane add, the 8 waves of an item through LDS, and the K-chunks of a row group
// through a fixed-order fix-up by the last-arriving workgroup, so results are deterministic (the reference
// accumulates with float atomics, CPU.patch:4014).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <vector>

#include "p8x_gemv.h"

namespace p8x {

// ------------------------------------------------------------------------------------------------ activation prep
// grid (nb, ncols), block 64
__global__ __launch_bounds__(64) void k_act_q8_128(const float *__restrict__ x, size_t ldx, const float *__restrict__ ic, int K,
                                                   int8_t *__restrict__ q, float *__restrict__ d, int32_t *__restrict__ sum) {
    const int b = blockIdx.x, n = blockIdx.y, lane = threadIdx.x;
    uint32_t packed;
    float dd;
    int s;
    quantize_block_q8_128(x + (size_t)n * ldx + 256 * b, ic + 256 * b, lane, packed, dd, s);
    reinterpret_cast<uint32_t *>(q + (size_t)n * K + 256 * b)[lane] = packed;
    s = half_wave_sum(s, lane);
    const int nsl = K / 128;
    if ((lane & 31) == 0) {
        d[(size_t)n * nsl + 2 * b + (lane >> 5)] = dd;
        if (sum) sum[(size_t)n * nsl + 2 * b + (lane >> 5)] = s;
    }
}

// x16 precision mode (vrc_prep_block16, CPU.patch:575-616): per 128-column half, d = max|x'| / 8191, q = round-half-even
// (x' * (1/d)) (14 bits), split q = 128 hi + lo with hi = (q + 64) >> 7: two int8 planes scaled 128 d and d. grid (nb,
// ncols), block 64 (lane l: x' elements 4l .. 4l+3); outputs like k_act_q8_128 per plane.
__global__ __launch_bounds__(64) void k_act_x16(const float *__restrict__ x, size_t ldx, const float *__restrict__ ic, int K,
                                                int8_t *__restrict__ qh, float *__restrict__ dh, int32_t *__restrict__ sh,
                                                int8_t *__restrict__ ql, float *__restrict__ dl, int32_t *__restrict__ sl, int qstride) {
    const int b = blockIdx.x, n = blockIdx.y, lane = threadIdx.x;
    BlockLane in;
    in.load(x + (size_t)n * ldx + 256 * b, ic + 256 * b, lane);
    float v[4];
    rotate_block_lane(in, lane, v);
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = half_wave_max(am, lane);
    const float dd = div_rn(am, 8191.f);
    const float id = dd > 0.f ? div_rn(1.f, dd) : 0.f;
    int hi[4], lo[4], s_hi = 0, s_lo = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int q = __float2int_rn(v[e] * id);
        hi[e] = (q + 64) >> 7;
        lo[e] = q - 128 * hi[e];
        s_hi += hi[e];
        s_lo += lo[e];
    }
    auto pack = [](const int (&a)[4]) {
        return (uint32_t)(uint8_t)a[0] | ((uint32_t)(uint8_t)a[1] << 8) | ((uint32_t)(uint8_t)a[2] << 16) | ((uint32_t)(uint8_t)a[3] << 24);
    };
    const size_t qo = (size_t)n * qstride + 256 * b;
    reinterpret_cast<uint32_t *>(qh + qo)[lane] = pack(hi);
    reinterpret_cast<uint32_t *>(ql + qo)[lane] = pack(lo);
    s_hi = half_wave_sum(s_hi, lane);
    s_lo = half_wave_sum(s_lo, lane);
    const int nsl = K / 128;
    if ((lane & 31) == 0) {
        const size_t so = (size_t)n * (qstride / 128) + 2 * b + (lane >> 5);
        dh[so] = 128.f * dd;
        dl[so] = dd;
        if (sh) sh[so] = s_hi;
        if (sl) sl[so] = s_lo;
    }
    (void)nsl;
}

// x16 products: y[n][ro] = (plane sums: hi column 2n + lo column 2n + 1, already in original rows) + the clamp delta
// of row ro on the original activations, as the reference sums its two planes then adds the delta (CPU.patch:1193)
__global__ __launch_bounds__(256) void k_x16_combine(const float *__restrict__ yv, int rows, const float *__restrict__ x, size_t ldx,
                                                     const int *__restrict__ cp, const uint16_t *__restrict__ cc, const float *__restrict__ cv,
                                                     float *__restrict__ y, size_t ldy) {
    const int ro = blockIdx.x * 256 + threadIdx.x, n = blockIdx.y;
    if (ro >= rows) return;
    float v = yv[(size_t)(2 * n) * rows + ro] + yv[(size_t)(2 * n + 1) * rows + ro];
    const float *xr = x + (size_t)n * ldx;
    for (int e = cp[ro]; e < cp[ro + 1]; ++e) v += cv[e] * xr[cc[e]];
    y[(size_t)n * ldy + ro] = v;
}

// out[r] = silu(g[r]) * u[r], silu(g) = g / (1 + e^-g) (ggml's swiglu): the gated input from two finished products
__global__ __launch_bounds__(256) void k_glu_rows(const float *__restrict__ g, const float *__restrict__ u, int rows, float *__restrict__ out) {
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r >= rows) return;
    const float gate = g[r], up = u[r];
    out[r] = gate / (1.0f + expf(-gate)) * up;
}

// block_q8_1 over x' (ggml layout: fp16 d, fp16 s = d * sum q, 32 int8). 8 lanes per 32-column block.
__global__ __launch_bounds__(64) void k_act_q8_1(const float *__restrict__ x, size_t ldx, const float *__restrict__ ic, int K,
                                                 uint8_t *__restrict__ blocks) {
    const int b = blockIdx.x, n = blockIdx.y, lane = threadIdx.x;
    uint32_t packed;
    float dd, s;
    quantize_block_q8_1(x + (size_t)n * ldx + 256 * b, ic + 256 * b, lane, packed, dd, s);
    uint8_t *blk = blocks + ((size_t)n * (K / 32) + 8 * b + (lane >> 3)) * 36;
    reinterpret_cast<uint32_t *>(blk + 4)[lane & 7] = packed;
    if ((lane & 7) == 0) *reinterpret_cast<uint32_t *>(blk) = (uint32_t)float_to_half(dd) | ((uint32_t)float_to_half(s) << 16);
}

// K-split of a single-GEMV launch: about one task per workgroup slot, at least two tiles per wave, chunks no
// larger than the LDS activation buffer allows.
int class_set(const size_t hist[8], bool in_order) {
    int m = 0;
    for (int c = 1; c < 8; ++c) if (hist[c]) m |= 1 << c;
    // a one-class set decodes whole runs as its class: only when no tile is class 0 (all-zero, skipped); its
    // row-group and task kernels compute payload offsets, so the tiles must also be in order (else the enclosing set)
    if (!hist[0] && in_order)
        for (int cm : {kCmC3, kCmC6})
            if ((m & ~cm) == 0) return cm;
    for (int cm : {kCmC234, kCmC2346})
        if ((m & ~cm) == 0) return cm;
    return kCmAll;
}

// K-chunks: enough that a chunk's activations (columns x blocks) fit the LDS buffer; one column also splits in
// two when the row groups fill at most half the CUs and K is long (e.g. ffn_down)
int rg_plan(const p8x_tensor *t, int ncols, int *kc) {
    const int kmax = kRgMaxBlocks / ncols;
    int nks = (t->nb + kmax - 1) / kmax;
    if (ncols == 1 && nks == 1 && 2 * t->ng <= num_cus() && t->nb >= 32) nks = 2;
    *kc = (t->nb + nks - 1) / nks;
    return (t->nb + *kc - 1) / *kc;
}

static int q81_cm(const p8x_tensor *t, int ncols) {
    return ncols == 1 && class_set(t->class_tiles, t->lin_words != 0) == kCmC3 ? kCmC3 : kCmAll;
}

GemvPlan gemv_plan(const p8x_tensor *t, int ncols, int act, bool partials) {
    GemvPlan p;
    const int cm = partials || act == P8X_ACT_X16 ? kCmAll : act == P8X_ACT_Q8_1 ? q81_cm(t, ncols) : class_set(t->class_tiles, t->lin_words != 0);
    p.gpt = gemv_waves(ncols, act, partials, cm);
    const int octets = (t->ng + p.gpt - 1) / p.gpt;
    const int slots = gemv_wg_per_cu(ncols, act, partials, cm) * num_cus();
    int nks = (slots + octets - 1) / octets;
    nks = std::min(nks, std::max(1, t->nb / 2));
    nks = std::max(nks, (t->nb + kchunk_max(ncols) - 1) / kchunk_max(ncols));
    nks = std::min(nks, t->nb);
    p.bpk = (t->nb + nks - 1) / nks;
    p.nks = (t->nb + p.bpk - 1) / p.bpk;
    p.items = octets * p.nks;
    p.grid = std::min(p.items, slots);
    return p;
}


static void fill_job(GemvJob &g, const p8x_tensor *t, const void *q, const float *d, const float *x, size_t ldx,
                     float *y, size_t ldy, int32_t *partials, int nks, int kchunk, int gpt, int task0);

// the tensor's metadata as a GemvJob in device memory (activations, outputs and K plan unset), for launches that
// pick their job at run time
int upload_job(p8x_tensor *t) {
    GemvJob g;
    fill_job(g, t, nullptr, nullptr, nullptr, 0, nullptr, 0, nullptr, 1, t->nb, 1, 0);
    if (hipMalloc((void **)&t->djob, sizeof(GemvJob)) != hipSuccess) return set_error(P8X_ERR_NOMEM, "p8x_prepare: hipMalloc job");
    return hip_check(hipMemcpy(t->djob, &g, sizeof g, hipMemcpyHostToDevice), "p8x_prepare: job");
}

static void fill_job(GemvJob &g, const p8x_tensor *t, const void *q, const float *d, const float *x, size_t ldx,
                     float *y, size_t ldy, int32_t *partials, int nks, int kchunk, int gpt, int task0) {
    g = GemvJob{};
    g.M = t->M; g.S = t->Sg; g.D = t->D; g.prm = t->prm; g.prmd = t->prmd;
    g.cp = t->cp; g.cc = t->cc; g.cv = t->cv;
    g.q = q; g.d = d; g.x = x; g.ldx = (unsigned)ldx; g.y = y; g.ldy = (unsigned)ldy; g.partials = partials;
    g.wpart = t->wpart; g.wcnt = t->wcnt; g.wslot = t->wslot;
    g.rows = t->rows; g.K = t->K; g.nb = t->nb; g.ng = t->ng; g.nsl = t->nsl; g.lin = t->lin_words;
    g.kchunk = kchunk; g.nks = nks; g.task0 = task0; g.ntasks = ((t->ng + gpt - 1) / gpt) * nks;
    g.dbytes = (unsigned)(t->kbytes - offset_D(t->nt));
    g.ic = t->ic;
    g.g0 = 0; g.gend = t->ng; g.prows = t->rows;
}

// vec_dot over the row groups g0 .. g0 + ng - 1 with the whole tensor's plan (so the rows' results equal the whole
// call's): y at those groups' original rows, partials [ncols][32 ng][blocks]
int launch_gemv_range(const p8x_tensor *t, int act, const void *q, const float *d, int ncols, const float *x, size_t ldx,
                      float *y, size_t ldy, int32_t *partials, int g0, int ng, hipStream_t st) {
    const int cm = class_set(t->class_tiles, t->lin_words != 0);
    if (partials) {   // integer partials: one column per launch
        const GemvPlan p1 = gemv_plan(t, 1, act, true);
        if (p1.nks > 1 && (size_t)p1.nks * t->rows > t->wpart_floats) return set_error(P8X_ERR_UNSUPPORTED, "gemv: partial workspace too small");
        GemvJob job0;
        fill_job(job0, t, q, d, x, ldx, y, ldy, partials, p1.nks, p1.bpk, p1.gpt, 0);
        job0.g0 = g0; job0.gend = g0 + ng; job0.prows = 32 * ng;
        job0.ntasks = ((ng + p1.gpt - 1) / p1.gpt) * p1.nks;
        for (int n = 0; n < ncols; ++n) {
            GemvJob jn = job0;
            const size_t qcol = act == P8X_ACT_Q8_128 ? (size_t)t->K : (size_t)36 * (t->K / 32);
            jn.q = (const uint8_t *)q + n * qcol;
            if (d) jn.d = d + (size_t)n * t->nsl;
            if (x) jn.x = x + (size_t)n * ldx;
            jn.y = y + (size_t)n * ldy;
            jn.partials = partials + (size_t)n * 32 * ng * (act == P8X_ACT_Q8_128 ? t->nsl : t->K / 32);
            const int rc = launch_gemv_partials(act, jn, t->a2, st);
            if (rc) return rc;
        }
        return P8X_OK;
    }
    const GemvPlan p = gemv_plan(t, ncols, act, false);
    if (p.nks > 1 && (size_t)p.nks * ncols * t->rows > t->wpart_floats) return set_error(P8X_ERR_UNSUPPORTED, "gemv: partial workspace too small");
    GemvJob job0;
    fill_job(job0, t, q, d, x, ldx, y, ldy, nullptr, p.nks, p.bpk, p.gpt, 0);
    job0.g0 = g0; job0.gend = g0 + ng;
    job0.ntasks = ((ng + p.gpt - 1) / p.gpt) * p.nks;
    if (act == P8X_ACT_Q8_128) return launch_gemv_q8(ncols, cm, job0, job0.ntasks, t->a2, st);
    return launch_gemv_q81(ncols, q81_cm(t, ncols), job0, job0.ntasks, t->a2, st);
}

int launch_gemv(const p8x_tensor *t, int act, const void *q, const float *d, int ncols, const float *x, size_t ldx,
                float *y, size_t ldy, int32_t *partials, hipStream_t st) {
    const int cm = class_set(t->class_tiles, t->lin_words != 0);
    if (partials) return launch_gemv_range(t, act, q, d, ncols, x, ldx, y, ldy, partials, 0, t->ng, st);
    // the row-group kernel: one column, or two columns of a one-class tensor with K <= 8192 (measured faster
    // than the multi-column task kernel there, slower for longer K and more columns)
    if (act == P8X_ACT_Q8_128 && !q && (ncols == 1 || (ncols == 2 && t->nb <= 32 && (cm == kCmC3 || cm == kCmC6)))) {
        // one linear, x quantized in the launch
        int kc;
        const int nks = rg_plan(t, ncols, &kc);
        if (nks == 1 || (size_t)nks * ncols * t->rows <= t->wpart_floats) {
            RgJobs R{};
            fill_job(R.j0, t, nullptr, nullptr, x, ldx, y, ldy, nullptr, nks, kc, 1, 0);
            R.njobs = 1;
            return launch_gemv_rg(ncols, cm, R, t->ng, t->a2, st);
        }
    }
    const GemvPlan p = gemv_plan(t, ncols, act, false);
    if (p.nks > 1 && (size_t)p.nks * ncols * t->rows > t->wpart_floats) return set_error(P8X_ERR_UNSUPPORTED, "gemv: partial workspace too small");
    GemvJob job0;
    fill_job(job0, t, q, d, x, ldx, y, ldy, nullptr, p.nks, p.bpk, p.gpt, 0);
    if (act == P8X_ACT_Q8_128) return launch_gemv_q8(ncols, cm, job0, job0.ntasks, t->a2, st);
    return launch_gemv_q81(ncols, q81_cm(t, ncols), job0, job0.ntasks, t->a2, st);
}

// The row-group plan of several linears on the same activations (out == nullptr), or of a gate / up pair with the
// swiglu epilogue (out != nullptr: n == 2, tensors[0] = gate): jobs, workgroups per job, K-chunks. Also sets the
// class set of the tensors and their row groups in total. Shapes, codebook and rotation are checked by the caller.
int plan_gemv_multi(const p8x_tensor *const *ts, int n, const float *x, size_t ldx, float *const *y, const size_t *ldy, float *out,
                    RgJobs &R, int &cm, int &ng) {
    size_t hist[8] = {0};
    bool in_order = true;
    ng = 0;
    for (int i = 0; i < n; ++i) {
        for (int c = 0; c < 8; ++c) hist[c] += ts[i]->class_tiles[c];
        ng += ts[i]->ng;
        in_order = in_order && ts[i]->lin_words != 0;
    }
    cm = class_set(hist, in_order);
    // the K plan of the combined row groups: K-chunks that fit the LDS buffer, split in two when they fill at most
    // half the CUs and K is long (the single-call rule)
    const p8x_tensor *t0 = ts[0];
    int nks = (t0->nb + kRgMaxBlocks - 1) / kRgMaxBlocks;
    if (nks == 1 && 2 * ng <= num_cus() && t0->nb >= 32) nks = 2;
    const int kc = (t0->nb + nks - 1) / nks;
    nks = (t0->nb + kc - 1) / kc;
    R = RgJobs{};
    R.njobs = n;
    fill_job(R.j0, t0, nullptr, nullptr, x, ldx, out ? nullptr : y[0], out ? 0 : ldy[0], nullptr, nks, kc, 1, 0);
    // workgroups per job: ceil(its row groups / per) per K-chunk, with per = ceil(all row groups / CUs)
    const int per = (ng + num_cus() - 1) / num_cus();
    for (int i = 0; i <= kRgMaxJobs; ++i) R.wgbase[i] = 0x7FFFFFFF;
    R.wgbase[0] = 0;
    for (int i = 0; i < n; ++i) {
        if (nks > 1 && (size_t)nks * ts[i]->rows > ts[i]->wpart_floats) return set_error(P8X_ERR_UNSUPPORTED, "multi GEMV: partial workspace too small");
        R.jt[i] = (kptr<const GemvJob>)ts[i]->djob;
        R.y[i] = out ? nullptr : y[i];
        R.ldy[i] = out ? 0u : (unsigned)ldy[i];
        R.wgbase[i + 1] = R.wgbase[i] + (ts[i]->ng + per - 1) / per * nks;
    }
    for (int i = n; i < kRgMaxJobs; ++i) R.jt[i] = (kptr<const GemvJob>)ts[0]->djob;   // never selected
    R.wgbase[kRgMaxJobs] = R.wgbase[n];   // the total
    if (out) {
        R.glu = 1;
        R.glu_out = out;
        R.glu_slot = t0->wglu;
    }
    return P8X_OK;
}

int launch_gemv_multi(const p8x_tensor *const *ts, int n, const float *x, size_t ldx, float *const *y, const size_t *ldy, float *out,
                      hipStream_t st) {
    RgJobs R;
    int cm = 0, ng = 0;
    const int rc = plan_gemv_multi(ts, n, x, ldx, y, ldy, out, R, cm, ng);
    if (rc) return rc;
    return launch_gemv_rg_multi(cm, R, ng, ts[0]->a2, st);
}

// ------------------------------------------------------------------------------------------------ grouped launches
struct ActJob {
    const float *x; unsigned ldx; const float *ic; int K, nb;
    int8_t *q;             // [ncols][nb] blocks in the broadcast layout of k_act_q8_128_batch
    int blk0;              // first 256-block of this job in the launch
};

// grid (ceil(total blocks / 4), ncols), block 256: the k_act_q8_128 body for a list of jobs, one 256-block per
// wave; blk_job gives each block's job. Output in the grouped kernel's broadcast layout (kBcastBlockBytes per block
// and column): entry (hs, i) at hs * 256 + 16 i holds {word i, word 16 + i, d, 0} of half hs (word t = the four
// int8 of chunk t, d = the half's scale as f32), so a lane of row r = 2 hs + (0|1) loads everything its tile needs
// from one column with one 16-byte load.
__global__ __launch_bounds__(256) void k_act_q8_128_batch(const ActJob *__restrict__ jobs, const uint32_t *__restrict__ blk_job, int total) {
    const int gb = 4 * blockIdx.x + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), n = blockIdx.y, lane = threadIdx.x & 63;
    if (gb >= total) return;
    const ActJob &J = jobs[as_const(blk_job)[gb]];
    const int b = gb - J.blk0;
    uint32_t packed;
    float dd;
    int s;
    quantize_block_q8_128(J.x + (size_t)n * J.ldx + 256 * b, J.ic + 256 * b, lane, packed, dd, s);
    const int hs = lane >> 5, t = lane & 31;
    uint32_t *e = reinterpret_cast<uint32_t *>(J.q + ((size_t)n * J.nb + b) * kBcastBlockBytes + 256 * hs + 16 * (t & 15));
    if (t < 16) {
        e[0] = packed;
        e[2] = __builtin_bit_cast(uint32_t, dd);
        e[3] = 0u;
    } else {
        e[1] = packed;
    }
}

// The same prep in the matrix-core kernel's layout (k_gemv_wave_mx): column n's block b as the 256-byte record
// (b ncols + n) (the int8 of half 0, then half 1), the halves' scales after all records at [b][n][2].
__global__ __launch_bounds__(256) void k_act_q8_128_mx_batch(const ActJob *__restrict__ jobs, const uint32_t *__restrict__ blk_job, int total) {
    const int gb = 4 * blockIdx.x + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), n = blockIdx.y, lane = threadIdx.x & 63;
    if (gb >= total) return;
    const ActJob &J = jobs[as_const(blk_job)[gb]];
    const int b = gb - J.blk0, ncols = (int)gridDim.y;
    uint32_t packed;
    float dd;
    int s;
    quantize_block_q8_128(J.x + (size_t)n * J.ldx + 256 * b, J.ic + 256 * b, lane, packed, dd, s);
    const int hs = lane >> 5, t = lane & 31;
    const size_t rec = (size_t)b * ncols + n;
    reinterpret_cast<uint32_t *>(J.q + rec * kMxRecBytes + 128 * hs)[t] = packed;
    if (t == 0) reinterpret_cast<float *>(J.q + (size_t)ncols * J.nb * kMxRecBytes)[2 * rec + hs] = dd;
}

// The x16 form of the batch prep (P8X_ACT_X16, the arithmetic of k_act_x16): grid (ceil(total blocks / 4), ncols),
// column n's two planes written as virtual columns 2n (hi, scale 128 d) and 2n + 1 (lo, scale d) of the broadcast
// layout (MX false) or of the matrix-core kernel's records (MX true, 2 ncols virtual columns), so the grouped kernel
// multiplies them as 2 ncols columns.
template <bool MX>
__global__ __launch_bounds__(256) void k_act_x16_batch(const ActJob *__restrict__ jobs, const uint32_t *__restrict__ blk_job, int total) {
    const int gb = 4 * blockIdx.x + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), n = blockIdx.y, lane = threadIdx.x & 63;
    if (gb >= total) return;
    const ActJob &J = jobs[as_const(blk_job)[gb]];
    const int b = gb - J.blk0;
    BlockLane in;
    in.load(J.x + (size_t)n * J.ldx + 256 * b, J.ic + 256 * b, lane);
    float v[4];
    rotate_block_lane(in, lane, v);
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = half_wave_max(am, lane);
    const float dd = div_rn(am, 8191.f);
    const float id = dd > 0.f ? div_rn(1.f, dd) : 0.f;
    uint32_t ph = 0, pl = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int q = __float2int_rn(v[e] * id);
        const int hi = (q + 64) >> 7, lo = q - 128 * hi;
        ph |= (uint32_t)(uint8_t)hi << (8 * e);
        pl |= (uint32_t)(uint8_t)lo << (8 * e);
    }
    const int hs = lane >> 5, t = lane & 31;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        if constexpr (MX) {
            const int ncv = 2 * (int)gridDim.y;
            const size_t rec = (size_t)b * ncv + 2 * n + p;
            reinterpret_cast<uint32_t *>(J.q + rec * kMxRecBytes + 128 * hs)[t] = p ? pl : ph;
            if (t == 0) reinterpret_cast<float *>(J.q + (size_t)ncv * J.nb * kMxRecBytes)[2 * rec + hs] = p ? dd : 128.f * dd;
        } else {
            uint32_t *e = reinterpret_cast<uint32_t *>(J.q + ((size_t)(2 * n + p) * J.nb + b) * kBcastBlockBytes + 256 * hs + 16 * (t & 15));
            if (t < 16) {
                e[0] = p ? pl : ph;
                e[2] = __builtin_bit_cast(uint32_t, p ? dd : 128.f * dd);
                e[3] = 0u;
            } else {
                e[1] = p ? pl : ph;
            }
        }
    }
}

// Finishing launch of a grouped GEMV. Rows that carry clamp-delta entries (bit 15 of prmd) go to the first blocks,
// one thread per such row: it sums the row's K-chunk partials in chunk order and adds its delta entries (resolved at
// batch creation, so its loads do not wait on one another beyond the activation gather); these blocks come first so
// that their chain of dependent loads overlaps the plain blocks instead of ending the launch. The plain blocks take
// 1024 sorted rows of one job each (4 per thread): per column, sorted row r sums its K-chunk partials in chunk order
// (coalesced reads, four chunks' loads issued together) and is written to its original row prmd[r] (a scatter
// inside the job's output). Plain block 8k + x runs on XCD x (workgroups go to the XCDs round robin by index, and
// the delta blocks are padded to a multiple of 8), and every plain block of a job is on one XCD, so the job's
// output lines fill in one L2. Block table entries: job | 1024-row block of the job << 24, or kFinNone (padding).
constexpr int kFinRows = 1024;
constexpr uint32_t kFinNone = 0xFFFFFFFFu;

struct FinishJob {
    const float *wpart; const int16_t *pinv; const uint16_t *prmd;
    const int *cp; const uint16_t *cc; const float *cv; const float *x;
    float *y;
    unsigned ldx, ldy;   // column strides of x and y
    int rows, nks, ncol;
    int planes;          // 1: x16, the partials hold 2 ncol virtual columns (hi 2n, lo 2n + 1) and column n is their sum
};

// a row with clamp-delta entries, resolved when the batch is created: its sorted row (partials) and original
// row, and its entries [e0, e1) of the batch's (column, value) list
struct FinDelta { int job, r, ro, e0, e1; };
struct FinEntry { int col; float val; };

__global__ __launch_bounds__(256) void k_gemv_finish(const FinishJob *__restrict__ jobs, const uint32_t *__restrict__ blk_job, int ndblk,
                                                     const FinDelta *__restrict__ drows, const FinEntry *__restrict__ ent, int ndrows) {
    if ((int)blockIdx.x < ndblk) {
        const int i = (int)blockIdx.x * 256 + threadIdx.x;
        if (i >= ndrows) return;
        const FinDelta d = drows[i];
        const FinishJob &J = jobs[d.job];
        const gptr<const float> wp = as_global(J.wpart);
        const int ncv = J.planes ? 2 * J.ncol : J.ncol;
        auto colsum = [&](int c) {
            float v = 0.f;
            for (int ks = 0; ks < J.nks; ++ks) v += wp[((size_t)ks * ncv + c) * J.rows + d.r];
            return v;
        };
        for (int n = 0; n < J.ncol; ++n) {
            float v = J.planes ? colsum(2 * n) + colsum(2 * n + 1) : colsum(n);   // x16: the two planes, then the delta
            if (J.x) {
                const gptr<const float> x = as_global(J.x) + (size_t)n * J.ldx;
                for (int e = d.e0; e < d.e1; ++e) v += as_global(ent)[e].val * x[as_global(ent)[e].col];
            }
            as_global_rw(J.y)[(size_t)n * J.ldy + d.ro] = v;
        }
        return;
    }
    const uint32_t e = as_const(blk_job)[blockIdx.x - ndblk];
    if (e == kFinNone) return;
    const FinishJob &J = jobs[e & 0xFFFFFFu];
    const int r0 = (int)(e >> 24) * kFinRows + threadIdx.x;
    const gptr<const float> wp = as_global(J.wpart);
    const int ncv = J.planes ? 2 * J.ncol : J.ncol;
    int r[4];
    uint32_t pd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r[i] = min(r0 + 256 * i, J.rows - 1);
        pd[i] = as_global(J.prmd)[r[i]];
    }
    // virtual column c of the four rows summed over the K-chunks in chunk order (four chunks' loads issued together)
    auto colsum = [&](int c, float (&v)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = 0.f;
        for (int k0 = 0; k0 < J.nks; k0 += 4) {
            float p[4][4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int i = 0; i < 4; ++i) p[k][i] = k0 + k < J.nks ? wp[((size_t)(k0 + k) * ncv + c) * J.rows + r[i]] : 0.f;
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (k0 + k < J.nks) v[i] += p[k][i];
        }
    };
    for (int n = 0; n < J.ncol; ++n) {
        float v[4];
        if (J.planes) {
            float lo[4];
            colsum(2 * n, v);
            colsum(2 * n + 1, lo);
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] += lo[i];
        } else {
            colsum(n, v);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (r0 + 256 * i < J.rows && !(pd[i] & 0x8000u)) as_global_rw(J.y)[(size_t)n * J.ldy + pd[i]] = v[i];
    }
}

int check_shared_input(const p8x_tensor *const *ts, int n, const float *x, size_t ldx, const char *what) {
    for (int i = 0; i < n; ++i) {
        if (!ts[i]) return set_error(P8X_ERR_ARG, "%s: tensor %d is null", what, i);
        // one tensor twice would share its workspace (K-chunk partial rows, meeting slots) between two jobs
        for (int k = 0; k < i; ++k)
            if (ts[k] == ts[i]) return set_error(P8X_ERR_ARG, "%s: tensor %d is listed twice", what, k);
        if (ts[i]->K != ts[0]->K) return set_error(P8X_ERR_ARG, "%s: tensor %d has K %d, tensor 0 has %d", what, i, ts[i]->K, ts[0]->K);
        if (memcmp(ts[i]->a2_host, ts[0]->a2_host, sizeof ts[0]->a2_host))
            return set_error(P8X_ERR_UNSUPPORTED, "%s: tensor %d has a different codebook", what, i);
        if (ts[i]->ic_hash != ts[0]->ic_hash || ts[i]->ic_host.size() != ts[0]->ic_host.size() ||
            memcmp(ts[i]->ic_host.data(), ts[0]->ic_host.data(), 4 * ts[0]->ic_host.size()))
            return set_error(P8X_ERR_UNSUPPORTED, "%s: tensor %d rotates its input differently (column scales c or signs); call it alone", what, i);
    }
    if (!x || ldx < (size_t)ts[0]->K || ldx % 4 || ((uintptr_t)x & 15))
        return set_error(P8X_ERR_ARG, "%s: x null or ldx %zu (x 16-byte aligned, ldx %% 4 == 0)", what, ldx);
    return P8X_OK;
}

}  // namespace p8x

struct p8x_gemv_batch {
    int njobs = 0, ncols = 1, cm = 0, total_tasks = 0, total_blocks = 0;
    int act = P8X_ACT_Q8_128, ncv = 1;   // activation mode; columns the grouped kernel multiplies (x16: 2 ncols planes)
    int split_jobs = 0, small_launch = 0, waves = 0;   // plan facts reported by p8x_gemv_batch_info
    bool mx = false;               // the matrix-core kernel (and its activation layout)
    unsigned *ctr = nullptr;       // its unit counters (in work)
    uint32_t *d_ujob = nullptr;    // unit -> job
    p8x::FinishJob *d_fin = nullptr;   // finishing launch (one column)
    uint32_t *d_fblk = nullptr;        // its block -> job
    p8x::FinDelta *d_fdrows = nullptr; // its rows with clamp-delta entries
    p8x::FinEntry *d_fent = nullptr;   // and their (column, value) entries
    int fin_blocks = 0, fin_ndrows = 0;
    const uint32_t *a2 = nullptr;
    p8x::GemvJob *d_jobs = nullptr;
    p8x::ActJob *d_act = nullptr;
    uint32_t *d_ablk = nullptr;        // activation prep: 256-block -> job
    void *work = nullptr;   // activations, partial rows and counters of every job
};

using namespace p8x;

extern "C" {

void p8x_gemv_batch_release(p8x_gemv_batch *b) {
    if (!b) return;
    if (b->d_jobs) (void)hipFree(b->d_jobs);
    if (b->d_act) (void)hipFree(b->d_act);
    if (b->d_ablk) (void)hipFree(b->d_ablk);
    if (b->d_ujob) (void)hipFree(b->d_ujob);
    if (b->d_fin) (void)hipFree(b->d_fin);
    if (b->d_fblk) (void)hipFree(b->d_fblk);
    if (b->d_fdrows) (void)hipFree(b->d_fdrows);
    if (b->d_fent) (void)hipFree(b->d_fent);
    if (b->work) (void)hipFree(b->work);
    delete b;
}

int p8x_gemv_batch_create(const p8x_tensor *const *tensors, const float *const *x, const size_t *ldx,
                          float *const *y, const size_t *ldy, int njobs, int ncols, p8x_gemv_batch **out) {
    return p8x_gemv_batch_create_act(tensors, x, ldx, y, ldy, njobs, ncols, P8X_ACT_Q8_128, out);
}

int p8x_gemv_batch_create_act(const p8x_tensor *const *tensors, const float *const *x, const size_t *ldx,
                              float *const *y, const size_t *ldy, int njobs, int ncols, int act, p8x_gemv_batch **out) {
    return p8x_gemv_batch_create_ex(tensors, x, ldx, y, ldy, njobs, ncols, act, P8X_GEMV_KERNEL_AUTO, out);
}

int p8x_gemv_batch_create_ex(const p8x_tensor *const *tensors, const float *const *x, const size_t *ldx,
                             float *const *y, const size_t *ldy, int njobs, int ncols, int act, int kernel, p8x_gemv_batch **out) {
    if (kernel != P8X_GEMV_KERNEL_AUTO && kernel != P8X_GEMV_KERNEL_DOT4 && kernel != P8X_GEMV_KERNEL_MFMA)
        return set_error(P8X_ERR_ARG, "p8x_gemv_batch_create: kernel %d", kernel);
    if (!tensors || !x || !ldx || !y || !ldy || !out || njobs < 1) return set_error(P8X_ERR_ARG, "p8x_gemv_batch_create: bad arguments");
    if (njobs >= (1 << 24)) return set_error(P8X_ERR_ARG, "p8x_gemv_batch_create: %d jobs (at most %d)", njobs, (1 << 24) - 1);
    if (ncols < 1 || ncols > P8X_MAX_COLS) return set_error(P8X_ERR_ARG, "p8x_gemv_batch_create: ncols %d", ncols);
    if (act != P8X_ACT_Q8_128 && act != P8X_ACT_X16) return set_error(P8X_ERR_ARG, "p8x_gemv_batch_create: act %d (P8X_ACT_Q8_128 or P8X_ACT_X16)", act);
    if (act == P8X_ACT_X16 && 2 * ncols > P8X_MAX_COLS) return set_error(P8X_ERR_ARG, "p8x_gemv_batch_create: x16 takes at most %d columns", P8X_MAX_COLS / 2);
    const int ncv = act == P8X_ACT_X16 ? 2 * ncols : ncols;   // the grouped kernel's columns (x16: both planes)
    *out = nullptr;
    size_t hist[8] = {0};
    for (int i = 0; i < njobs; ++i) {
        const p8x_tensor *t = tensors[i];
        if (!t || !x[i] || !y[i]) return set_error(P8X_ERR_ARG, "p8x_gemv_batch_create: job %d has a null pointer", i);
        if (ldx[i] < (size_t)t->K || ldx[i] % 4 || ((uintptr_t)x[i] & 15) || ldy[i] < (size_t)t->rows)
            return set_error(P8X_ERR_ARG, "p8x_gemv_batch_create: job %d strides/alignment", i);
        if (memcmp(t->a2_host, tensors[0]->a2_host, sizeof t->a2_host))
            return set_error(P8X_ERR_UNSUPPORTED, "p8x_gemv_batch_create: job %d has a different codebook", i);
        for (int c = 0; c < 8; ++c) hist[c] += t->class_tiles[c];
    }
    // workspace layout: unit counters | per job: activations [ncv][nb] in the broadcast layout | partials
    // [nks][ncv][rows]
    std::vector<GemvJob> jobs(njobs);
    std::vector<ActJob> ajobs(njobs);
    std::vector<size_t> off_q(njobs), off_p(njobs);
    size_t bytes = 0;
    auto take = [&](size_t n) { const size_t o = bytes; bytes = align16(bytes + n); return o; };
    const size_t off_ctr = take(kWaveCtrBytes);
    int blk0 = 0;
    std::vector<uint32_t> ablk;   // activation prep: 256-block -> job
    const int cm = class_set(hist);
    // class-3 batches of kMxMinCols..8 columns (x16: virtual columns, two per column) run on the matrix cores unless
    // the caller chose a kernel (the same bits either way)
    if (kernel == P8X_GEMV_KERNEL_MFMA && !wave_mx(cm, ncv))
        return set_error(P8X_ERR_UNSUPPORTED, "p8x_gemv_batch_create: the matrix-core kernel takes class-3 batches of 2..8 multiplied columns");
    const bool mx = kernel == P8X_GEMV_KERNEL_MFMA || (kernel == P8X_GEMV_KERNEL_AUTO && wave_mx(cm, ncv) && ncv >= kMxMinCols);
    const int launch_waves = mx ? mx_wg_per_cu() * num_cus() * mx_waves() : wave_wg_per_cu(cm, ncv) * num_cus() * wave_waves(cm, ncv);
    // wave-independent units: (row group, whole K)
    std::vector<int> kcs(njobs);
    bool small_launch = false;
    for (int i = 0; i < njobs; ++i) kcs[i] = tensors[i]->nb;
    {
        // Units are handed out longest first, so the launch drains on the units of the last jobs. Those jobs are
        // split along K (units of >= 4 blocks, partial rows summed by the finishing launch) until about two
        // rounds of the launch's waves have short units to finish on.
        const long need = 2L * launch_waves;
        std::vector<int> order(njobs);
        for (int i = 0; i < njobs; ++i) order[i] = i;
        std::stable_sort(order.begin(), order.end(), [&](int a, int c) { return tensors[a]->nb > tensors[c]->nb; });
        long have = 0;
        for (int r = njobs - 1; r >= 0 && have < need; --r) {
            const p8x_tensor *t = tensors[order[r]];
            const int nks = std::min(4, std::max(1, t->nb / 4));
            kcs[order[r]] = (t->nb + nks - 1) / nks;
            have += (long)t->ng * ((t->nb + kcs[order[r]] - 1) / kcs[order[r]]);
        }
        // a small launch (one layer, say) still has fewer units than waves: every job in units of two blocks or
        // more, so that more waves stream (the finishing launch sums up to 16 chunks per row)
        small_launch = have < need;
        if (small_launch)
            for (int i = 0; i < njobs; ++i) {
                const int nks = std::min(16, std::max(1, tensors[i]->nb / 2));
                kcs[i] = (tensors[i]->nb + nks - 1) / nks;
            }
    }
    for (int i = 0; i < njobs; ++i) {
        const p8x_tensor *t = tensors[i];
        const int kc = kcs[i];
        const int nks = (t->nb + kc - 1) / kc;
        off_q[i] = take((size_t)ncv * t->nb * kBcastBlockBytes);   // also holds the matrix-core layout (mx_act_bytes)
        off_p[i] = take(4 * (size_t)nks * ncv * t->rows);   // partial rows (the finishing launch reads them)
        fill_job(jobs[i], t, nullptr, nullptr, x[i], ldx[i], y[i], ldy[i], nullptr, nks, kc, 1, 0);
        ajobs[i] = ActJob{x[i], (unsigned)ldx[i], t->ic, t->K, t->nb, nullptr, blk0};
        blk0 += t->nb;
        ablk.insert(ablk.end(), (size_t)t->nb, (uint32_t)i);
    }
    p8x_gemv_batch *b = new p8x_gemv_batch();
    b->njobs = njobs; b->ncols = ncols; b->cm = cm; b->total_blocks = blk0;
    b->act = act; b->ncv = ncv;
    b->a2 = tensors[0]->a2;
    int rc;
    if (hipMalloc(&b->work, bytes) != hipSuccess || hipMalloc((void **)&b->d_jobs, sizeof(GemvJob) * njobs) != hipSuccess ||
        hipMalloc((void **)&b->d_act, sizeof(ActJob) * njobs) != hipSuccess || hipMalloc((void **)&b->d_ablk, 4 * (size_t)blk0) != hipSuccess) {
        p8x_gemv_batch_release(b);
        return set_error(P8X_ERR_NOMEM, "p8x_gemv_batch_create: hipMalloc");
    }
    uint8_t *w = (uint8_t *)b->work;
    b->ctr = (unsigned *)(w + off_ctr);
    for (int i = 0; i < njobs; ++i) {
        jobs[i].q = w + off_q[i];
        jobs[i].d = nullptr;
        ajobs[i].q = (int8_t *)(w + off_q[i]);
        jobs[i].wpart = (float *)(w + off_p[i]);
        jobs[i].wcnt = nullptr;
    }
    std::map<const uint32_t *, const p8x_tensor *> tensor_of;   // the sorted jobs find their tensor by M
    for (int i = 0; i < njobs; ++i) tensor_of[tensors[i]->M] = tensors[i];
    // task numbering: longest units (most blocks per unit) first, so that dynamic scheduling ends on short ones
    std::stable_sort(jobs.begin(), jobs.end(), [](const GemvJob &a, const GemvJob &c) {
        return std::min(a.kchunk, a.nb) > std::min(c.kchunk, c.nb);
    });
    int task0 = 0;
    for (auto &j : jobs) { j.task0 = task0; task0 += j.ntasks; }
    b->total_tasks = task0;
    b->small_launch = small_launch;
    b->waves = launch_waves;
    b->mx = mx;
    for (int i = 0; i < njobs; ++i) b->split_jobs += kcs[i] < tensors[i]->nb;
    {
        // unit -> job table
        std::vector<uint32_t> uj((size_t)task0);
        for (int i = 0; i < njobs; ++i)
            for (int u = 0; u < jobs[i].ntasks; ++u) uj[(size_t)jobs[i].task0 + u] = (uint32_t)i;
        std::vector<FinishJob> fin(njobs);
        std::vector<FinDelta> fdr;
        std::vector<FinEntry> fent;
        // jobs to XCDs, largest first onto the least loaded; then block 8k + x = the k-th block of XCD x's jobs
        std::vector<std::vector<uint32_t>> xb(kXcds);
        std::vector<int> order(njobs);
        for (int i = 0; i < njobs; ++i) order[i] = i;
        std::stable_sort(order.begin(), order.end(), [&](int a, int c) { return jobs[a].rows > jobs[c].rows; });
        for (int i : order) {
            const GemvJob &g = jobs[i];
            size_t x = 0;
            for (size_t k = 1; k < xb.size(); ++k) if (xb[k].size() < xb[x].size()) x = k;
            for (int r = 0, s = 0; r < g.rows; r += kFinRows, ++s) xb[x].push_back((uint32_t)i | ((uint32_t)s << 24));
        }
        size_t per = 0;
        for (const auto &l : xb) per = std::max(per, l.size());
        std::vector<uint32_t> fblk(kXcds * per, kFinNone);
        for (int x = 0; x < kXcds; ++x)
            for (size_t k = 0; k < xb[x].size(); ++k) fblk[kXcds * k + x] = xb[x][k];
        for (int i = 0; i < njobs; ++i) {
            const GemvJob &g = jobs[i];
            const p8x_tensor *t = tensor_of[g.M];
            fin[i] = FinishJob{g.wpart, t->pinv, t->prmd, g.cp, g.cc, g.cv, g.x, g.y, g.ldx, g.ldy, g.rows, g.nks, ncols, act == P8X_ACT_X16 ? 1 : 0};
            if (t->dorig.empty()) continue;
            // the tensor's delta CSR and inverse permutation, read back once (set-up time)
            std::vector<int> cp(t->rows + 1);
            std::vector<int16_t> pinv(t->rows);
            std::vector<uint16_t> cc(std::max(1, t->nd));
            std::vector<float> cv(std::max(1, t->nd));
            if ((rc = hip_check(hipMemcpy(cp.data(), t->cp, 4 * cp.size(), hipMemcpyDeviceToHost), "p8x_gemv_batch_create: delta rows")) ||
                (rc = hip_check(hipMemcpy(pinv.data(), t->pinv, 2 * pinv.size(), hipMemcpyDeviceToHost), "p8x_gemv_batch_create: delta rows")) ||
                (t->nd > 0 && (rc = hip_check(hipMemcpy(cc.data(), t->cc, 2 * (size_t)t->nd, hipMemcpyDeviceToHost), "p8x_gemv_batch_create: delta rows"))) ||
                (t->nd > 0 && (rc = hip_check(hipMemcpy(cv.data(), t->cv, 4 * (size_t)t->nd, hipMemcpyDeviceToHost), "p8x_gemv_batch_create: delta rows")))) {
                p8x_gemv_batch_release(b);
                return rc;
            }
            for (int ro : t->dorig) {
                const int e0 = (int)fent.size();
                for (int e = cp[ro]; e < cp[ro + 1]; ++e) fent.push_back(FinEntry{(int)cc[e], cv[e]});
                fdr.push_back(FinDelta{i, (int)pinv[ro], ro, e0, (int)fent.size()});
            }
        }
        b->fin_blocks = (int)fblk.size();
        b->fin_ndrows = (int)fdr.size();
        if (hipMalloc((void **)&b->d_fin, sizeof(FinishJob) * njobs) != hipSuccess ||
            hipMalloc((void **)&b->d_fblk, 4 * fblk.size()) != hipSuccess ||
            hipMalloc((void **)&b->d_fdrows, sizeof(FinDelta) * std::max<size_t>(1, fdr.size())) != hipSuccess ||
            hipMalloc((void **)&b->d_fent, sizeof(FinEntry) * std::max<size_t>(1, fent.size())) != hipSuccess) {
            p8x_gemv_batch_release(b);
            return set_error(P8X_ERR_NOMEM, "p8x_gemv_batch_create: finishing jobs");
        }
        if ((rc = hip_check(hipMemcpy(b->d_fin, fin.data(), sizeof(FinishJob) * njobs, hipMemcpyHostToDevice), "p8x_gemv_batch_create: finishing jobs")) ||
            (rc = hip_check(hipMemcpy(b->d_fblk, fblk.data(), 4 * fblk.size(), hipMemcpyHostToDevice), "p8x_gemv_batch_create: finishing blocks")) ||
            (!fdr.empty() && (rc = hip_check(hipMemcpy(b->d_fdrows, fdr.data(), sizeof(FinDelta) * fdr.size(), hipMemcpyHostToDevice),
                                             "p8x_gemv_batch_create: finishing delta rows"))) ||
            (!fent.empty() && (rc = hip_check(hipMemcpy(b->d_fent, fent.data(), sizeof(FinEntry) * fent.size(), hipMemcpyHostToDevice),
                                              "p8x_gemv_batch_create: finishing delta entries")))) {
            p8x_gemv_batch_release(b);
            return rc;
        }
        if (hipMalloc((void **)&b->d_ujob, 4 * uj.size()) != hipSuccess) {
            p8x_gemv_batch_release(b);
            return set_error(P8X_ERR_NOMEM, "p8x_gemv_batch_create: unit table");
        }
        if ((rc = hip_check(hipMemcpy(b->d_ujob, uj.data(), 4 * uj.size(), hipMemcpyHostToDevice), "p8x_gemv_batch_create: unit table"))) {
            p8x_gemv_batch_release(b);
            return rc;
        }
    }
    if ((rc = hip_check(hipMemset(b->work, 0, bytes), "p8x_gemv_batch_create: clear")) ||
        (rc = hip_check(hipMemcpy(b->d_jobs, jobs.data(), sizeof(GemvJob) * njobs, hipMemcpyHostToDevice), "p8x_gemv_batch_create: jobs")) ||
        (rc = hip_check(hipMemcpy(b->d_act, ajobs.data(), sizeof(ActJob) * njobs, hipMemcpyHostToDevice), "p8x_gemv_batch_create: act jobs")) ||
        (rc = hip_check(hipMemcpy(b->d_ablk, ablk.data(), 4 * ablk.size(), hipMemcpyHostToDevice), "p8x_gemv_batch_create: act blocks"))) {
        p8x_gemv_batch_release(b);
        return rc;
    }
    *out = b;
    return P8X_OK;
}

int p8x_gemv_batch_run_stage(const p8x_gemv_batch *b, int stage, void *stream) {
    return p8x_gemv_batch_run_stage_timed(b, stage, stream, nullptr, nullptr);
}

int p8x_gemv_batch_run_stage_timed(const p8x_gemv_batch *b, int stage, void *stream, void *ev_start, void *ev_stop) {
    if (!b) return set_error(P8X_ERR_ARG, "p8x_gemv_batch_run: null batch");
    hipStream_t st = (hipStream_t)stream;
    hipEvent_t e0 = (hipEvent_t)ev_start, e1 = (hipEvent_t)ev_stop;
    if (stage == 0) {
        const dim3 grid((b->total_blocks + 3) / 4, b->ncols);
        auto kern = b->act == P8X_ACT_X16 ? (b->mx ? k_act_x16_batch<true> : k_act_x16_batch<false>)
                                          : b->mx ? k_act_q8_128_mx_batch : k_act_q8_128_batch;
        if (e0 || e1)
            hipExtLaunchKernelGGL(kern, grid, dim3(256), 0, st, e0, e1, 0, (const ActJob *)b->d_act, (const uint32_t *)b->d_ablk, b->total_blocks);
        else
            hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, (const ActJob *)b->d_act, (const uint32_t *)b->d_ablk, b->total_blocks);
        return hip_check(hipGetLastError(), "batch activation prep launch");
    }
    if (stage == 1) {
        if (b->mx) return launch_gemv_wave_mx(b->ncv, b->d_jobs, b->d_ujob, b->total_tasks, b->ctr, b->a2, st, e0, e1);
        return launch_gemv_wave(b->ncv, b->cm, b->d_jobs, b->d_ujob, b->total_tasks, b->ctr, b->a2, st, e0, e1);
    }
    if (stage == 2) {   // partial rows to original rows with the clamp delta
        // the delta blocks first, padded to a multiple of the XCD count so plain block 8k + x still lands on XCD x
        const int ndblk = (b->fin_ndrows + 255) / 256, ndpad = (ndblk + kXcds - 1) / kXcds * kXcds;
        const dim3 grid(ndpad + b->fin_blocks);
        if (e0 || e1)
            hipExtLaunchKernelGGL(k_gemv_finish, grid, dim3(256), 0, st, e0, e1, 0, (const FinishJob *)b->d_fin, (const uint32_t *)b->d_fblk, ndpad,
                                  (const FinDelta *)b->d_fdrows, (const FinEntry *)b->d_fent, b->fin_ndrows);
        else
            hipLaunchKernelGGL(k_gemv_finish, grid, dim3(256), 0, st, (const FinishJob *)b->d_fin, (const uint32_t *)b->d_fblk, ndpad,
                               (const FinDelta *)b->d_fdrows, (const FinEntry *)b->d_fent, b->fin_ndrows);
        return hip_check(hipGetLastError(), "k_gemv_finish launch");
    }
    return set_error(P8X_ERR_ARG, "p8x_gemv_batch_run_stage: stage %d", stage);
}


int p8x_mul_mat_vec_multi(const p8x_tensor *const *tensors, int n, const float *x, size_t ldx, float *const *y, const size_t *ldy, void *stream) {
    if (!tensors || !y || !ldy || n < 1 || n > kRgMaxJobs) return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec_multi: bad arguments (1..%d tensors)", kRgMaxJobs);
    int rc;
    if ((rc = check_shared_input(tensors, n, x, ldx, "p8x_mul_mat_vec_multi"))) return rc;
    for (int i = 0; i < n; ++i)
        if (!y[i] || ldy[i] < (size_t)tensors[i]->rows) return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec_multi: y %d null or short", i);
    return launch_gemv_multi(tensors, n, x, ldx, y, ldy, nullptr, (hipStream_t)stream);
}

// The shared-input calls with another activation mode. Q8_1: each tensor's block_q8_1 GEMV quantizes x in its own
// launch (every tensor rotates its input the same way, so the blocks are the same); X16: the planes are prepared once
// (in tensor 0's workspace) and each tensor multiplies them as two columns into its plane rows, then its combine
// (planes summed, then the delta).
static int multi_act(const p8x_tensor *const *ts, int n, int act, const float *x, size_t ldx, float *const *y, const size_t *ldy, hipStream_t st) {
    const p8x_tensor *t0 = ts[0];
    int rc;
    if (act == P8X_ACT_Q8_1) {   // each GEMV's tasks quantize their chunks (the tensors share the rotation)
        for (int i = 0; i < n; ++i)
            if ((rc = launch_gemv(ts[i], P8X_ACT_Q8_1, nullptr, nullptr, 1, x, ldx, y[i], ldy[i], nullptr, st))) return rc;
        return P8X_OK;
    }
    if ((rc = launch_act_x16(t0, x, 1, ldx, t0->wq, t0->wd, nullptr, t0->wq + t0->K, t0->wd + t0->nsl, nullptr, 2 * t0->K, st))) return rc;
    for (int i = 0; i < n; ++i) {
        const p8x_tensor *t = ts[i];
        if ((rc = launch_gemv(t, P8X_ACT_Q8_128, t0->wq, t0->wd, 2, nullptr, 0, t->wy, t->rows, nullptr, st))) return rc;
        hipLaunchKernelGGL(k_x16_combine, dim3((t->rows + 255) / 256, 1), dim3(256), 0, st, (const float *)t->wy, t->rows, x, ldx,
                           (const int *)t->cp, (const uint16_t *)t->cc, (const float *)t->cv, y[i], ldy[i]);
        if ((rc = hip_check(hipGetLastError(), "k_x16_combine launch"))) return rc;
    }
    return P8X_OK;
}

int p8x_mul_mat_vec_multi_act(const p8x_tensor *const *tensors, int n, int act, const float *x, size_t ldx, float *const *y, const size_t *ldy,
                              void *stream) {
    if (act == P8X_ACT_Q8_128) return p8x_mul_mat_vec_multi(tensors, n, x, ldx, y, ldy, stream);
    if (act != P8X_ACT_Q8_1 && act != P8X_ACT_X16) return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec_multi_act: act %d", act);
    if (!tensors || !y || !ldy || n < 1 || n > kRgMaxJobs) return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec_multi_act: bad arguments (1..%d tensors)", kRgMaxJobs);
    int rc;
    if ((rc = check_shared_input(tensors, n, x, ldx, "p8x_mul_mat_vec_multi_act"))) return rc;
    for (int i = 0; i < n; ++i)
        if (!y[i] || ldy[i] < (size_t)tensors[i]->rows) return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec_multi_act: y %d null or short", i);
    return multi_act(tensors, n, act, x, ldx, y, ldy, (hipStream_t)stream);
}

int p8x_mul_mat_vec_glu_act(const p8x_tensor *gate, const p8x_tensor *up, int act, const float *x, size_t ldx, float *out, void *stream) {
    if (act == P8X_ACT_Q8_128) return p8x_mul_mat_vec_glu(gate, up, x, ldx, out, stream);
    if (act != P8X_ACT_Q8_1 && act != P8X_ACT_X16) return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec_glu_act: act %d", act);
    const p8x_tensor *ts[2] = {gate, up};
    if (!gate || !up || !out) return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec_glu_act: null pointer");
    int rc;
    if ((rc = check_shared_input(ts, 2, x, ldx, "p8x_mul_mat_vec_glu_act"))) return rc;
    if (gate->rows != up->rows) return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec_glu_act: gate has %d rows, up %d", gate->rows, up->rows);
    // the two products in original rows in each tensor's plane rows past the x16 planes (row block 2), then the gate
    hipStream_t st = (hipStream_t)stream;
    float *const ys[2] = {gate->wy + 2 * (size_t)gate->rows, up->wy + 2 * (size_t)up->rows};
    const size_t ldys[2] = {(size_t)gate->rows, (size_t)up->rows};
    if ((rc = multi_act(ts, 2, act, x, ldx, ys, ldys, st))) return rc;
    hipLaunchKernelGGL(k_glu_rows, dim3((gate->rows + 255) / 256), dim3(256), 0, st, (const float *)ys[0], (const float *)ys[1], gate->rows, out);
    return hip_check(hipGetLastError(), "k_glu_rows launch");
}

int p8x_mul_mat_vec_glu(const p8x_tensor *gate, const p8x_tensor *up, const float *x, size_t ldx, float *out, void *stream) {
    const p8x_tensor *ts[2] = {gate, up};
    if (!gate || !up || !out) return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec_glu: null pointer");
    int rc;
    if ((rc = check_shared_input(ts, 2, x, ldx, "p8x_mul_mat_vec_glu"))) return rc;
    if (gate->rows != up->rows) return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec_glu: gate has %d rows, up %d", gate->rows, up->rows);
    return launch_gemv_multi(ts, 2, x, ldx, nullptr, nullptr, out, (hipStream_t)stream);
}

int p8x_gemv_batch_info(const p8x_gemv_batch *b, p8x_batch_info *out) {
    if (!b || !out) return set_error(P8X_ERR_ARG, "p8x_gemv_batch_info: null pointer");
    out->njobs = b->njobs; out->ncols = b->ncols; out->class_set = b->cm; out->units = b->total_tasks;
    out->split_jobs = b->split_jobs; out->small_launch = b->small_launch; out->waves = b->waves; out->matrix_cores = b->mx ? 1 : 0;
    return P8X_OK;
}

int p8x_gemv_batch_run(const p8x_gemv_batch *b, void *stream) {
    int rc = 0;
    for (int stage = 0; stage < 3 && !rc; ++stage) rc = p8x_gemv_batch_run_stage(b, stage, stream);
    return rc;
}

}  // extern "C"

namespace p8x {

int launch_act_q8_128(const p8x_tensor *t, const float *x, int ncols, size_t ldx, int8_t *q, float *d, int32_t *sum, hipStream_t st) {
    hipLaunchKernelGGL(k_act_q8_128, dim3(t->nb, ncols), dim3(64), 0, st, x, ldx, (const float *)t->ic, t->K, q, d, sum);
    return hip_check(hipGetLastError(), "k_act_q8_128 launch");
}

int launch_act_x16(const p8x_tensor *t, const float *x, int ncols, size_t ldx, int8_t *qh, float *dh, int32_t *sh, int8_t *ql, float *dl,
                   int32_t *sl, int qstride, hipStream_t st) {
    hipLaunchKernelGGL(k_act_x16, dim3(t->nb, ncols), dim3(64), 0, st, x, ldx, (const float *)t->ic, t->K, qh, dh, sh, ql, dl, sl, qstride);
    return hip_check(hipGetLastError(), "k_act_x16 launch");
}

// x16 products of ncols <= 4 columns: both planes of every column quantized into the handle's workspace as 2 ncols
// virtual columns (hi of column n at 2n, lo at 2n + 1), one 8-bit-per-128 GEMV over them into the plane rows, then
// the combine pass
int launch_gemv_x16(const p8x_tensor *t, const float *x, int ncols, size_t ldx, float *y, size_t ldy, hipStream_t st) {
    return launch_gemv_x16_on(t, x, ncols, ldx, y, ldy, t->wq, t->wd, false, st);
}

// the same with the planes' buffers given (q [2 ncols][K], d [2 ncols][nsl]); have: they already hold x's planes
int launch_gemv_x16_on(const p8x_tensor *t, const float *x, int ncols, size_t ldx, float *y, size_t ldy, int8_t *q, float *d, bool have,
                       hipStream_t st) {
    int rc;
    if (!have && (rc = launch_act_x16(t, x, ncols, ldx, q, d, nullptr, q + t->K, d + t->nsl, nullptr, 2 * t->K, st))) return rc;
    if ((rc = launch_gemv(t, P8X_ACT_Q8_128, q, d, 2 * ncols, nullptr, 0, t->wy, t->rows, nullptr, st))) return rc;
    hipLaunchKernelGGL(k_x16_combine, dim3((t->rows + 255) / 256, ncols), dim3(256), 0, st, (const float *)t->wy, t->rows, x, ldx,
                       (const int *)t->cp, (const uint16_t *)t->cc, (const float *)t->cv, y, ldy);
    return hip_check(hipGetLastError(), "k_x16_combine launch");
}

// ---------------------------------------------------------------------------------------- prepared-activation reuse
// The activation most recently prepared by a call in x16 or block_q8_1 mode, kept for later calls on the same input
// within one graph evaluation (p8x_graph_begin): one file-scope device array per GPU (no allocation; its address
// from hipGetSymbolAddress, resolved at prepare), a host-side key per device.
static __device__ __align__(256) uint8_t act_cache[kActCacheBytes];

struct ActKey {
    unsigned epoch = 0;
    const float *x = nullptr;
    size_t ldx = 0;
    int ncols = 0, act = -1, K = 0;
    uint64_t ic_hash = 0;
    const void *stream = nullptr;
    bool operator==(const ActKey &o) const {
        return epoch == o.epoch && x == o.x && ldx == o.ldx && ncols == o.ncols && act == o.act && K == o.K && ic_hash == o.ic_hash &&
               stream == o.stream;
    }
};
static std::mutex g_act_mu;
static void *g_act_buf[kMaxActDevices];
static ActKey g_act_key[kMaxActDevices];
static std::atomic<unsigned> g_epoch{0};

int act_cache_resolve(int device) {
    if (device < 0 || device >= kMaxActDevices) return set_error(P8X_ERR_UNSUPPORTED, "activation cache: device %d beyond %d", device, kMaxActDevices);
    std::lock_guard<std::mutex> lk(g_act_mu);
    if (g_act_buf[device]) return P8X_OK;
    int cur = 0, rc;
    if ((rc = hip_check(hipGetDevice(&cur), "activation cache: hipGetDevice"))) return rc;
    if (cur != device && (rc = hip_check(hipSetDevice(device), "activation cache: hipSetDevice"))) return rc;
    void *ptr = nullptr;
    rc = hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(act_cache)), "activation cache: hipGetSymbolAddress");
    if (cur != device) (void)hipSetDevice(cur);
    if (rc) return rc;
    g_act_buf[device] = ptr;
    return P8X_OK;
}

void act_epoch_advance() { g_epoch.fetch_add(1u, std::memory_order_relaxed); }

uint8_t *act_reuse(const p8x_tensor *t, int act, const float *x, int ncols, size_t ldx, size_t bytes, hipStream_t st, bool *have) {
    *have = false;
    const unsigned ep = g_epoch.load(std::memory_order_relaxed);
    if (ep == 0 || bytes > kActCacheBytes || t->device < 0 || t->device >= kMaxActDevices) return nullptr;
    ActKey k;
    k.epoch = ep; k.x = x; k.ldx = ldx; k.ncols = ncols; k.act = act; k.K = t->K; k.ic_hash = t->ic_hash; k.stream = st;
    std::lock_guard<std::mutex> lk(g_act_mu);
    if (!g_act_buf[t->device]) return nullptr;
    *have = g_act_key[t->device] == k;
    g_act_key[t->device] = k;
    return static_cast<uint8_t *>(g_act_buf[t->device]);
}

int launch_act_q8_1(const p8x_tensor *t, const float *x, int ncols, size_t ldx, void *blocks, hipStream_t st) {
    hipLaunchKernelGGL(k_act_q8_1, dim3(t->nb, ncols), dim3(64), 0, st, x, ldx, (const float *)t->ic, t->K, (uint8_t *)blocks);
    return hip_check(hipGetLastError(), "k_act_q8_1 launch");
}

}  // namespace p8x
