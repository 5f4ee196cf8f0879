// p8x_gemv.h -- fused decode + GEMV kernel templates (instantiated in p8x_gemv_q8.hip / p8x_gemv_q8b.hip /
// p8x_gemv_q81.hip so the builds run in parallel).
//
// Persistent workgroups of 8 waves build the 64 KB replicated coset table once, then walk tasks
// (job, octet of 8 row groups, K-chunk). Each wave owns one row group over the task's K-chunk: no
// barrier or cross-wave reduction inside the main loop. Per tile, the wave decodes (p8x_lane.h) and takes
// v_dot4 products of the looked-up int8x4 codewords (coset folded in) with the activation chunk, an LDS
// broadcast because chunk order is the same in every lane. Per lane-slice: isum = sum_s dot_s << SH_s
// (CPU.patch:646-662); y_row += float(isum) * d * S. The next tile's payload is in flight while the
// current one is decoded. The two half-slices of a row meet through one cross-lane add; the K-chunks of a
// row group through a fixed-order fix-up by the last-arriving wave, so results are deterministic (the
// reference accumulates with float atomics, CPU.patch:4014).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <type_traits>

#include "p8x_act.h"
#include "p8x_internal.h"
#include "p8x_lane.h"

namespace p8x {

#ifndef GEMV_NBUF_C3
#define GEMV_NBUF_C3 3
#endif


// ------------------------------------------------------------------------------------------------ fused decode + GEMV
// One GEMV of a launch. A launch walks a list of these (one entry for p8x_mul_mat_vec, many for a grouped
// launch); tasks are numbered across the list: task = (job, octet of 8 row groups, K-chunk).
struct GemvJob {
    const uint32_t *M;
    const uint16_t *S;               // row scales regrouped by row group: [ng][nb][32]
    const uint32_t *D; const int16_t *prm;
    const uint16_t *prmd;            // prm with bit 15 set on rows that carry clamp-delta entries
    const int *cp; const uint16_t *cc; const float *cv;
    const void *q; const float *d;   // Q8_128: int8 [ncol][K] + f32 [ncol][K/128]; Q8_1: block_q8_1 [ncol][K/32];
                                     // grouped launches (k_gemv_wave): q in the broadcast layout, d unused
                                     // (Q8_128 with q null: each task quantizes its chunk of x itself, with ic)
    const float *ic;
    const float *x; unsigned ldx;    // original activations for the clamp delta (nullptr: no delta)
    float *y; unsigned ldy;
    int32_t *partials;               // optional integer partials (sorted rows)
    float *wpart; unsigned *wcnt;    // K-chunk partial rows [nks][ncol][rows] and arrival counters [ng]
    unsigned long long *wslot;       // one column in two K-chunks: per-row meeting slots [rows], 0 between calls
    int rows, K, nb, ng, nsl;
    unsigned lin;                    // one-class tensor with its tiles in order: payload words per tile (tile t at
                                     // word t * lin of D), else 0 (offsets from the tile words M)
    int kchunk, nks, task0, ntasks;
    unsigned dbytes;                 // payload region bytes (D .. end of the slot's payload)
    int g0, gend, prows;             // task kernel: row groups g0 .. gend - 1; partials rows (32 g0 ..) with row stride prows
};

// LDS activation bytes per task: ncol x kchunk x 512. The 16-byte-load kernels keep each 128-column half of a
// block at [n][block][half][64 words] (word i = chunk i, the second 32 words a copy that nothing reads; the
// staging writes whole 256-byte rows); the other kernels use the first half of each row pair. Every lane of a half
// reads chunk k at word k (a broadcast). Sized so that two workgroups (64 KB table + this + scales each) share one
// CU's 160 KB.
constexpr int kXBytes = 15360;

__host__ __device__ constexpr int kchunk_max(int ncol) { return kXBytes / (512 * ncol); }

template <int NCOL, int ACT>
struct GemvSmem {
    static constexpr int kScales = NCOL * (ACT == P8X_ACT_Q8_128 ? 2 : 8) * kchunk_max(NCOL);
    static constexpr int kXW = kXBytes / 4 / NCOL, kNSC = kScales / NCOL;   // per-column strides of xq, xd
    uint32_t tab[kTabWords];   // first member: LDS address 0, so table addresses need no base add
    uint32_t xq[kXBytes / 4];  // [ncol][kchunk][2][64] words (16-byte-load kernels) or [ncol][kchunk][64] words
    float xd[kScales];         // [ncol][scales of the chunk]
};

// class sets with their own instantiations: class 3 only (the 2-bit bulk), class 6 only (4-bit attn_v),
// classes 2-4 (mixed ffn_down), classes 2-4 and 6 (a whole model of the B4 mix), everything. The one-class sets
// decode every tile of a run as that class; the others read each tile's class (class 0 tiles are skipped).
constexpr int kCmC3 = 1 << 3, kCmC6 = 1 << 6, kCmC234 = (1 << 2) | (1 << 3) | (1 << 4), kCmC2346 = kCmC234 | (1 << 6), kCmAll = 0xFE;

// Waves per workgroup (each owns one row group of a task) and the waves per SIMD the registers are sized for.
// LDS holds two workgroups per CU; a variant that fits 64 VGPRs (one column, class 3, 16-byte loads) runs
// 16-wave workgroups, 8 waves per SIMD; the others 8-wave workgroups at 4 (<= 128 VGPRs) or 2 waves per SIMD.
__host__ __device__ constexpr int gemv_waves(int ncol, int act, bool partials, int cm) {
    return ncol == 1 && act == P8X_ACT_Q8_128 && !partials && cm == kCmC3 ? 16 : 8;
}
__host__ __device__ constexpr int gemv_waves_per_eu(int ncol, int act, bool partials, int cm) {
    return gemv_waves(ncol, act, partials, cm) == 16 ? 8 : ncol == 1 && cm == kCmC3 ? 4 : 2;
}
__host__ __device__ constexpr int gemv_wg_per_cu(int ncol, int act, bool partials, int cm) {
    return 4 * gemv_waves_per_eu(ncol, act, partials, cm) >= 2 * gemv_waves(ncol, act, partials, cm) ? 2 : 1;
}

template <int NCOL, int ACT>
struct TaskCtx {
    const GemvJob *J;   // the task's descriptor (kernel argument, or a copy of the launch's job array entry)
    int g, b0, nbl, hs, j;
    uint32_t bankbytes;
    int xlane;          // 16-byte-load kernels: the half's word offset hs * 64 in a block's activation words
};

// Q8_128 activations without integer partials load the payload in 16-byte groups (whole lines per instruction)
template <int ACT, bool PARTIALS>
__host__ __device__ constexpr bool gemv_quad_loads() { return ACT == P8X_ACT_Q8_128 && !PARTIALS; }

template <int NCOL, int ACT, bool PARTIALS, int C, typename SM>
__device__ __forceinline__ void gemv_tile(const TaskCtx<NCOL, ACT> &c, const SM &sm, const RawSlice<C> &raw, int b, float (&yacc)[NCOL]) {
    constexpr int NST = nstage_of(C), SH1 = sh1_of(C), SH2 = sh2_of(C);
    constexpr int NSUB = ACT == P8X_ACT_Q8_128 ? 1 : 4;   // integer sums per lane-slice
    constexpr int XW = SM::kXW;                            // LDS words per column
    constexpr int NSC = SM::kNSC;
    LaneSlice<C> ls;
    ls.from_raw(raw);
    ls.prepare(c.bankbytes);
    const int bl = b - c.b0;
    int acc[NST][NCOL][NSUB];
#pragma unroll
    for (int s = 0; s < NST; ++s)
#pragma unroll
        for (int n = 0; n < NCOL; ++n)
#pragma unroll
            for (int u = 0; u < NSUB; ++u) acc[s][n][u] = 0;
    const uint32_t *xbase = sm.xq + (bl * 256 + c.hs * 128) / 4;
#pragma unroll
    for (int t4 = 0; t4 < 8; ++t4) {
        uint4 xv[NCOL];
#pragma unroll
        for (int n = 0; n < NCOL; ++n) xv[n] = *reinterpret_cast<const uint4 *>(xbase + n * XW + 4 * t4);
        const uint32_t hq = ls.group_bytes(t4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = 4 * t4 + e;
            const int u = NSUB == 1 ? 0 : (t >> 3);
            uint32_t w[3];
            w[0] = lds_word(sm.tab, ls.template addr<0>(t, hq));
            if constexpr (NST > 1) w[1] = lds_word(sm.tab, ls.template addr<1>(t, hq));
            if constexpr (NST > 2) w[2] = lds_word(sm.tab, ls.template addr<2>(t, hq));
#pragma unroll
            for (int n = 0; n < NCOL; ++n) {
                const uint32_t xc = e == 0 ? xv[n].x : e == 1 ? xv[n].y : e == 2 ? xv[n].z : xv[n].w;
#pragma unroll
                for (int s = 0; s < NST; ++s) acc[s][n][u] = __builtin_amdgcn_sdot4((int)w[s], (int)xc, acc[s][n][u], false);
            }
        }
        __asm__ volatile("" ::: "memory");   // one group of 4 chunks at a time: bounds the live registers
    }
    const float sc = half_to_float(raw.s);
#pragma unroll
    for (int n = 0; n < NCOL; ++n) {
#pragma unroll
        for (int u = 0; u < NSUB; ++u) {
            int isum = acc[0][n][u] * (1 << SH1);
            if constexpr (NST > 1) isum += acc[1][n][u] * (1 << SH2);
            if constexpr (NST > 2) isum += acc[2][n][u];
            if constexpr (PARTIALS) {
                const int r = 32 * (c.g - c.J->g0) + c.j;
                if constexpr (ACT == P8X_ACT_Q8_128) as_global_rw(c.J->partials)[((size_t)n * c.J->prows + r) * c.J->nsl + 2 * b + c.hs] = isum;
                else as_global_rw(c.J->partials)[((size_t)n * c.J->prows + r) * (c.J->K / 32) + 8 * b + 4 * c.hs + u] = isum;
            }
            const float dsc = ACT == P8X_ACT_Q8_128 ? sm.xd[n * NSC + 2 * bl + c.hs] : sm.xd[n * NSC + 8 * bl + 4 * c.hs + u];
            yacc[n] += ((float)isum * dsc) * sc;
        }
    }
}

using lds_cptr = __attribute__((address_space(3))) const uint32_t *;

// Integer sums of one tile from 16-byte-group payload loads: every lane of a half reads activation chunk k of
// column n at xl[n * XW + k] (four chunks as one 16-byte LDS broadcast read), and looks up the codewords in the
// table at LDS 0.
template <int NCOL, int C, int XW>
__device__ __forceinline__ void quad_isum(const uint32_t *tab, const QuadSlice<C> &raw, uint32_t bankbytes, lds_cptr xl, int (&isum)[NCOL]) {
    constexpr int NST = nstage_of(C), SH1 = sh1_of(C), SH2 = sh2_of(C);
    const uint32_t H = raw.coset_bits();
    int acc[NST][NCOL];
#pragma unroll
    for (int s = 0; s < NST; ++s)
#pragma unroll
        for (int n = 0; n < NCOL; ++n) acc[s][n] = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        u32x4 xv[NCOL];
#pragma unroll
        for (int n = 0; n < NCOL; ++n) xv[n] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4 *>(xl + n * XW + 4 * q);
        const uint32_t hq = coset_bytes(H, bankbytes, q);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int k = 4 * q + e;
            uint32_t w[3];
            w[0] = lds_word(tab, raw.template addr<0>(k, hq));
            if constexpr (NST > 1) w[1] = lds_word(tab, raw.template addr<1>(k, hq));
            if constexpr (NST > 2) w[2] = lds_word(tab, raw.template addr<2>(k, hq));
#pragma unroll
            for (int n = 0; n < NCOL; ++n) {
                const uint32_t xc = e == 0 ? xv[n].x : e == 1 ? xv[n].y : e == 2 ? xv[n].z : xv[n].w;
#pragma unroll
                for (int s = 0; s < NST; ++s) acc[s][n] = __builtin_amdgcn_sdot4((int)w[s], (int)xc, acc[s][n], false);
            }
        }
        __asm__ volatile("" ::: "memory");   // one group of 4 chunks at a time: bounds the live registers
    }
#pragma unroll
    for (int n = 0; n < NCOL; ++n) {
        isum[n] = acc[0][n] * (1 << SH1);
        if constexpr (NST > 1) isum[n] += acc[1][n] * (1 << SH2);
        if constexpr (NST > 2) isum[n] += acc[2][n];
    }
}

// One tile from 16-byte-group payload loads (8-bit-per-128 activations, no partials)
template <int NCOL, int C, typename SM>
__device__ __forceinline__ void gemv_tile_quad(const TaskCtx<NCOL, P8X_ACT_Q8_128> &c, const SM &sm, const QuadSlice<C> &raw, int b,
                                               float (&yacc)[NCOL]) {
    constexpr int XW = SM::kXW;
    constexpr int NSC = SM::kNSC;
    const int bl = b - c.b0;
    // the tile's activation base in one register: left to itself the compiler folds the array's LDS offset
    // (64 KB, past the table) into every read, which then does not fit the read's offset field
    lds_cptr xl = (lds_cptr)(sm.xq + bl * 128 + c.xlane);
    __asm__ volatile("" : "+v"(xl));
    int isum[NCOL];
    quad_isum<NCOL, C, XW>(sm.tab, raw, c.bankbytes, xl, isum);
    const float sc = half_to_float(raw.s);
#pragma unroll
    for (int n = 0; n < NCOL; ++n) yacc[n] += ((float)isum[n] * sm.xd[n * NSC + 2 * bl + c.hs]) * sc;
}

// A run of consecutive tiles of class C in row group g: the run's extent is found from the tile words
// first, then NBUF register buffers rotate so that NBUF - 1 following tiles are in flight while the current
// one is decoded. Every step issues its prefetch (past the run's end through an empty resource, which reads
// zeros without memory traffic), so the loop body is straight-line and the wait counts stay exact.
// begin() finds the run and issues its first NBUF - 1 tiles; finish() decodes the run and returns the first
// block after it. Between the two the caller may do other work (the loads stay in flight).
template <int NCOL, int ACT, bool PARTIALS, int C, int NBUF, bool ONLY_C>
struct GemvRun {
    static constexpr int NW = nw_of(C);
    static constexpr bool QUAD = gemv_quad_loads<ACT, PARTIALS>();
    using Slice = std::conditional_t<QUAD, QuadSlice<C>, RawSlice<C>>;
    Slice buf[NBUF];
    int b, e;
    uint32_t wn;   // tile word of the next prefetch, read one step ahead so its scalar load is never waited on at once
    // lane part of the payload offsets: one base (16-byte groups) or the NW word offsets
    std::conditional_t<QUAD, uint32_t, uint32_t[NW]> vo;
    uint32_t vp;   // 16-byte groups: the lane's trailing-pair offset (classes with NW % 4 == 2)
    uint32_t vs;

    __device__ __forceinline__ kptr<const uint32_t> mrow(const TaskCtx<NCOL, ACT> &c) const {
        return as_const(c.J->M) + (size_t)c.g * c.J->nb;   // tile words: scalar loads
    }
    // one-class runs compute their payload offsets (the host picks a one-class instantiation only for tensors whose
    // tiles are in order, GemvJob::lin): no tile-word load ahead of the first tile
    __device__ __forceinline__ bool linear(const TaskCtx<NCOL, ACT> &) const { return ONLY_C; }
    __device__ __forceinline__ void issue(const TaskCtx<NCOL, ACT> &c, Slice &r, int ta) {
        const GemvJob &J = *c.J;
        const bool ok = ta < e;
        const int tc = ok ? ta : b;
        const uint32_t toff = linear(c) ? ((uint32_t)c.g * (uint32_t)J.nb + (uint32_t)tc) * J.lin * 4u : (wn & 0x1FFFFFFFu) * 4u;
        const uint32_t soff = ((uint32_t)c.g * (uint32_t)J.nb + (uint32_t)tc) * 64u;   // scales [g][b][32]
        const uint32_t sbytes = (uint32_t)J.nb * J.rows * 2u;
        __builtin_amdgcn_s_setprio(2);   // loads issued at raised priority (see wave_run)
        if constexpr (QUAD) r.load(buffer_rsrc(J.D, ok ? J.dbytes : 0u), toff, vo, vp, buffer_rsrc(J.S, ok ? sbytes : 0u), soff, vs);
        else r.load(buffer_rsrc(J.D, ok ? J.dbytes : 0u), toff, vo, buffer_rsrc(J.S, ok ? sbytes : 0u), soff, vs);
        __builtin_amdgcn_s_setprio(0);
        if (!linear(c)) wn = mrow(c)[min(ta + 1, e - 1)];
    }
    __device__ __forceinline__ void begin(const TaskCtx<NCOL, ACT> &c, int b_, int bend) {
        b = b_;
        e = bend;   // ONLY_C: every tile of the tensor has class C
        if constexpr (!ONLY_C) {
            e = b + 1;
            while (e < bend && (mrow(c)[e] >> 29) == (uint32_t)C) ++e;
        }
        if constexpr (QUAD) {
            vo = QuadSlice<C>::quad_offset(c.hs, c.j);
            vp = QuadSlice<C>::pair_offset(c.hs, c.j);
        } else {
            RawSlice<C>::lane_offsets((uint32_t)(c.hs * NW * 32), c.j, vo);
        }
        vs = 2u * (uint32_t)c.j;
        wn = linear(c) ? 0u : mrow(c)[b];
#pragma unroll
        for (int i = 0; i < NBUF - 1; ++i) issue(c, buf[i], b + i);
    }
    template <typename SM>
    __device__ __forceinline__ void tile(const TaskCtx<NCOL, ACT> &c, const SM &sm, const Slice &r0_, int t, float (&yacc)[NCOL]) {
        Slice r = r0_;
        pin(r.w);
        pin(r.s);
        if constexpr (QUAD) gemv_tile_quad<NCOL, C>(c, sm, r, t, yacc);
        else gemv_tile<NCOL, ACT, PARTIALS, C>(c, sm, r, t, yacc);
    }
    template <typename SM>
    __device__ __forceinline__ int finish(const TaskCtx<NCOL, ACT> &c, const SM &sm, float (&yacc)[NCOL]) {
        // whole groups of NBUF tiles: the loop body is straight-line, so the same loads are in flight at every
        // back edge
        int base = b;
        for (; base + NBUF <= e; base += NBUF) {
#pragma unroll
            for (int i = 0; i < NBUF; ++i) {
                issue(c, buf[(i + NBUF - 1) % NBUF], base + i + NBUF - 1);
                tile(c, sm, buf[i], base + i, yacc);
            }
        }
        // the last e - base < NBUF tiles are already in flight in buf[0 ..]
#pragma unroll
        for (int i = 0; i < NBUF - 1; ++i)
            if (base + i < e) tile(c, sm, buf[i], base + i, yacc);
        return e;
    }
};

template <int NCOL, int ACT, bool PARTIALS, int C, int NBUF, bool ONLY_C, typename SM>
__device__ __forceinline__ int gemv_run(const TaskCtx<NCOL, ACT> &c, const SM &sm, int b, int bend, float (&yacc)[NCOL]) {
    GemvRun<NCOL, ACT, PARTIALS, C, NBUF, ONLY_C> run;
    run.begin(c, b, bend);
    return run.finish(c, sm, yacc);
}

// prefetch depth (register buffers) per variant
__host__ __device__ constexpr int gemv_nbuf(int ncol, int c) { return ncol == 1 && c == 3 ? GEMV_NBUF_C3 : 2; }

// K-chunk fix-up publication. The chunk's partial rows go out as agent-scope atomic stores (on gfx950 these
// carry sc1: written through the XCD's L2 to the agent's coherence point, so a workgroup on another XCD sees
// them). A vector store counts against vmcnt until the memory system acknowledges it, and stores and atomics to
// different addresses may complete out of order, so the wave waits for vmcnt(0) before it counts its arrival:
// when another wave's arrival RMW returns a count that includes this one, these stores are complete. This is the
// agent-scope release of the AMDGPU memory model without its L2 write-back, which only plain (cached) stores
// need. The last arrival's loads are agent-scope atomic loads (sc1, served from the coherence point) issued after
// its RMW returned. Returns the counter's value before the increment (wave-uniform).
__device__ __forceinline__ unsigned arrive_after_stores(unsigned *ctr, int lane) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");   // partial-row stores complete before the arrival
    unsigned old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    __asm__ volatile("" ::: "memory");   // the partial loads that follow stay below the arrival
    return old;
}

// Two producers of one value (the two K-halves of a row, or a row's gate and up products) meet through one 64-bit
// agent-scope atomic exchange on the row's slot, which holds 0 between calls: each puts (1 + its index) << 32 |
// bits(value) there; the one that gets a nonzero old value arrived second, takes the partner's index and value from
// it and puts the slot back to 0. The value travels inside the RMW itself, so nothing has to be ordered before it
// (no separate partial store, no vmcnt wait, no counter): one memory round trip instead of three. The reset store
// is complete before anything later in the stream (kernel boundary) or in the step launch (the barrier's vmcnt(0))
// uses the slot again. Returns true for the second arrival, with the partner's index and value.
__device__ __forceinline__ bool pair_meet(gptr<unsigned long long> slot, int me, float v, int &other_idx, float &other) {
    const unsigned long long mine = ((unsigned long long)(1 + me) << 32) | __float_as_uint(v);
    const unsigned long long old = __hip_atomic_exchange(slot, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((old >> 32) == 0ull) return false;
    other_idx = (int)(old >> 32) - 1;
    other = __uint_as_float((uint32_t)old);
    __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// The row group's sums after one K-chunk: the two half-slices meet through one cross-lane add; the K-chunks of
// the row group meet in a fixed order (the last-arriving wave sums them), so results are deterministic; then the
// clamp delta and the row permutation on the way out.
template <int NCOL>
__device__ __forceinline__ void gemv_rows_out(const GemvJob &J, int g, int ks, int lane, float (&yacc)[NCOL]) {
    // global address-space views throughout: FLAT operations here would make the compiler wait for every
    // vector load at once in the tile loops (a pending FLAT access forces full waits)
    const int j = lane & 31;
    // half-slice 1 joins half-slice 0; lanes 0..31 hold the 32 rows
#pragma unroll
    for (int n = 0; n < NCOL; ++n) yacc[n] += __shfl_xor(yacc[n], 32);
    bool final_rows = J.nks == 1;
    if (J.nks > 1) {
        // K-chunk fix-up without agent-scope fences (on gfx950 those write back and invalidate the XCD's whole
        // L2): agent-coherent partial rows, the arrival counted once they are complete (arrive_after_stores), the
        // last arrival reads the partials with agent-coherent loads and sums them in chunk order.
        const gptr<float> wpart = as_global_rw(J.wpart);
        if (lane < 32)
#pragma unroll
            for (int n = 0; n < NCOL; ++n)
                __hip_atomic_store(&wpart[((size_t)ks * NCOL + n) * J.rows + 32 * g + j], yacc[n], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned old = arrive_after_stores(J.wcnt + g, lane);
        const gptr<unsigned> wcnt = as_global_rw(J.wcnt);
        final_rows = old == (unsigned)(J.nks - 1);
        if (final_rows) {
            if (lane < 32)
#pragma unroll
                for (int n = 0; n < NCOL; ++n) {
                    // issue 8 partial loads at a time (one memory round trip per 8 chunks), sum in chunk order
                    float sacc = 0.f;
                    for (int k0 = 0; k0 < J.nks; k0 += 8) {
                        float pv[8];
#pragma unroll
                        for (int i = 0; i < 8; ++i)
                            pv[i] = k0 + i < J.nks ? __hip_atomic_load(&wpart[((size_t)(k0 + i) * NCOL + n) * J.rows + 32 * g + j],
                                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
#pragma unroll
                        for (int i = 0; i < 8; ++i)
                            if (k0 + i < J.nks) sacc += pv[i];
                    }
                    yacc[n] = sacc;
                }
            if (lane == 0) __hip_atomic_store(&wcnt[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (final_rows && lane < 32) {
        const int ro = as_global(J.prm)[32 * g + j];
        const gptr<const int> cp = as_global(J.cp);
        const gptr<const uint16_t> cc = as_global(J.cc);
        const gptr<const float> cv = as_global(J.cv);
        const gptr<float> y = as_global_rw(J.y);
#pragma unroll
        for (int n = 0; n < NCOL; ++n) {
            float v = yacc[n];
            if (J.x) {
                const gptr<const float> xr = as_global(J.x) + (size_t)n * J.ldx;
                for (int e = cp[ro]; e < cp[ro + 1]; ++e) v += cv[e] * xr[cc[e]];
            }
            y[(size_t)n * J.ldy + ro] = v;
        }
    }
}

template <int NCOL, int ACT, bool PARTIALS, int CM>
__global__ __launch_bounds__(64 * gemv_waves(NCOL, ACT, PARTIALS, CM))
__attribute__((amdgpu_waves_per_eu(gemv_waves_per_eu(NCOL, ACT, PARTIALS, CM), gemv_waves_per_eu(NCOL, ACT, PARTIALS, CM))))
void k_gemv(GemvJob job0, int total_tasks, const uint32_t *__restrict__ a2) {
    __shared__ GemvSmem<NCOL, ACT> sm;   // static: the table sits at LDS address 0 at compile time
    constexpr int WAVES = gemv_waves(NCOL, ACT, PARTIALS, CM), NT = 64 * WAVES;
    constexpr int NSC = GemvSmem<NCOL, ACT>::kScales / NCOL;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    TaskCtx<NCOL, ACT> c;
    c.hs = lane >> 5; c.j = lane & 31;
    c.bankbytes = (uint32_t)(c.j << 2) * 0x01010101u;
    c.xlane = c.hs * 64;
    build_coset_table<NT>(sm.tab, a2, tid);
    for (int task = blockIdx.x; task < total_tasks; task += gridDim.x) {
        const GemvJob &J = job0;
        c.J = &J;
        const int local = task - J.task0, oct = local / J.nks, ks = local % J.nks;
        c.b0 = ks * J.kchunk;
        c.nbl = min(J.kchunk, J.nb - c.b0);
        c.g = J.g0 + WAVES * oct + w;
        // stage this task's activations and scales
        __syncthreads();
        bool scales_staged = false;
        if constexpr (gemv_quad_loads<ACT, PARTIALS>()) {
            // [n][block][half][64]: word i of a half = activation word (i & 31) of that half
            if (J.q) {
                for (int i = tid; i < NCOL * c.nbl * 128; i += NT) {
                    const int n = i / (c.nbl * 128), wi = i % (c.nbl * 128);
                    const int src = (wi >> 7) * 64 + ((wi >> 6) & 1) * 32 + (wi & 31);
                    sm.xq[n * (kXBytes / 4 / NCOL) + wi] = as_global(reinterpret_cast<const uint32_t *>((const int8_t *)J.q + (size_t)n * J.K + 256 * c.b0))[src];
                }
            } else {   // the chunk's blocks quantized here, one wave per (column, block): no separate prep launch
                for (int pi = w; pi < NCOL * c.nbl; pi += WAVES) {
                    const int n = pi / c.nbl, bl = pi % c.nbl;
                    uint32_t packed;
                    float dd;
                    int qs;
                    quantize_block_q8_128(J.x + (size_t)n * J.ldx + 256 * (c.b0 + bl), J.ic + 256 * (c.b0 + bl), lane, packed, dd, qs);
                    uint32_t *xw = sm.xq + n * (kXBytes / 4 / NCOL) + bl * 128 + (lane >> 5) * 64 + (lane & 31);
                    xw[0] = packed;
                    xw[32] = packed;
                    if ((lane & 31) == 0) sm.xd[n * NSC + 2 * bl + (lane >> 5)] = dd;
                }
                scales_staged = true;
            }
        } else if (ACT == P8X_ACT_Q8_1 && !PARTIALS && !J.q) {
            // block_q8_1 of the chunk's blocks quantized here, one wave per (column, block); the scales staged are
            // the fp16 values a block_q8_1 stores
            for (int pi = w; pi < NCOL * c.nbl; pi += WAVES) {
                const int n = pi / c.nbl, bl = pi % c.nbl;
                uint32_t packed;
                float dd, s;
                quantize_block_q8_1(J.x + (size_t)n * J.ldx + 256 * (c.b0 + bl), J.ic + 256 * (c.b0 + bl), lane, packed, dd, s);
                sm.xq[n * (kXBytes / 4 / NCOL) + bl * 64 + lane] = packed;
                if ((lane & 7) == 0) sm.xd[n * NSC + 8 * bl + (lane >> 3)] = half_to_float(float_to_half(dd));
            }
            scales_staged = true;
        } else {
            for (int i = tid; i < NCOL * c.nbl * 64; i += NT) {
                const int n = i / (c.nbl * 64), wi = i % (c.nbl * 64);
                uint32_t v;
                if constexpr (ACT == P8X_ACT_Q8_128) v = as_global(reinterpret_cast<const uint32_t *>((const int8_t *)J.q + (size_t)n * J.K + 256 * c.b0))[wi];
                else v = as_global(reinterpret_cast<const uint32_t *>((const uint8_t *)J.q + ((size_t)n * (J.K / 32) + 8 * c.b0 + wi / 8) * 36 + 4))[wi % 8];
                sm.xq[n * (kXBytes / 4 / NCOL) + wi] = v;
            }
        }
        if (!scales_staged) {
            constexpr int PER = ACT == P8X_ACT_Q8_128 ? 2 : 8;
            for (int i = tid; i < NCOL * PER * c.nbl; i += NT) {
                const int n = i / (PER * c.nbl), si = i % (PER * c.nbl);
                float v;
                if constexpr (ACT == P8X_ACT_Q8_128) v = as_global(J.d)[(size_t)n * J.nsl + 2 * c.b0 + si];
                else v = half_to_float(*as_global(reinterpret_cast<const uint16_t *>((const uint8_t *)J.q + ((size_t)n * (J.K / 32) + 8 * c.b0 + si) * 36)));
                sm.xd[n * NSC + si] = v;
            }
        }
        __syncthreads();
        if (c.g >= J.gend) continue;
        float yacc[NCOL];
#pragma unroll
        for (int n = 0; n < NCOL; ++n) yacc[n] = 0.f;
        const int bend = c.b0 + c.nbl;
        for (int b = c.b0; b < bend;) {
            const uint32_t mt = as_const(J.M)[(size_t)c.g * J.nb + b];
            // CM: the tile classes this instantiation decodes (chosen from the tensor's class histogram)
            switch (mt >> 29) {
                case 1: if constexpr ((CM >> 1) & 1) { b = gemv_run<NCOL, ACT, PARTIALS, 1, gemv_nbuf(NCOL, 1), CM == (1 << 1)>(c, sm, b, bend, yacc); break; } [[fallthrough]];
                case 2: if constexpr ((CM >> 2) & 1) { b = gemv_run<NCOL, ACT, PARTIALS, 2, gemv_nbuf(NCOL, 2), CM == (1 << 2)>(c, sm, b, bend, yacc); break; } [[fallthrough]];
                case 3: if constexpr ((CM >> 3) & 1) { b = gemv_run<NCOL, ACT, PARTIALS, 3, gemv_nbuf(NCOL, 3), CM == (1 << 3)>(c, sm, b, bend, yacc); break; } [[fallthrough]];
                case 4: if constexpr ((CM >> 4) & 1) { b = gemv_run<NCOL, ACT, PARTIALS, 4, gemv_nbuf(NCOL, 4), CM == (1 << 4)>(c, sm, b, bend, yacc); break; } [[fallthrough]];
                case 5: if constexpr ((CM >> 5) & 1) { b = gemv_run<NCOL, ACT, PARTIALS, 5, gemv_nbuf(NCOL, 5), CM == (1 << 5)>(c, sm, b, bend, yacc); break; } [[fallthrough]];
                case 6: if constexpr ((CM >> 6) & 1) { b = gemv_run<NCOL, ACT, PARTIALS, 6, gemv_nbuf(NCOL, 6), CM == (1 << 6)>(c, sm, b, bend, yacc); break; } [[fallthrough]];
                case 7: if constexpr ((CM >> 7) & 1) { b = gemv_run<NCOL, ACT, PARTIALS, 7, gemv_nbuf(NCOL, 7), CM == (1 << 7)>(c, sm, b, bend, yacc); break; } [[fallthrough]];
                default:
                    if constexpr (PARTIALS) {   // class 0: zero weights
                        const int r = 32 * (c.g - J.g0) + c.j;
                        for (int n = 0; n < NCOL; ++n) {
                            if constexpr (ACT == P8X_ACT_Q8_128) as_global_rw(J.partials)[((size_t)n * J.prows + r) * J.nsl + 2 * b + c.hs] = 0;
                            else for (int u = 0; u < 4; ++u) as_global_rw(J.partials)[((size_t)n * J.prows + r) * (J.K / 32) + 8 * b + 4 * c.hs + u] = 0;
                        }
                    }
                    ++b;
                    break;
            }
        }
        gemv_rows_out<NCOL>(J, c.g, ks, lane, yacc);
    }
}



template <int NCOL, int ACT, bool PARTIALS, int CM>
static int launch_gemv_t(const GemvJob &job0, int tasks, const uint32_t *a2, hipStream_t st) {
    constexpr int NT = 64 * gemv_waves(NCOL, ACT, PARTIALS, CM);
    const int grid = std::min(tasks, gemv_wg_per_cu(NCOL, ACT, PARTIALS, CM) * num_cus());
    hipLaunchKernelGGL((k_gemv<NCOL, ACT, PARTIALS, CM>), dim3(grid), dim3(NT), 0, st, job0, tasks, a2);
    return hip_check(hipGetLastError(), "k_gemv launch");
}

// ------------------------------------------------------------------------------------------------ single GEMV, latency path
// 8-bit-per-128 activations, one linear per launch (the drop-in p8x_mul_mat_vec call; one column, or two of a
// one-class tensor). Such a launch has few tiles, so latency rules: a workgroup takes whole 32-row groups over
// its K-chunk (the whole K, or one of J.nks chunks when the activations do not fit the LDS buffer at once or
// the tensor has too few row groups to fill the CUs), quantizes that part of the activations itself into LDS
// once (the prep's arithmetic, one wave per 256-block and column), its waves split the chunk into contiguous
// block ranges, and the partial rows meet in LDS in a fixed order. K-chunks of a row group meet through the
// fixed-order fix-up of the multi-column kernel (agent-coherent partial rows, an arrival counter, the last
// arrival sums the chunks in order).
constexpr int kRgMaxBlocks = 112;   // activation blocks in LDS (columns x blocks of the K-chunk)
// up to two columns: 16 waves at 128 VGPRs; more (instantiable, measured slower than the task kernel): 8 at 256
__host__ __device__ constexpr int rg_waves(int ncol) { return ncol <= 2 ? 16 : 8; }

template <int NCOL, int WAVES = rg_waves(NCOL)>
struct RgSmem {
    static constexpr int kXW = kRgMaxBlocks * 128 / NCOL, kNSC = 2 * kRgMaxBlocks / NCOL;   // per-column strides
    uint32_t tab[kTabWords];             // LDS address 0
    uint32_t xq[kRgMaxBlocks * 128];     // [column][block][half][64 words] (word i = chunk i of the half)
    float xd[2 * kRgMaxBlocks];          // [column][block][half]
    float red[2][WAVES][NCOL][32];       // per wave: its K range's row sums (two sets, alternating row groups)
};

// quantize the wave's items w, w + 16, ... (item i = column i / nbk, block i % nbk of the chunk; loaded in `in`)
// into the LDS activation layout, G items at a time
template <int G, int NCOL, int WAVES = rg_waves(NCOL), int RQ = kRgMaxBlocks / WAVES>
__device__ __forceinline__ void rg_quantize(int nbk, RgSmem<NCOL> &sm, const BlockLane (&in)[RQ], int w, int lane) {
#pragma unroll
    for (int i0 = 0; i0 < RQ; i0 += G) {
        if (w + i0 * WAVES >= NCOL * nbk) break;
        uint32_t packed[G];
        float dd[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            int qs;
            if (i0 + g < RQ) quantize_loaded_q8_128(in[i0 + g], lane, packed[g], dd[g], qs);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int it = w + (i0 + g) * WAVES;
            if (i0 + g < RQ && it < NCOL * nbk) {
                const int n = it / nbk, bl = it % nbk;   // column, block of the chunk
                uint32_t *xw = sm.xq + n * RgSmem<NCOL>::kXW + bl * 128 + (lane >> 5) * 64 + (lane & 31);
                xw[0] = packed[g];
                xw[32] = packed[g];
                if ((lane & 31) == 0) sm.xd[n * RgSmem<NCOL>::kNSC + 2 * bl + (lane >> 5)] = dd[g];
            }
        }
    }
}

// Linears of one launch of the row-group kernel: 1..kRgMaxJobs GEMVs on the same activations (same x, K and rotation
// sg / c: q/k/v, or gate/up), row groups numbered across the jobs (job i owns gbase[i] .. gbase[i + 1] - 1). With glu,
// jobs 0 (gate) and 1 (up) do not write their rows: each row's two values meet through a per-row arrival counter and
// the second arrival writes out[row] = silu(gate) * up (ggml's swiglu).
// Job 0 travels by value (a single call reads only it); with several jobs each workgroup serves one job: workgroups
// wgbase[i] .. wgbase[i + 1] - 1 take job i, whose tensor metadata comes from its tensor's device copy jt[i] and
// its output from y[i] / ldy[i] (selected once, by comparisons: indexing the arguments at run time would copy them
// to scratch). Unused wgbase entries are INT_MAX.
// Timeline build (make timeline, -DP8X_TIMELINE; never the product library): thread 0 of every row-group workgroup
// records s_memrealtime (100 MHz) at its start, once the kernel-argument fields are in, once its first loads are in
// (it waits for them there, which the product kernel does not), after the table and the quantization, after the
// barrier, after its tiles and at its end, into records [kTimelineRecords][8] = {block << 32 | grid, 7 stamps}.
#ifdef P8X_TIMELINE
#define P8X_STAMP(k) do { if (threadIdx.x == 0) stamp[k] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define P8X_STAMP(k) do {} while (0)
#endif
constexpr int kRgMaxJobs = 4;
struct RgJobs {
    GemvJob j0;                        // job 0: activations, K plan and rotation of every job
    kptr<const GemvJob> jt[kRgMaxJobs];   // tensor metadata of each job (device memory, read-only: scalar loads)
    float *y[kRgMaxJobs];
    unsigned ldy[kRgMaxJobs];
    int wgbase[kRgMaxJobs + 1];
    int njobs;
    int glu;
    float *glu_out;        // [rows] original rows
    unsigned long long *glu_slot;   // [rows] gate / up meeting slots by original row, 0 between calls
#ifdef P8X_TIMELINE
    unsigned long long *tl;
#endif
};

template <typename T>
__device__ __forceinline__ T pick(int jb, T a0, T a1, T a2, T a3) { return jb == 0 ? a0 : jb == 1 ? a1 : jb == 2 ? a2 : a3; }

// The second of a row's two arrivals (gate: job 0, up: job 1) computes silu(gate) * up and writes it, agent-coherent
// (read by a later stage of the step launch): the values meet through the row's slot (pair_meet).
__device__ __forceinline__ void glu_meet(unsigned long long *slot, float *out, int jb, int r, float v, bool active) {
    int oi;
    float other;
    if (active && pair_meet(as_global_rw(slot) + r, jb, v, oi, other)) {
        const float gate = jb == 0 ? v : other, up = jb == 0 ? other : v;
        __hip_atomic_store(&as_global_rw(out)[r], gate / (1.0f + expf(-gate)) * up, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}
__device__ __forceinline__ void glu_meet(const RgJobs &R, int jb, int r, float v, bool active) {
    glu_meet(R.glu_slot, R.glu_out, jb, r, v, active);
}

// SPLIT: J.nks K-chunks (else the whole K, J.nks == 1). NCOL columns of x (stride J.ldx) and y (stride J.ldy);
// NCOL x (blocks of a chunk) <= kRgMaxBlocks. gc row groups at a time: the waves form gc teams of WAVES / gc,
// team t takes row group g0 + t * (workgroups per chunk) over the chunk, so that a workgroup with several row
// groups streams them together instead of one after another. The activations, K plan and rotation come from job 0.
template <int CM, bool SPLIT, int NCOL, bool TEAMS, bool MULTI>
__global__ __launch_bounds__(64 * rg_waves(NCOL)) __attribute__((amdgpu_waves_per_eu(rg_waves(NCOL) / 4, rg_waves(NCOL) / 4)))
void k_gemv_rg(RgJobs jobs, const uint32_t *__restrict__ a2, int gc_) {
#ifdef P8X_TIMELINE
    unsigned long long stamp[7] = {0, 0, 0, 0, 0, 0, 0};
    stamp[0] = __builtin_amdgcn_s_memrealtime();   // before any kernel-argument load
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#endif
    const int gc = TEAMS ? gc_ : 1;   // without teams: one row group at a time, all waves on it
    constexpr int WAVES = rg_waves(NCOL), RQ = kRgMaxBlocks / WAVES;
    __shared__ RgSmem<NCOL> sm;
    // the argument fields the x loads need, requested in the first round of scalar loads with the job ranges
    // (left to the scheduler, some land in a second round behind the job selection's branches)
    if constexpr (MULTI)
        __asm__ volatile("" ::"s"(jobs.j0.x), "s"(jobs.j0.ic), "s"(jobs.j0.ldx), "s"(jobs.j0.kchunk), "s"(jobs.j0.nks), "s"(jobs.j0.nb),
                         "s"(jobs.wgbase[1]), "s"(jobs.wgbase[2]), "s"(jobs.wgbase[3]), "s"(jobs.wgbase[4]), "s"(jobs.jt[0]),
                         "s"(jobs.jt[1]), "s"(jobs.jt[2]), "s"(jobs.jt[3]));
    else
        __asm__ volatile("" ::"s"(jobs.j0.x), "s"(jobs.j0.ic), "s"(jobs.j0.ldx), "s"(jobs.j0.kchunk), "s"(jobs.j0.nks), "s"(jobs.j0.nb));
    // this workgroup's job, its index among the job's workgroups and their count
    int jb = 0, wgl = (int)blockIdx.x, nwg = (int)gridDim.x;
    GemvJob JL = jobs.j0;
    if constexpr (MULTI) {
        const int bi = (int)blockIdx.x;
        jb = (bi >= jobs.wgbase[1]) + (bi >= jobs.wgbase[2]) + (bi >= jobs.wgbase[3]);
        const int wb = pick(jb, jobs.wgbase[0], jobs.wgbase[1], jobs.wgbase[2], jobs.wgbase[3]);
        wgl = bi - wb;
        nwg = pick(jb, jobs.wgbase[1], jobs.wgbase[2], jobs.wgbase[3], jobs.wgbase[4]) - wb;
        JL = *(const GemvJob *)pick(jb, jobs.jt[0], jobs.jt[1], jobs.jt[2], jobs.jt[3]);
        // the x loads take only argument fields (the jobs share K and the rotation ic bit for bit, which the host
        // checks), so they are issued before the job's tensor record arrives
        JL.x = jobs.j0.x; JL.ldx = jobs.j0.ldx; JL.nks = jobs.j0.nks; JL.kchunk = jobs.j0.kchunk;
        JL.ic = jobs.j0.ic; JL.nb = jobs.j0.nb;
        JL.y = pick(jb, jobs.y[0], jobs.y[1], jobs.y[2], jobs.y[3]);
        JL.ldy = pick(jb, jobs.ldy[0], jobs.ldy[1], jobs.ldy[2], jobs.ldy[3]);
    }
    const GemvJob &J = JL;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    TaskCtx<NCOL, P8X_ACT_Q8_128> c;
    c.J = &J;
    c.hs = lane >> 5; c.j = lane & 31;
    c.bankbytes = (uint32_t)(c.j << 2) * 0x01010101u;
    c.xlane = c.hs * 64;
    // workgroup b (of the job's nwg): K-chunk ks = b % nks of row groups b / nks, b / nks + nwg / nks, ...
    const int nks = SPLIT ? J.nks : 1;
    const int ks = SPLIT ? wgl % nks : 0, nbk = SPLIT ? min(J.kchunk, J.nb - ks * J.kchunk) : J.nb;
    c.b0 = ks * J.kchunk; c.nbl = nbk;
    const int wpg = WAVES / gc, team = w / wpg, wk = w % wpg;   // waves beyond gc teams stay idle
    const int per = nbk / wpg, rem = nbk % wpg;
    int b0 = c.b0 + wk * per + min(wk, rem), b1 = b0 + per + (wk < rem ? 1 : 0);   // the wave's K range
    if (team >= gc) b1 = b0;
    // Loads in the order their data is needed (vector loads return in order): the wave's activation blocks, the
    // codebook words of the table; then, for a one-class tensor, the wave's first run of tiles (its first row group
    // over its K range), whose payload stays in flight while the table is written and x is quantized.
    BlockLane in[RQ];
#pragma unroll
    for (int i = 0; i < RQ; ++i) {
        const int it = w + i * WAVES, n = NCOL == 1 ? 0 : it / nbk, bk = c.b0 + (NCOL == 1 ? it : it % nbk);   // column, block
        if (it < NCOL * nbk) in[i].load(J.x + (size_t)n * J.ldx + 256 * bk, J.ic + 256 * bk, lane);
        else in[i] = BlockLane{};   // quantized alongside (results dropped): defined values
    }
#ifdef P8X_TIMELINE
    __asm__ volatile("" :: "s"(J.M), "s"(J.ng));
#endif
    P8X_STAMP(1);
    CosetTableFill<64 * WAVES> fill;
    fill.load(a2, tid);
    constexpr int PC = CM == kCmC3 ? 3 : CM == kCmC6 ? 6 : 0;
    GemvRun<NCOL, P8X_ACT_Q8_128, false, PC ? PC : 3, gemv_nbuf(NCOL, PC ? PC : 3), true> pre;
    const int gstep = nwg / nks;
    const int gfirst = wgl / nks + min(team, gc - 1) * gstep;
    const bool pre_on = PC != 0 && team < gc && gfirst < J.ng && b0 < b1;
    __asm__ volatile("" ::: "memory");
    if constexpr (PC != 0) {
        // on every path (a wave without work requests one in-range tile it never reads), so that no control-flow
        // merge before the table stores makes the compiler wait for these loads there
        c.g = min(gfirst, J.ng - 1);
        const int bb = pre_on ? b0 : min(b0, J.nb - 1);
        pre.begin(c, bb, pre_on ? b1 : bb + 1);
    }
    __asm__ volatile("" ::: "memory");
#ifdef P8X_TIMELINE
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
#endif
    P8X_STAMP(2);
    fill.store(sm.tab, tid);
    // the blocks of a wave are independent: quantized G at a time in straight-line code, so their cross-lane
    // chains overlap (one at a time they cost a full chain latency each)
    if (NCOL * nbk <= WAVES) rg_quantize<1, NCOL>(nbk, sm, in, w, lane);
    else if (NCOL * nbk <= 2 * WAVES) rg_quantize<2, NCOL>(nbk, sm, in, w, lane);
    else rg_quantize<4, NCOL>(nbk, sm, in, w, lane);
    P8X_STAMP(3);
    __syncthreads();
    P8X_STAMP(4);
    int set = 0;
    const GemvJob &JB = J;
    bool first = true;
    for (int g0 = wgl / nks; g0 < J.ng; g0 += gstep * gc, set ^= 1) {
        const int g = g0 + min(team, gc - 1) * gstep;   // this wave's row group
        const bool lead = wk == 0 && team < gc && g < J.ng;   // the team's first wave: epilogue of row group g
        c.g = g;
        // the output row, read before the tile loads so that the epilogue finds it in a register
        int ro = 0;
        if (lead && lane < 32) ro = as_global(JB.prmd)[32 * g + lane];
        float yacc[NCOL];
#pragma unroll
        for (int n = 0; n < NCOL; ++n) yacc[n] = 0.f;
        int bstart = b0;
        if (PC != 0 && first && pre_on) bstart = pre.finish(c, sm, yacc);   // the run begun before the prep
        first = false;
        for (int b = bstart; b < (g < J.ng ? b1 : b0);) {
            if constexpr (PC != 0) {   // one class: no tile word to read
                b = gemv_run<NCOL, P8X_ACT_Q8_128, false, PC, gemv_nbuf(NCOL, PC), true>(c, sm, b, b1, yacc);
                continue;
            }
            const uint32_t mt = as_const(JB.M)[(size_t)g * JB.nb + b];
            switch (mt >> 29) {
                case 1: if constexpr ((CM >> 1) & 1) { b = gemv_run<NCOL, P8X_ACT_Q8_128, false, 1, gemv_nbuf(NCOL, 1), CM == (1 << 1)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                case 2: if constexpr ((CM >> 2) & 1) { b = gemv_run<NCOL, P8X_ACT_Q8_128, false, 2, gemv_nbuf(NCOL, 2), CM == (1 << 2)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                case 3: if constexpr ((CM >> 3) & 1) { b = gemv_run<NCOL, P8X_ACT_Q8_128, false, 3, gemv_nbuf(NCOL, 3), CM == (1 << 3)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                case 4: if constexpr ((CM >> 4) & 1) { b = gemv_run<NCOL, P8X_ACT_Q8_128, false, 4, gemv_nbuf(NCOL, 4), CM == (1 << 4)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                case 5: if constexpr ((CM >> 5) & 1) { b = gemv_run<NCOL, P8X_ACT_Q8_128, false, 5, gemv_nbuf(NCOL, 5), CM == (1 << 5)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                case 6: if constexpr ((CM >> 6) & 1) { b = gemv_run<NCOL, P8X_ACT_Q8_128, false, 6, gemv_nbuf(NCOL, 6), CM == (1 << 6)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                case 7: if constexpr ((CM >> 7) & 1) { b = gemv_run<NCOL, P8X_ACT_Q8_128, false, 7, gemv_nbuf(NCOL, 7), CM == (1 << 7)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                default: ++b; break;   // class 0: zero weights
            }
        }
        P8X_STAMP(5);
#pragma unroll
        for (int n = 0; n < NCOL; ++n) {
            yacc[n] += __shfl_xor(yacc[n], 32);
            if (lane < 32) sm.red[set][w][n][lane] = yacc[n];
        }
        // one barrier per round of row groups: a wave writes this set again two rounds later, after the team
        // leads have passed the next round's barrier, so they have read it by then
        __syncthreads();
        if (lead) {
            float v[NCOL];
#pragma unroll
            for (int n = 0; n < NCOL; ++n) {
                v[n] = 0.f;
                if (lane < 32)
                    for (int i = 0; i < wpg; ++i) v[n] += sm.red[set][w + i][n][lane];
            }
            bool fin = lane < 32;   // lanes that finish their row here
            if constexpr (SPLIT) {
                if (NCOL == 1 && nks == 2) {   // two K-halves: each row's halves meet in its slot (pair_meet)
                    int oi;
                    float other;
                    fin = fin && pair_meet(as_global_rw(JB.wslot) + 32 * g + lane, ks, v[0], oi, other);
                    if (fin) v[0] = ks == 0 ? v[0] + other : other + v[0];   // chunk 0 + chunk 1 either way
                } else {   // K-chunks: the last arrival sums them in chunk order
                    const gptr<float> wpart = as_global_rw(JB.wpart);
                    const gptr<unsigned> wcnt = as_global_rw(JB.wcnt);
                    if (lane < 32)
#pragma unroll
                        for (int n = 0; n < NCOL; ++n)
                            __hip_atomic_store(&wpart[((size_t)ks * NCOL + n) * JB.rows + 32 * g + lane], v[n], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (arrive_after_stores(JB.wcnt + g, lane) != (unsigned)(nks - 1)) continue;
                    if (lane < 32)
#pragma unroll
                        for (int n = 0; n < NCOL; ++n) {
                            v[n] = 0.f;
                            for (int k = 0; k < nks; ++k)
                                v[n] += __hip_atomic_load(&wpart[((size_t)k * NCOL + n) * JB.rows + 32 * g + lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        }
                    if (lane == 0) __hip_atomic_store(&wcnt[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            const int r = ro & 0x7FFF;
            float vo[NCOL];
#pragma unroll
            for (int n = 0; n < NCOL; ++n) {
                vo[n] = v[n];
                if (fin && (ro & 0x8000)) {
                    const gptr<const float> xr = as_global(J.x) + (size_t)n * J.ldx;   // the shared activations
                    for (int e = as_global(JB.cp)[r]; e < as_global(JB.cp)[r + 1]; ++e) vo[n] += as_global(JB.cv)[e] * xr[as_global(JB.cc)[e]];
                }
            }
            if (MULTI && jobs.glu) {
                glu_meet(jobs, jb, r, vo[0], fin);
            } else if (fin) {
#pragma unroll
                for (int n = 0; n < NCOL; ++n) as_global_rw(J.y)[(size_t)n * J.ldy + r] = vo[n];
            }
        }
    }
#ifdef P8X_TIMELINE
    if (tid == 0) {
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        stamp[6] = __builtin_amdgcn_s_memrealtime();
        // the record slot is taken last: a returning atomic on one counter that every workgroup hits would
        // otherwise sit inside the first stamped interval
        const unsigned slot = __hip_atomic_fetch_add((unsigned *)(jobs.tl + kTimelineRecords * 8), 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        if (slot < kTimelineRecords) {
            unsigned long long *o = jobs.tl + (size_t)slot * 8;
            o[0] = ((unsigned long long)blockIdx.x << 32) | gridDim.x;
            for (int k = 0; k < 7; ++k) o[1 + k] = stamp[k];
        }
    }
#endif
}

// ng = the row groups of all jobs; the K plan (nks) is job 0's
template <int CM, int NCOL, bool MULTI>
static int launch_gemv_rg_t(const RgJobs &jobs_, int ng, const uint32_t *a2, hipStream_t st) {
    RgJobs jobs = jobs_;
#ifdef P8X_TIMELINE
    jobs.tl = timeline_buf();
#endif
    // whole row groups per workgroup, evenly: ceil(ng / ceil(ng / CUs)) workgroups per K-chunk, one per CU
    const int per = (ng + num_cus() - 1) / num_cus();
    // a workgroup's row groups are streamed together (teams of waves), up to 4 at a time
    const int gc = std::min(per, 4);
    const int nks = jobs.j0.nks;
    // several jobs: each takes ceil(its row groups / per) workgroups per K-chunk (wgbase, set by the caller)
    const int grid = MULTI ? jobs.wgbase[4] : (ng + per - 1) / per * nks;
    if (nks > 1) hipLaunchKernelGGL((k_gemv_rg<CM, true, NCOL, false, MULTI>), dim3(grid), dim3(64 * rg_waves(NCOL)), 0, st, jobs, a2, 1);
    else if (gc > 1) hipLaunchKernelGGL((k_gemv_rg<CM, false, NCOL, true, MULTI>), dim3(grid), dim3(64 * rg_waves(NCOL)), 0, st, jobs, a2, gc);
    else hipLaunchKernelGGL((k_gemv_rg<CM, false, NCOL, false, MULTI>), dim3(grid), dim3(64 * rg_waves(NCOL)), 0, st, jobs, a2, 1);
    return hip_check(hipGetLastError(), "k_gemv_rg launch");
}

// ------------------------------------------------------------------------------------------------ wave-independent GEMV
// 1..8 columns of 8-bit-per-128 activations, grouped launches (the decode stream). Each wave is its own worker:
// it takes a unit (job, row group, K-chunk) from a device counter, streams that row group's tiles, and leaves
// the sorted-row partials for the finishing launch. Activations never pass through LDS: with the payload in chunk
// order every lane of a half multiplies chunk k by the same activation word, which the v_dot4 instruction takes
// straight from a DPP broadcast (row_newbcast) of two registers loaded with the tile; LDS serves the codeword
// lookups alone. Nothing waits on another wave after the table is built, so a slow wave delays only its own unit
// and the launch drains with at most one unit per wave. Units are numbered in job order; the job list is ordered
// by decreasing unit length, so the long units start first.
// One column of class 3 fits 64 VGPRs: 16-wave workgroups, 8 waves per SIMD; one column of classes 6 or 2-4
// 8-wave workgroups at 4 (128 VGPRs), every class at 2. Two to four columns of one class: 16-wave workgroups
// (one per CU) at 4 waves per SIMD; five to eight columns or mixed classes (more than 128 VGPRs): 8-wave
// workgroups at 2.
__host__ __device__ constexpr int wave_waves(int cm, int ncol = 1) {
    return ncol == 1 ? (cm == kCmC3 ? 16 : 8) : ncol <= 4 && (cm == kCmC3 || cm == kCmC6) ? 16 : 8;
}
__host__ __device__ constexpr int wave_per_eu(int cm, int ncol = 1) {
    return ncol == 1 ? (cm == kCmC3 ? 8 : cm == kCmAll ? 2 : 4) : ncol <= 4 && (cm == kCmC3 || cm == kCmC6) ? 4 : 2;
}
__host__ __device__ constexpr int wave_wg_per_cu(int cm, int ncol = 1) { return 4 * wave_per_eu(cm, ncol) / wave_waves(cm, ncol); }
// prefetch depth of the class-3 runs (register buffers hold NCOL activation words and scales each)
__host__ __device__ constexpr int wave_nbuf_c3(int ncol) { return ncol == 1 ? GEMV_NBUF_C3 : 2; }

// bytes per 256-column block and column of the grouped launch's activations (k_act_q8_128_batch)
constexpr uint32_t kBcastBlockBytes = 512;

struct WaveSmem {
    uint32_t tab[kTabWords];   // LDS address 0
};

// A tile's payload with its activation words: per column, the lane's broadcast-layout entry {word i, word 16 + i,
// d, 0} of its half (lane 16 r + i, half hs = r >> 1: the rows of 16 lanes the DPP broadcast works in). All four
// words are kept: the compiler (ROCm 7.2) shrinks a 16-byte buffer load of which only three words are used to an
// 8-byte load and reads the wrong word for the third.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
template <int C, int NCOL>
struct WaveSlice {
    QuadSlice<C> p;
    u32x4_t x[NCOL];
};

// acc += dot4(x broadcast from lane B of each 16-lane row, w): v_dot4c_i32_i8 with a DPP row_newbcast source
// (gfx90a and later), as asm: the compiler does not fold a DPP move into this instruction. Wait states, measured on
// gfx950 against a CPU sum of the same sequences: these dots chain through their accumulators back to back
// exactly, but an ordinary VALU instruction that reads a dot's result needs two wait states after it, and a DPP
// read needs two after a VALU write of its source. Every block therefore starts and ends with s_nop 1 (the asm
// cannot see which instructions the compiler places around it).
#define P8X_DL(A, X, W, B) "v_dot4c_i32_i8_dpp %" #A ", %" #X ", %" #W " row_newbcast:" #B " row_mask:0xf bank_mask:0xf\n\t"
#define P8X_R1(W, B) P8X_DL(0, 1, W, B)
#define P8X_G1(B0, B1, B2, B3) "s_nop 1\n\t" P8X_R1(2, B0) P8X_R1(3, B1) P8X_R1(4, B2) P8X_R1(5, B3) "s_nop 1"
#define P8X_R2(W, B) P8X_DL(0, 2, W, B) P8X_DL(1, 3, W, B)
#define P8X_G2(B0, B1, B2, B3) "s_nop 1\n\t" P8X_R2(4, B0) P8X_R2(5, B1) P8X_R2(6, B2) P8X_R2(7, B3) "s_nop 1"
#define P8X_R3(W, B) P8X_DL(0, 3, W, B) P8X_DL(1, 4, W, B) P8X_DL(2, 5, W, B)
#define P8X_G3(B0, B1, B2, B3) "s_nop 1\n\t" P8X_R3(6, B0) P8X_R3(7, B1) P8X_R3(8, B2) P8X_R3(9, B3) "s_nop 1"
#define P8X_R4(W, B) P8X_DL(0, 4, W, B) P8X_DL(1, 5, W, B) P8X_DL(2, 6, W, B) P8X_DL(3, 7, W, B)
#define P8X_G4(B0, B1, B2, B3) "s_nop 1\n\t" P8X_R4(8, B0) P8X_R4(9, B1) P8X_R4(10, B2) P8X_R4(11, B3) "s_nop 1"
#define P8X_R5(W, B) P8X_DL(0, 5, W, B) P8X_DL(1, 6, W, B) P8X_DL(2, 7, W, B) P8X_DL(3, 8, W, B) P8X_DL(4, 9, W, B)
#define P8X_G5(B0, B1, B2, B3) "s_nop 1\n\t" P8X_R5(10, B0) P8X_R5(11, B1) P8X_R5(12, B2) P8X_R5(13, B3) "s_nop 1"
#define P8X_R6(W, B) P8X_DL(0, 6, W, B) P8X_DL(1, 7, W, B) P8X_DL(2, 8, W, B) P8X_DL(3, 9, W, B) P8X_DL(4, 10, W, B) P8X_DL(5, 11, W, B)
#define P8X_G6(B0, B1, B2, B3) "s_nop 1\n\t" P8X_R6(12, B0) P8X_R6(13, B1) P8X_R6(14, B2) P8X_R6(15, B3) "s_nop 1"
#define P8X_R7(W, B) P8X_DL(0, 7, W, B) P8X_DL(1, 8, W, B) P8X_DL(2, 9, W, B) P8X_DL(3, 10, W, B) P8X_DL(4, 11, W, B) P8X_DL(5, 12, W, B) P8X_DL(6, 13, W, B)
#define P8X_G7(B0, B1, B2, B3) "s_nop 1\n\t" P8X_R7(14, B0) P8X_R7(15, B1) P8X_R7(16, B2) P8X_R7(17, B3) "s_nop 1"
#define P8X_R8(W, B) P8X_DL(0, 8, W, B) P8X_DL(1, 9, W, B) P8X_DL(2, 10, W, B) P8X_DL(3, 11, W, B) P8X_DL(4, 12, W, B) P8X_DL(5, 13, W, B) P8X_DL(6, 14, W, B) P8X_DL(7, 15, W, B)
#define P8X_G8(B0, B1, B2, B3) "s_nop 1\n\t" P8X_R8(16, B0) P8X_R8(17, B1) P8X_R8(18, B2) P8X_R8(19, B3) "s_nop 1"

// one group of four chunks (Q & 3 of the register pair) for every column: acc[n] += sum_e dot4(x[n] from lane
// 4 Q + e, w[e]), the chunks in order, the columns interleaved
template <int Q, int NCOL>
__device__ __forceinline__ void dot4_bcast(int (&a)[NCOL], const uint32_t (&x)[NCOL], const uint32_t (&w)[4]) {
    static_assert(Q >= 0 && Q < 4 && NCOL >= 1 && NCOL <= 8, "four groups per register pair, 1..8 columns");
#define P8X_PASS(...) __VA_ARGS__
#define P8X_GQ(G, OUTS, INS) \
    if constexpr (Q == 0) __asm__(G(0, 1, 2, 3) : OUTS : INS); \
    else if constexpr (Q == 1) __asm__(G(4, 5, 6, 7) : OUTS : INS); \
    else if constexpr (Q == 2) __asm__(G(8, 9, 10, 11) : OUTS : INS); \
    else __asm__(G(12, 13, 14, 15) : OUTS : INS);
#define P8X_W "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3])
    if constexpr (NCOL == 1) {
        P8X_GQ(P8X_G1, P8X_PASS("+v"(a[0])), P8X_PASS("v"(x[0]), P8X_W))
    } else if constexpr (NCOL == 2) {
        P8X_GQ(P8X_G2, P8X_PASS("+v"(a[0]), "+v"(a[1])), P8X_PASS("v"(x[0]), "v"(x[1]), P8X_W))
    } else if constexpr (NCOL == 3) {
        P8X_GQ(P8X_G3, P8X_PASS("+v"(a[0]), "+v"(a[1]), "+v"(a[2])), P8X_PASS("v"(x[0]), "v"(x[1]), "v"(x[2]), P8X_W))
    } else if constexpr (NCOL == 4) {
        P8X_GQ(P8X_G4, P8X_PASS("+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3])), P8X_PASS("v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), P8X_W))
    } else if constexpr (NCOL == 5) {
        P8X_GQ(P8X_G5, P8X_PASS("+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4])), P8X_PASS("v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), P8X_W))
    } else if constexpr (NCOL == 6) {
        P8X_GQ(P8X_G6, P8X_PASS("+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5])), P8X_PASS("v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), P8X_W))
    } else if constexpr (NCOL == 7) {
        P8X_GQ(P8X_G7, P8X_PASS("+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6])), P8X_PASS("v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), P8X_W))
    } else if constexpr (NCOL == 8) {
        P8X_GQ(P8X_G8, P8X_PASS("+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7])), P8X_PASS("v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]), P8X_W))
    }
#undef P8X_W
#undef P8X_GQ
#undef P8X_PASS
}
#undef P8X_DL
#undef P8X_R1
#undef P8X_G1
#undef P8X_R2
#undef P8X_G2
#undef P8X_R3
#undef P8X_G3
#undef P8X_R4
#undef P8X_G4
#undef P8X_R5
#undef P8X_G5
#undef P8X_R6
#undef P8X_G6
#undef P8X_R7
#undef P8X_G7
#undef P8X_R8
#undef P8X_G8

// chunks 4Q .. 4Q + 3 of one tile: the codewords of every stage, then their products with each column's broadcast
// activation words
template <int C, int NCOL, int Q>
__device__ __forceinline__ void wave_group(const uint32_t *tab, const QuadSlice<C> &p, uint32_t H, uint32_t bankbytes,
                                           const uint32_t (&xa)[NCOL], const uint32_t (&xb)[NCOL], int (&acc)[nstage_of(C)][NCOL]) {
    constexpr int NST = nstage_of(C);
    const uint32_t hq = coset_bytes(H, bankbytes, Q);
    uint32_t w[NST][4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        w[0][e] = lds_word(tab, p.template addr<0>(4 * Q + e, hq));
        if constexpr (NST > 1) w[1][e] = lds_word(tab, p.template addr<1>(4 * Q + e, hq));
        if constexpr (NST > 2) w[2][e] = lds_word(tab, p.template addr<2>(4 * Q + e, hq));
    }
#pragma unroll
    for (int s = 0; s < NST; ++s) dot4_bcast<Q & 3, NCOL>(acc[s], Q < 4 ? xa : xb, w[s]);
    __asm__ volatile("" ::: "memory");   // one group of 4 chunks at a time: bounds the live registers
}

template <int C, int NCOL, int... Q>
__device__ __forceinline__ void wave_groups(const uint32_t *tab, const QuadSlice<C> &p, uint32_t H, uint32_t bankbytes,
                                            const uint32_t (&xa)[NCOL], const uint32_t (&xb)[NCOL], int (&acc)[nstage_of(C)][NCOL],
                                            std::integer_sequence<int, Q...>) {
    (wave_group<C, NCOL, Q>(tab, p, H, bankbytes, xa, xb, acc), ...);
}

// One tile of a wave: integer sums per column (isum = sum_s dot_s << SH_s, CPU.patch:646-662), then
// y += isum * d * S.
template <int C, int NCOL>
__device__ __forceinline__ void wave_tile(const uint32_t *tab, int lane, const WaveSlice<C, NCOL> &r_, float (&yacc)[NCOL]) {
    constexpr int NST = nstage_of(C), SH1 = sh1_of(C), SH2 = sh2_of(C);
    const int j = lane & 31;
    WaveSlice<C, NCOL> r = r_;
    pin(r.p.w);
    pin(r.p.s);
    uint32_t xa[NCOL], xb[NCOL];
    float xd[NCOL];
#pragma unroll
    for (int n = 0; n < NCOL; ++n) {
        uint32_t v[4] = {r.x[n][0], r.x[n][1], r.x[n][2], r.x[n][3]};
        pin(v);
        xa[n] = v[0];
        xb[n] = v[1];
        xd[n] = __builtin_bit_cast(float, v[2]);
    }
    const uint32_t H = r.p.coset_bits();
    int acc[NST][NCOL];
#pragma unroll
    for (int s = 0; s < NST; ++s)
#pragma unroll
        for (int n = 0; n < NCOL; ++n) acc[s][n] = 0;
    wave_groups<C, NCOL>(tab, r.p, H, (uint32_t)(j << 2) * 0x01010101u, xa, xb, acc, std::make_integer_sequence<int, 8>{});
    const float sc = half_to_float(r.p.s);
#pragma unroll
    for (int n = 0; n < NCOL; ++n) {
        int isum = acc[0][n] * (1 << SH1);
        if constexpr (NST > 1) isum += acc[1][n] * (1 << SH2);
        if constexpr (NST > 2) isum += acc[2][n];
        yacc[n] += ((float)isum * xd[n]) * sc;
    }
}

// a run of consecutive tiles of class C in row group g, NBUF tiles in flight (the gemv_run scheme)
template <int C, int NBUF, bool ONLY_C, int NCOL>
__device__ __forceinline__ int wave_run(const GemvJob &J, const uint32_t *tab, int g, int b, int bend, int lane, float (&yacc)[NCOL]) {
    const int hs = lane >> 5, j = lane & 31;
    const kptr<const uint32_t> mrow = as_const(J.M) + (size_t)g * J.nb;
    int e = bend;
    if constexpr (!ONLY_C) {
        e = b + 1;
        while (e < bend && (mrow[e] >> 29) == (uint32_t)C) ++e;
    }
    // activations [NCOL][nb] blocks in the broadcast layout: lane 16 r + i loads entry (hs = r >> 1, i) =
    // {word i, word 16 + i, d, 0} of its column's block
    const uint32_t sbytes = (uint32_t)J.nb * J.rows * 2u, qbytes = (uint32_t)(NCOL * J.nb) * kBcastBlockBytes;
    const uint32_t vo = QuadSlice<C>::quad_offset(hs, j), vp = QuadSlice<C>::pair_offset(hs, j);
    const uint32_t vs = 2u * (uint32_t)j, vq = 256u * (uint32_t)hs + 16u * (uint32_t)(lane & 15);
    uint32_t wn = mrow[b];
    auto issue = [&](WaveSlice<C, NCOL> &r, int ta) {
        const bool ok = ta < e;
        const int tc = ok ? ta : b;
        const uint32_t toff = (wn & 0x1FFFFFFFu) * 4u;
        const uint32_t soff = ((uint32_t)g * (uint32_t)J.nb + (uint32_t)tc) * 64u;   // scales [g][b][32]
        // past the run's end the resources have no records: the loads read zeros without memory traffic.
        // The wave issues its loads at raised priority, so the arbiter lets it put the next tile in flight
        // ahead of other waves' decode work (about 1% on the class-3 stream).
        __builtin_amdgcn_s_setprio(2);
        r.p.load(buffer_rsrc(J.D, ok ? J.dbytes : 0u), toff, vo, vp, buffer_rsrc(J.S, ok ? sbytes : 0u), soff, vs);
        const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(J.q, ok ? qbytes : 0u);
#pragma unroll
        for (int n = 0; n < NCOL; ++n) {
            r.x[n] = __builtin_amdgcn_raw_buffer_load_b128(rq, vq, ((uint32_t)n * (uint32_t)J.nb + (uint32_t)tc) * kBcastBlockBytes, 0);
        }
        __builtin_amdgcn_s_setprio(0);
        wn = mrow[min(ta + 1, e - 1)];
    };
    auto tile = [&](const WaveSlice<C, NCOL> &r) { wave_tile<C, NCOL>(tab, lane, r, yacc); };
    WaveSlice<C, NCOL> buf[NBUF];
#pragma unroll
    for (int i = 0; i < NBUF - 1; ++i) issue(buf[i], b + i);
    int base = b;
    for (; base + NBUF <= e; base += NBUF) {
#pragma unroll
        for (int i = 0; i < NBUF; ++i) {
            issue(buf[(i + NBUF - 1) % NBUF], base + i + NBUF - 1);
            tile(buf[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < NBUF - 1; ++i)
        if (base + i < e) tile(buf[i]);
    return e;
}

// Unit scheduling. Device-scope atomics on one address serialize far from the CUs, so the units are dealt to
// np = min(kWaveParts, workgroups) partitions (unit u to partition u % np), each with its own counter pair
// kWaveCtrStride words apart; workgroup b serves partition b % np. A wave's first unit in its partition is its rank there (no
// atomic); after that it takes the next from the partition's counter.
constexpr int kWaveParts = 32, kWaveCtrStride = 64;
constexpr size_t kWaveCtrBytes = sizeof(unsigned) * kWaveParts * kWaveCtrStride;

__device__ __forceinline__ unsigned wave_atomic_add(unsigned *p, int lane) {
    unsigned v = 0;
    if (lane == 0) v = __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __builtin_amdgcn_readfirstlane(v);
}

// A wave unit's rows: the half-slices meet through one cross-lane add, and lanes 0..31 store the row group's 32
// sorted-row partials of K-chunk ks to wpart [nks][NCOL][rows] (one 128-byte line per column, no loads, no
// atomics, so nothing waits on the loads in flight). The batch's finishing launch sums the K-chunks in order,
// applies the clamp delta and writes original rows.
template <int NCOL>
__device__ __forceinline__ void wave_rows_store(const GemvJob &J, int g, int ks, int lane, float (&yacc)[NCOL]) {
#pragma unroll
    for (int n = 0; n < NCOL; ++n) {
        const float v = yacc[n] + __shfl_xor(yacc[n], 32);
        if (lane < 32) as_global_rw(J.wpart)[((size_t)ks * NCOL + n) * J.rows + 32 * g + lane] = v;
    }
}

// ctr[part * kWaveCtrStride + 0]: units the partition has handed out beyond the first round; + 1: waves that have
// left. Both start at 0 and the partition's last wave to leave puts them back, so launches on one stream reuse
// them (concurrent launches that share the counters race).
template <int CM, int NCOL>
__global__ __launch_bounds__(64 * wave_waves(CM, NCOL)) __attribute__((amdgpu_waves_per_eu(wave_per_eu(CM, NCOL), wave_per_eu(CM, NCOL))))
void k_gemv_wave(const GemvJob *__restrict__ jobs, const uint32_t *__restrict__ ujob, int total_units, unsigned *ctr,
                 const uint32_t *__restrict__ a2) {
    constexpr int WAVES = wave_waves(CM, NCOL);
    __shared__ WaveSmem sm;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    build_coset_table<64 * WAVES>(sm.tab, a2, tid);
    __syncthreads();
    const int np = min(kWaveParts, (int)gridDim.x), part = blockIdx.x % np;
    const int nwp = (((int)gridDim.x - 1 - part) / np + 1) * WAVES;   // waves serving this partition
    unsigned *pc = ctr + part * kWaveCtrStride;
    int k = (blockIdx.x / np) * WAVES + w;
    // each later take waits for its atomic, which also drains the previous unit's stores: the tile loops start
    // with loads only in flight, so their wait counts stay exact
    for (int u = part + np * k; u < total_units; u = part + np * k) {
        const int jc = (int)as_const(ujob)[u];
        const GemvJob &J = jobs[jc];
        const int local = u - J.task0, g = local / J.nks, ks = local % J.nks;
        const int b0 = ks * J.kchunk, bend = min(b0 + J.kchunk, J.nb);
        float yacc[NCOL];
#pragma unroll
        for (int n = 0; n < NCOL; ++n) yacc[n] = 0.f;
        for (int b = b0; b < bend;) {
            const uint32_t mt = as_const(J.M)[(size_t)g * J.nb + b];
            switch (mt >> 29) {
                case 1: if constexpr ((CM >> 1) & 1) { b = wave_run<1, 2, CM == (1 << 1), NCOL>(J, sm.tab, g, b, bend, lane, yacc); break; } [[fallthrough]];
                case 2: if constexpr ((CM >> 2) & 1) { b = wave_run<2, 2, CM == (1 << 2), NCOL>(J, sm.tab, g, b, bend, lane, yacc); break; } [[fallthrough]];
                case 3: if constexpr ((CM >> 3) & 1) { b = wave_run<3, wave_nbuf_c3(NCOL), CM == (1 << 3), NCOL>(J, sm.tab, g, b, bend, lane, yacc); break; } [[fallthrough]];
                case 4: if constexpr ((CM >> 4) & 1) { b = wave_run<4, 2, CM == (1 << 4), NCOL>(J, sm.tab, g, b, bend, lane, yacc); break; } [[fallthrough]];
                case 5: if constexpr ((CM >> 5) & 1) { b = wave_run<5, 2, CM == (1 << 5), NCOL>(J, sm.tab, g, b, bend, lane, yacc); break; } [[fallthrough]];
                case 6: if constexpr ((CM >> 6) & 1) { b = wave_run<6, 2, CM == (1 << 6), NCOL>(J, sm.tab, g, b, bend, lane, yacc); break; } [[fallthrough]];
                case 7: if constexpr ((CM >> 7) & 1) { b = wave_run<7, 2, CM == (1 << 7), NCOL>(J, sm.tab, g, b, bend, lane, yacc); break; } [[fallthrough]];
                default: ++b; break;   // class 0: zero weights
            }
        }
        wave_rows_store<NCOL>(J, g, ks, lane, yacc);
        k = nwp + (int)wave_atomic_add(pc, lane);
    }
    const unsigned left = wave_atomic_add(pc + 1, lane);
    if (lane == 0 && left == (unsigned)nwp - 1) {
        __hip_atomic_store(pc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pc + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// e0 / e1 (optional): HIP events the runtime records at the kernel's own start and end (hipExtLaunchKernel)
template <int CM, int NCOL>
static int launch_gemv_wave_t(const GemvJob *jobs, const uint32_t *ujob, int units, unsigned *ctr, const uint32_t *a2, hipStream_t st,
                              hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr) {
    const int grid = wave_wg_per_cu(CM, NCOL) * num_cus();
    if (e0 || e1)
        hipExtLaunchKernelGGL((k_gemv_wave<CM, NCOL>), dim3(grid), dim3(64 * wave_waves(CM, NCOL)), 0, st, e0, e1, 0, jobs, ujob, units, ctr, a2);
    else
        hipLaunchKernelGGL((k_gemv_wave<CM, NCOL>), dim3(grid), dim3(64 * wave_waves(CM, NCOL)), 0, st, jobs, ujob, units, ctr, a2);
    return hip_check(hipGetLastError(), "k_gemv_wave launch");
}

// ------------------------------------------------------------------------------------------------ matrix-core GEMV
// 2..8 columns of class-3 tiles in grouped launches. A tile's integer products form a small matrix product,
// (32 rows x 128 K) x (128 K x columns) per 128-column half, which v_mfma_i32_32x32x32_i8 computes with the
// looked-up codewords as the B operand (n = row = lane & 31) and the activations as A (m = column; rows of A past
// the batch are zeros): per tile 8 MFMAs replace 32 v_dot4 per column and lane. Lane (row j, half hs) looks up its
// 32 codewords as the broadcast kernel does; one v_permlane32_swap per pair (chunk k, chunk k + 16) turns the
// two halves' words into per-half operands (words 0..15: half 0, lanes 0..31 chunks 0..15 and lanes 32..63 chunks
// 16..31; words 16..31 the same of half 1), so that MFMA i of half h reads words 16 h + 4 i .. + 3: K bytes
// 16 i .. + 15 of the half in lanes 0..31 and 64 + 16 i .. in lanes 32..63. The activations come in a layout to
// match (k_act_q8_128_mx_batch, k_act_x16_batch<true>): per 256-block and column a 256-byte record (half 0, then half
// 1), the halves' scales [block][column][2] after the records. A wave loads its next tile's records and scales with
// one to three 16-byte loads per lane and, when it reaches that tile, copies them into its own LDS slot, from which
// lane (column m, group g) reads its A operands (64 bytes at 64 g of each half) and lane (row j, group g) the scales
// of columns 4 g .. 4 g + 3; so only 12 registers per tile in flight hold activations. The output lane (row j, group
// g) holds columns 4 g .. 4 g + 3, accumulated per half as the broadcast kernel does (y_h += ((float)isum d) S tile
// by tile, then half 0 + half 1): the same bits.
constexpr uint32_t kMxRecBytes = 256;   // activation record per 256-block and column
__host__ __device__ constexpr int mx_waves() { return 16; }
__host__ __device__ constexpr int mx_per_eu() { return 4; }
__host__ __device__ constexpr int mx_wg_per_cu() { return 4 * mx_per_eu() / mx_waves(); }
// activation bytes of a job: the records, then the scales
__host__ __device__ constexpr size_t mx_act_bytes(int ncols, int nb) { return (size_t)ncols * nb * (kMxRecBytes + 8); }
// a wave's LDS slot: the tile's records, then its scales (8 columns' worth)
template <int NCOL>
struct MxSlot {
    static constexpr int kRecWords = NCOL * kMxRecBytes / 4;
    uint32_t w[kRecWords + 16];   // records | scales [8][2]
    static constexpr int kScaleWord = kRecWords;
};
template <int NCOL>
struct MxSmem {
    uint32_t tab[kTabWords];   // LDS address 0
    MxSlot<NCOL> slot[mx_waves()];
};

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));

template <int NCOL>
struct MxSlice {
    static constexpr int NREC = (16 * NCOL + 63) / 64;   // 16-byte record pieces per lane
    QuadSlice<3> p;
    u32x4_t r[NREC];   // record piece l (and l + 64) of the tile's NCOL records
    u32x4_t d;         // scale piece l (lanes l < NCOL / 2, rounded up)
};

template <int NCOL>
__device__ __forceinline__ void mx_tile(const uint32_t *tab, MxSlot<NCOL> &slot, int lane, const MxSlice<NCOL> &r_, float (&ya)[2][4]) {
    constexpr int SH1 = sh1_of(3), NREC = MxSlice<NCOL>::NREC;
    static_assert(nstage_of(3) == 1, "one codeword per chunk");
    const int j = lane & 31, g = lane >> 5;
    MxSlice<NCOL> r = r_;
    pin(r.p.w);
    pin(r.p.s);
    // the tile's activations into the wave's slot (program order keeps the wave's own LDS accesses in order)
    u32x4_t *sv = reinterpret_cast<u32x4_t *>(slot.w);
#pragma unroll
    for (int q = 0; q < NREC; ++q)
        if (lane + 64 * q < 16 * NCOL) sv[lane + 64 * q] = r.r[q];
    if (lane < (NCOL + 1) / 2) sv[MxSlot<NCOL>::kScaleWord / 4 + lane] = r.d;
    const uint32_t H = r.p.coset_bits(), bankbytes = (uint32_t)(j << 2) * 0x01010101u;
    uint32_t w[32];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const uint32_t hq = coset_bytes(H, bankbytes, q);
#pragma unroll
        for (int e = 0; e < 4; ++e) w[4 * q + e] = lds_word(tab, r.p.template addr<0>(4 * q + e, hq));
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const auto sw = __builtin_amdgcn_permlane32_swap(w[k], w[k + 16], false, false);
        w[k] = sw[0];
        w[k + 16] = sw[1];
    }
    const int m = j;   // A row (column of the batch) of this lane
    const u32x4_t *arow = sv + (m * (int)kMxRecBytes + 64 * g) / 16;
    // lanes of rows past the batch keep zero operands and read nothing (their loads are masked off)
    u32x4_t xa[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xa[i] = u32x4_t{0u, 0u, 0u, 0u};
    if (m < NCOL) {
#pragma unroll
        for (int i = 0; i < 8; ++i) xa[i] = arow[8 * (i >> 2) + (i & 3)];   // half i / 4, 16-byte piece i % 4
    }
    const u32x4_t dv0 = sv[MxSlot<NCOL>::kScaleWord / 4 + 2 * g], dv1 = sv[MxSlot<NCOL>::kScaleWord / 4 + 2 * g + 1];
    const float sc = half_to_float(r.p.s);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        i32x16_t acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4_t xv = xa[4 * h + i];
            const i32x4_t a = {(int)xv[0], (int)xv[1], (int)xv[2], (int)xv[3]};
            const i32x4_t bw = {(int)w[16 * h + 4 * i], (int)w[16 * h + 4 * i + 1], (int)w[16 * h + 4 * i + 2], (int)w[16 * h + 4 * i + 3]};
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bw, acc, 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const u32x4_t dd = c < 2 ? dv0 : dv1;
            const float dsc = __uint_as_float(dd[2 * (c & 1) + h]);
            ya[h][c] += ((float)(acc[c] * (1 << SH1)) * dsc) * sc;
        }
    }
}

// a run of consecutive class-3 tiles of row group g, MX_NBUF - 1 ahead of the one multiplied (the wave_run scheme)
#ifndef MX_NBUF
#define MX_NBUF 2
#endif
template <int NCOL>
__device__ __forceinline__ int mx_run(const GemvJob &J, const uint32_t *tab, MxSlot<NCOL> &slot, int g, int b, int bend, int lane,
                                      float (&ya)[2][4]) {
    constexpr int NREC = MxSlice<NCOL>::NREC;
    const int hs = lane >> 5, j = lane & 31;
    const kptr<const uint32_t> mrow = as_const(J.M) + (size_t)g * J.nb;
    const int e = bend;
    const uint32_t sbytes = (uint32_t)J.nb * J.rows * 2u;
    const uint32_t qbytes = (uint32_t)(NCOL * J.nb) * kMxRecBytes, dbytes = (uint32_t)(NCOL * J.nb) * 8u;
    const uint32_t vo = QuadSlice<3>::quad_offset(hs, j), vp = QuadSlice<3>::pair_offset(hs, j);
    const uint32_t vs = 2u * (uint32_t)j;
    const uint8_t *dbase = reinterpret_cast<const uint8_t *>(J.q) + qbytes;
    uint32_t wn = mrow[b];
    auto issue = [&](MxSlice<NCOL> &r, int ta) {
        const bool ok = ta < e;
        const int tc = ok ? ta : b;
        const uint32_t toff = (wn & 0x1FFFFFFFu) * 4u;
        const uint32_t soff = ((uint32_t)g * (uint32_t)J.nb + (uint32_t)tc) * 64u;
        __builtin_amdgcn_s_setprio(2);
        r.p.load(buffer_rsrc(J.D, ok ? J.dbytes : 0u), toff, vo, vp, buffer_rsrc(J.S, ok ? sbytes : 0u), soff, vs);
        // the tile's NCOL records (16 NCOL pieces) and scales; pieces past them read zeros without traffic
        const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(J.q, ok ? qbytes : 0u), rdd = buffer_rsrc(dbase, ok ? dbytes : 0u);
        const uint32_t rec0 = (uint32_t)(tc * NCOL) * kMxRecBytes;
#pragma unroll
        for (int q = 0; q < NREC; ++q) {
            const int piece = lane + 64 * q;
            r.r[q] = __builtin_amdgcn_raw_buffer_load_b128(rq, piece < 16 * NCOL ? rec0 + 16u * (uint32_t)piece : 0x7FFFFF00u, 0, 0);
        }
        r.d = __builtin_amdgcn_raw_buffer_load_b128(rdd, lane < (NCOL + 1) / 2 ? (uint32_t)(tc * NCOL) * 8u + 16u * (uint32_t)lane : 0x7FFFFF00u, 0, 0);
        __builtin_amdgcn_s_setprio(0);
        wn = mrow[min(ta + 1, e - 1)];
    };
    MxSlice<NCOL> buf[MX_NBUF];
#pragma unroll
    for (int i = 0; i < MX_NBUF - 1; ++i) issue(buf[i], b + i);
    int base = b;
    for (; base + MX_NBUF <= e; base += MX_NBUF) {
#pragma unroll
        for (int i = 0; i < MX_NBUF; ++i) {
            issue(buf[(i + MX_NBUF - 1) % MX_NBUF], base + i + MX_NBUF - 1);
            mx_tile<NCOL>(tab, slot, lane, buf[i], ya);
        }
    }
#pragma unroll
    for (int i = 0; i < MX_NBUF - 1; ++i)
        if (base + i < e) mx_tile<NCOL>(tab, slot, lane, buf[i], ya);
    return e;
}

// Grouped launch of class-3 jobs with 2..8 columns (the unit scheduling of k_gemv_wave); lane (row j, group g)
// stores columns 4 g .. 4 g + 3 of its row's K-chunk partial
template <int NCOL>
__global__ __launch_bounds__(64 * mx_waves()) __attribute__((amdgpu_waves_per_eu(mx_per_eu(), mx_per_eu())))
void k_gemv_wave_mx(const GemvJob *__restrict__ jobs, const uint32_t *__restrict__ ujob, int total_units, unsigned *ctr,
                    const uint32_t *__restrict__ a2) {
    static_assert(NCOL >= 1 && NCOL <= 8, "1..8 columns");
    constexpr int WAVES = mx_waves();
    __shared__ MxSmem<NCOL> sm;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    build_coset_table<64 * WAVES>(sm.tab, a2, tid);
    MxSlot<NCOL> &slot = sm.slot[w];
    __syncthreads();
    const int np = min(kWaveParts, (int)gridDim.x), part = blockIdx.x % np;
    const int nwp = (((int)gridDim.x - 1 - part) / np + 1) * WAVES;
    unsigned *pc = ctr + part * kWaveCtrStride;
    int k = (blockIdx.x / np) * WAVES + w;
    const int j = lane & 31, cg = lane >> 5;
    for (int u = part + np * k; u < total_units; u = part + np * k) {
        const int jc = (int)as_const(ujob)[u];
        const GemvJob &J = jobs[jc];
        const int local = u - J.task0, g = local / J.nks, ks = local % J.nks;
        const int b0 = ks * J.kchunk, bend = min(b0 + J.kchunk, J.nb);
        float ya[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int c = 0; c < 4; ++c) ya[h][c] = 0.f;
        if (b0 < bend) mx_run<NCOL>(J, sm.tab, slot, g, b0, bend, lane, ya);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int col = 4 * cg + c;
            if (col < NCOL) as_global_rw(J.wpart)[((size_t)ks * NCOL + col) * J.rows + 32 * g + j] = ya[0][c] + ya[1][c];
        }
        k = nwp + (int)wave_atomic_add(pc, lane);
    }
    const unsigned left = wave_atomic_add(pc + 1, lane);
    if (lane == 0 && left == (unsigned)nwp - 1) {
        __hip_atomic_store(pc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pc + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int NCOL>
static int launch_gemv_wave_mx_t(const GemvJob *jobs, const uint32_t *ujob, int units, unsigned *ctr, const uint32_t *a2, hipStream_t st,
                                 hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr) {
    const int grid = mx_wg_per_cu() * num_cus();
    if (e0 || e1)
        hipExtLaunchKernelGGL((k_gemv_wave_mx<NCOL>), dim3(grid), dim3(64 * mx_waves()), 0, st, e0, e1, 0, jobs, ujob, units, ctr, a2);
    else
        hipLaunchKernelGGL((k_gemv_wave_mx<NCOL>), dim3(grid), dim3(64 * mx_waves()), 0, st, jobs, ujob, units, ctr, a2);
    return hip_check(hipGetLastError(), "k_gemv_wave_mx launch");
}

// defined in the instantiation units
int launch_gemv_q8(int ncols, int cm, const GemvJob &job0, int tasks, const uint32_t *a2, hipStream_t st);
// block_q8_1: one column of a class-3 tensor has its own instantiation (cm kCmC3), every other case the generic one
int launch_gemv_q81(int ncols, int cm, const GemvJob &job0, int tasks, const uint32_t *a2, hipStream_t st);
int launch_gemv_partials(int act, const GemvJob &job0, const uint32_t *a2, hipStream_t st);
int launch_gemv_rg(int ncols, int cm, const RgJobs &jobs, int ng, const uint32_t *a2, hipStream_t st);
int launch_gemv_rg_multi(int cm, const RgJobs &jobs, int ng, const uint32_t *a2, hipStream_t st);
// host planning shared by the multi-linear launch and the decode-step kernel (p8x_gemv.hip)
int plan_gemv_multi(const p8x_tensor *const *ts, int n, const float *x, size_t ldx, float *const *y, const size_t *ldy, float *out,
                    RgJobs &R, int &cm, int &ng);
int check_shared_input(const p8x_tensor *const *ts, int n, const float *x, size_t ldx, const char *what);
int class_set(const size_t hist[8], bool in_order = true);
int launch_gemv_wave(int ncols, int cm, const GemvJob *jobs, const uint32_t *ujob, int units, unsigned *ctr, const uint32_t *a2, hipStream_t st,
                     hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr);
// the matrix-core grouped launch (class 3, activations in the k_act_q8_128_mx_batch / k_act_x16_batch<true>
// layout), 2..8 columns
int launch_gemv_wave_mx(int ncols, const GemvJob *jobs, const uint32_t *ujob, int units, unsigned *ctr, const uint32_t *a2, hipStream_t st,
                        hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr);
// batches the matrix-core kernel can run (class set, columns it multiplies: x16 batches two per column), and from how
// many columns the plan takes it (on the Qwen3-14B stack it is slower at 2 columns, even at 3, and faster from 4:
// 0.84 / 0.96 ms against 0.92 / 1.43 ms per step at 4 / 8 columns)
__host__ __device__ constexpr bool wave_mx(int cm, int ncv) { return cm == kCmC3 && ncv >= 2 && ncv <= 8; }
constexpr int kMxMinCols = 4;

}  // namespace p8x
