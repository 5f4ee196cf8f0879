// p8x_step.hip -- a batch-1 decode step's chain of linears in one persistent launch.
//
// The reference launches one kernel per MUL_MAT node (CPU.patch:2615-2631, :4466-4521), so a step of L layers runs
// 4 L + 1 dependent launches (q/k/v, o, gate/up, down, then the head), each paying the launch and the kernel-boundary
// cache work, and each rebuilding the 64 KB coset table in every workgroup. Here one cooperative launch walks the
// whole chain with the table built once per workgroup. Two kernels:
//
// k_chain (chains whose tensors are all class 3 with their tiles in order: the decode stream of the shipped files'
// bulk) is a dataflow kernel with no grid barrier. Every output row a later stage reads is published as an 8-byte
// (value, tag) pair by one 64-bit store; the tag is the run's epoch mixed with the value, so a consumer polls the
// pairs themselves and accepts a value only once its tag matches (one memory round trip from the producer's store to
// the consumer's data, instead of store completion + barrier arrival + barrier release + data load). Each
// 16-wave workgroup splits into 4 sync waves and 12 compute waves:
//   * sync waves poll the stage's input blocks, combine the producer's parts (K-chunk partial sums in order; for a
//     swiglu input silu(gate) * up), rotate and quantize them into LDS, and after the compute phase sum the compute
//     waves' partial rows in a fixed order, add the clamp delta and publish;
//   * compute waves hold a ring of kChRing class-3 tiles in registers and issue each tile kChRing tiles ahead of its
//     use, across stage boundaries: a stage's weights are in flight while the previous stage's outputs are still
//     travelling. They never wait on a global value other than their own tiles (vector loads complete in order, so
//     a poll behind the prefetches would wait for all of them), which is why polling and stores are left to the
//     sync waves.
// Two workgroup barriers per stage order the roles (input in LDS -> compute -> partial rows in LDS -> epilogue).
// The run's epoch is read from device memory at the start and advanced by the last workgroup to finish, so runs
// replay from a HIP graph unchanged. Polls are bounded; a poll that gives up raises the fail flag, after which
// every poll returns at once and every wave still reaches every barrier and the end.
//
// k_step (any class set) runs the row-group GEMV body of k_gemv_rg per stage with a grid barrier between stages:
// per-XCD arrival counters, one counter above them, and a release word per XCD (the barrier targets derive from a
// device-side run counter, so this kernel also replays from a graph).
//
// Cross-workgroup hand-off rules. Published pairs are agent-scope 64-bit stores (sc1: written through the XCD's L2
// to the coherence point) and are read with agent-scope loads (sc1). A 16-byte load covers two whole pairs; the tag
// check also rejects a pair whose halves came from different stores, since a value with another epoch's or another
// value's tag fails it. k_step: outputs are agent-scope stores, every wave waits vmcnt(0) before the workgroup's
// arrival, inputs are agent-scope loads issued after the release was observed.
#include <climits>
#include <cstring>
#include <vector>

#include "../../include/p8x.h"
#include "p8x_gemv.h"

namespace p8x {

#ifdef P8X_TIMELINE
unsigned long long *timeline_buf() {
    static unsigned long long *b = nullptr;
    const size_t bytes = ((size_t)kTimelineRecords * 8 + 1) * 8;
    if (!b && hipMalloc((void **)&b, bytes) == hipSuccess) (void)hipMemset(b, 0, bytes);
    return b;
}
#endif

typedef unsigned long long u64;

// step-wide device words: [0] runs completed (the epoch source), [1] workgroups finished in this run, [2] fail flag,
// then (k_step) the barrier: top arrival counter at [32], per-XCD arrival counters at [64 + 32 x], release words at
// [320 + 32 x] (each on its own 128-byte line)
constexpr int kSyncWords = 640;
constexpr int kSwRuns = 0, kSwExit = 1, kSwFail = 2, kSwTop = 32, kSwXcd = 64, kSwRel = 320;

__device__ __forceinline__ unsigned ld_agent(const unsigned *p) {
    return __hip_atomic_load(const_cast<unsigned *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(unsigned *p, unsigned v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ unsigned add_agent(unsigned *p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A launch's end: the last workgroup to finish advances the run counter (read by every workgroup at the start of
// the next run) and resets the exit counter. Stream order makes both visible to the next launch.
__device__ __forceinline__ void run_exit(unsigned *words, unsigned run, int G) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (add_agent(words + kSwExit, 1u) == (unsigned)G - 1u) {
        st_agent(words + kSwExit, 0u);
        st_agent(words + kSwRuns, run);
    }
}

// ================================================================================================ k_chain
constexpr int kChWaves = 16, kChSync = 4, kChComp = kChWaves - kChSync;
constexpr int kChRing = 6;          // register tile buffers per compute wave (class 3: 9 VGPRs each)
constexpr int kChMaxBlk = 32;       // 256-blocks of a stage's input per workgroup (LDS activations)
constexpr int kChSlots = 4;         // units one compute wave's tile range may touch in a stage
constexpr int kChMaxStages = 224;   // stage records held in LDS
constexpr int kChMaxTiles = 320;    // tiles of a workgroup in one stage (their row scales in LDS)
constexpr uint32_t kChTileBytes = 2048;   // class 3: 2 half-slices x 8 words x 32 lanes x 4 bytes
constexpr uint32_t kChMix = 0x9E3779B1u;
constexpr int kBufSC1 = 16;         // buffer-load cache policy: sc1 (agent-coherent, served from the coherence point)

// One job of a stage (a linear on the stage's input). Outputs: y (plain floats at original rows) when the producer
// writes them itself (one K-chunk, no swiglu); pub, when a later stage reads this output: part p (K-chunk p) of
// original row r at pub[p * rows + r].
struct ChJob {
    const uint32_t *D;
    const uint16_t *Sg;
    const uint16_t *prmd;
    const int *cp;
    const uint16_t *cc;
    const float *cv;
    float *y;
    u64 *pub;
    unsigned dbytes;
    int rows;
};

// A stage's input: the caller's activations (parts == 0), or the published output of an earlier stage: `parts`
// K-chunk parts summed in order, and for a swiglu output the gate (pub[0]) and up (pub[1]) vectors, x = silu(gate)
// * up. out: the caller's buffer of that earlier output when its producer did not write it (split or swiglu), written
// here by designated readers (block bl of a workgroup's chunk by the workgroup of rank bl % active workgroups).
struct ChInput {
    const float *x;
    const u64 *pub[2];
    float *out;
    int parts, glu;
};

struct ChStage {
    ChJob job[kRgMaxJobs];
    ChInput in;
    const float *ic;
    int nj, nks, kchunk, nb, K;
    int ngo[kRgMaxJobs];   // row-group offsets of jobs 1..3 (INT_MAX when absent), then the total
};

// The compute waves' copy of a stage (LDS): each job's payload and the stage's row-group numbering.
struct ChTileJob {
    const uint32_t *D;
    unsigned dbytes, pad;
};
struct ChTileStage {
    ChTileJob job[kRgMaxJobs];
    int nb, pad[3];
    int ngo[kRgMaxJobs];
};
static_assert(sizeof(ChTileStage) == 96, "stage record: 96 bytes");

// A workgroup's share of stage s, computed on the host (no divisions in the kernel): K-chunk ks, block range
// [kb0, kb0 + nbk), its nr units u = r + k m (k < nr), and the number of workgroups of its K-chunk with work (nact).
struct ChPlanRec {
    int16_t nr, kb0, nbk, nact, r, m, ks, pad;
};
static_assert(sizeof(ChPlanRec) == 16, "plan record: 16 bytes");

// A clamp-delta entry of a workgroup, resolved on the host: stage, unit k of the workgroup's units of that stage,
// row j of the unit, the column within the workgroup's K-chunk (lcol) and the value. K-split stages give each entry to
// the K-chunk that holds its column (the consumers sum the chunks). Sorted by (stage, k, j, entry order of the row).
struct ChDelta {
    uint32_t skj;    // stage | k << 16 | j << 24
    uint32_t lcol;
    float val;
    uint32_t pad;
};
constexpr int kChMaxDelta = 256;   // entries per workgroup (LDS)
constexpr int kChMaxDes = 4;       // designated input blocks of a workgroup per stage held in LDS
constexpr int kChPoll = 2;         // sync waves 0 .. kChPoll - 1 poll the input, the others publish

// A workgroup's share of a stage: K-chunk ks (workgroups w with w % nks == ks, m of them), its units (job, row
// group) u = r + k m for k < nr, where r = w / nks and units are numbered over the jobs' row groups.
struct ChPlan {
    int ks, m, r, nr, kb0, nbk, nact;
};
__host__ __device__ inline ChPlan ch_plan(int nks, int kchunk, int nb, int U, int w, int G) {
    ChPlan p;
    p.ks = w % nks;
    p.m = (G - 1 - p.ks) / nks + 1;
    p.r = w / nks;
    p.nr = p.r < U ? (U - p.r + p.m - 1) / p.m : 0;
    p.kb0 = p.ks * kchunk;
    p.nbk = nb - p.kb0 < kchunk ? nb - p.kb0 : kchunk;
    p.nact = U < p.m ? U : p.m;
    return p;
}
// compute wave c's tiles [t0, t1) of the workgroup's T = nr * nbk (unit-major)
__host__ __device__ inline int ch_t0(int c, int T) { return c * T / kChComp; }

struct ChSmem {
    uint32_t tab[kTabWords];               // LDS address 0
    uint32_t xq[kChMaxBlk * 64];           // quantized input: [block][half][32 words]
    float xd[kChMaxBlk * 2];               // [block][half] scales
    float red[kChComp][kChSlots][32];      // compute waves' partial rows
    uint16_t sc[2][kChMaxTiles * 32];      // row scales of stage s in sc[s & 1]: [unit][block][row]
    f32x4 dsx[kChMaxDes][64];              // combined input blocks the workgroup writes to the caller's buffer
    int dsb[kChMaxDes];                    // and their global block indices (-1: none)
    ChTileStage ts[kChMaxStages];
    ChPlanRec pl[kChMaxStages];            // this workgroup's share of each stage
    ChDelta dl[kChMaxDelta];               // this workgroup's clamp-delta entries
    float dxv[kChMaxDelta];                // their input values (written while the input is quantized)
    int ndl;
    unsigned run;
#ifdef P8X_TIMELINE
    u64 tstamp;                            // compute wave 0: its tiles of the stage done
    u64 tpoll;                             // poller: its first quad's first whole load (100 MHz ticks; bit 63: ready)
    unsigned tprobes;                      // and the probes that quad needed | its rotation + quantization ticks << 16
#endif
};

__device__ __forceinline__ void ch_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ int rfl(int v) { return __builtin_amdgcn_readfirstlane(v); }
template <typename T>
__device__ __forceinline__ T *rfl_ptr(T *p) {
    const u64 v = (u64)(uintptr_t)p;
    const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)v), hi = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(v >> 32));
    return (T *)(uintptr_t)(((u64)hi << 32) | lo);
}

__device__ __forceinline__ u64 ch_pack(float v, unsigned run) {
    const unsigned b = __float_as_uint(v);
    return ((u64)(run ^ (b * kChMix)) << 32) | b;
}
__device__ __forceinline__ bool ch_ok(uint32_t v, uint32_t t, unsigned run) { return t == (run ^ (v * kChMix)); }

// ------------------------------------------------------------------------------------------------ compute waves
// One ring slot: a class-3 lane-slice, 8 payload words in two 16-byte loads (the row scales come from LDS, staged by
// the sync waves).
//
// The ring's loads are issued from inline asm and waited for by an explicit s_waitcnt fused with the slot's use:
// the compiler's own wait counts through this loop (stage boundaries with barriers between the tiles) fall back to
// waiting for every load in flight, which would drain the ring at each tile. A slot is used after the other
// kChRing - 1 slots were issued (2 vector-memory operations each), so vmcnt(2 (kChRing - 1)) means that its loads are
// complete; vector-memory operations the compiler adds anywhere in between only make that count conservative. The
// slot's registers are written by the load asm and read first by the wait asm (their "+v" operands); a test checks
// the built kernel for reads of them between the two (the asm comments name the registers).
typedef int i32x4_t __attribute__((ext_vector_type(4)));
constexpr int kChWaitVm = 2 * (kChRing - 1);

__device__ __forceinline__ i32x4_t ch_rsrc(const void *p, uint32_t bytes) {
    const u64 a = (u64)(uintptr_t)p;
    i32x4_t r;
    r.x = (int)(uint32_t)a;
    r.y = (int)((uint32_t)(a >> 32) & 0xFFFFu);
    r.z = (int)bytes;
    r.w = kBufFlags;
    return r;
}

struct ChSlot {
    u32x4_t a, b;   // payload words 0-3 and 4-7 of the lane-slice
    __device__ __forceinline__ void load(i32x4_t rd, uint32_t toff, uint32_t vo) {
        __asm__ volatile(
            "buffer_load_dwordx4 %0, %2, %3, %4 offen nt\n\t"
            "buffer_load_dwordx4 %1, %2, %3, %4 offen offset:512 nt ; ring load %0 %1"
            : "=&v"(a), "=&v"(b)
            : "v"(vo), "s"(rd), "s"(toff));
    }
    // the slot's loads complete (see above); afterwards its registers hold the loaded data
    __device__ __forceinline__ void wait() { __asm__ volatile("s_waitcnt vmcnt(%2) ; ring wait %0 %1" : "+v"(a), "+v"(b) : "n"(kChWaitVm)); }
};

// Position in a compute wave's tile sequence (wave-uniform): stage s, tiles left in it, unit k and block bl, and the
// stage's plan; for issuing, the current unit's payload and scale resources.
struct ChCur {
    int s, left, k, bl, nbk, kb0, r, m, nb, ngo1, ngo2, ngo3;
    int kfirst;
    uint32_t tile;   // (g * nb + kb0 + bl): tile index within the job
    const uint32_t *D;
    unsigned dbytes;
};

__device__ __forceinline__ void ch_unit(const ChSmem &sm, ChCur &q) {
    const int u = q.r + q.k * q.m;
    const int jb = (u >= q.ngo1) + (u >= q.ngo2) + (u >= q.ngo3);
    const int g = u - (jb == 0 ? 0 : jb == 1 ? q.ngo1 : jb == 2 ? q.ngo2 : q.ngo3);
    const ChTileJob &J = sm.ts[q.s].job[jb];
    q.D = rfl_ptr(J.D);
    q.dbytes = (unsigned)rfl((int)J.dbytes);
    q.tile = (uint32_t)(g * q.nb + q.kb0 + q.bl);
}

// stage s's plan for compute wave c: tiles left, first unit and block
__device__ __forceinline__ void ch_stage(const ChSmem &sm, ChCur &q, int s, int c) {
    q.s = s;
    const ChTileStage &S = sm.ts[s];
    const ChPlanRec &P = sm.pl[s];
    const int nr = rfl(P.nr), nbk = rfl(P.nbk);
    const int T = nr * nbk, t0 = ch_t0(c, T), t1 = ch_t0(c + 1, T);
    q.left = t1 - t0;
    q.nbk = nbk; q.kb0 = rfl(P.kb0); q.r = rfl(P.r); q.m = rfl(P.m); q.nb = rfl(S.nb);
    q.ngo1 = rfl(S.ngo[0]); q.ngo2 = rfl(S.ngo[1]); q.ngo3 = rfl(S.ngo[2]);
    q.k = nbk > 0 ? t0 / nbk : 0;
    q.bl = t0 - q.k * nbk;
    q.kfirst = q.k;
}

// issue cursor: the next tile into slot r (past the chain's end: an empty resource, no memory traffic), then advance
__device__ __forceinline__ void ch_issue(const ChSmem &sm, ChCur &q, int nst, int c, ChSlot &r, uint32_t vo) {
    const bool on = q.s < nst;
    // wave-uniform (the compiler cannot tell through the cursor's loops): scalar offsets, no waterfall loads
    const uint32_t tile = (uint32_t)rfl((int)q.tile);
    const uint32_t toff = on ? tile * kChTileBytes : 0u;
    __builtin_amdgcn_s_setprio(2);
    r.load(ch_rsrc(q.D, on ? q.dbytes : 0u), toff, vo);
    __builtin_amdgcn_s_setprio(0);
    if (!on) return;
    --q.left;
    ++q.tile;
    if (++q.bl == q.nbk) {
        q.bl = 0;
        ++q.k;
        if (q.left > 0) ch_unit(sm, q);
    }
    while (q.left == 0) {
        if (++q.s >= nst) return;
        ch_stage(sm, q, q.s, c);
        if (q.left > 0) ch_unit(sm, q);
    }
}

__device__ __forceinline__ void ch_flush(ChSmem &sm, int c, int slot, int lane, float &yacc) {
    const float v = yacc + __shfl_xor(yacc, 32);
    if (lane < 32) sm.red[c][slot][lane] = v;
    yacc = 0.f;
}

// Integer sum of one class-3 tile (the quad_isum products) with the LDS reads one group of four chunks ahead of the
// dot products and the accumulator pinned after each group: at most two groups' table words and activation words are
// live, which leaves the registers to the tile ring.
__device__ __forceinline__ int ch_isum(const uint32_t *tab, const QuadSlice<3> &raw, uint32_t bankbytes, lds_cptr xl) {
    const uint32_t H = raw.coset_bits();
    u32x4_t xv[2];
    uint32_t wv[2][4];
    auto fetch = [&](int q, int b) {
        xv[b] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t *>(xl + 4 * q);
        const uint32_t hq = coset_bytes(H, bankbytes, q);
#pragma unroll
        for (int e = 0; e < 4; ++e) wv[b][e] = lds_word(tab, raw.template addr<0>(4 * q + e, hq));
    };
    int acc = 0;
    fetch(0, 0);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        if (q + 1 < 8) fetch(q + 1, (q + 1) & 1);
        const int b = q & 1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t xc = xv[b][e];
            acc = __builtin_amdgcn_sdot4((int)wv[b][e], (int)xc, acc, false);
        }
        __asm__ volatile("" : "+v"(acc)::"memory");
    }
    return acc;
}

// one tile from ring slot `slot`: block bl of unit k, the row scale from the stage's LDS scales
__device__ __forceinline__ void ch_tile(const ChSmem &sm, ChSlot &slot, int s, int k, int bl, int nbk, int hs, int j, uint32_t bankbytes,
                                        float &yacc) {
    slot.wait();
    QuadSlice<3> r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r.w[i] = slot.a[i];
        r.w[4 + i] = slot.b[i];
    }
    lds_cptr xl = (lds_cptr)(sm.xq + bl * 64 + hs * 32);
    __asm__ volatile("" : "+v"(xl));
    const int isum = ch_isum(sm.tab, r, bankbytes, xl);
    const float sc = half_to_float(sm.sc[s & 1][(k * nbk + bl) * 32 + j]);
    yacc += ((float)isum * sm.xd[2 * bl + hs]) * sc;
}

__device__ __forceinline__ void chain_compute(ChSmem &sm, int nst, int c, int lane) {
    const int hs = lane >> 5, j = lane & 31;
    const uint32_t bankbytes = (uint32_t)(j << 2) * 0x01010101u;
    const uint32_t vo = QuadSlice<3>::quad_offset(hs, j);
    // issue cursor: the first stage with tiles for this wave, then kChRing tiles ahead
    ChCur iq;
    iq.s = 0;
    ch_stage(sm, iq, 0, c);
    while (iq.left == 0 && ++iq.s < nst) ch_stage(sm, iq, iq.s, c);
    if (iq.s < nst) ch_unit(sm, iq);
    ChSlot ring[kChRing];
#pragma unroll
    for (int i = 0; i < kChRing; ++i) ch_issue(sm, iq, nst, c, ring[i], vo);
    // compute cursor
    ChCur q;
    ch_barrier();   // B1 of stage 0: its input is in LDS
    ch_stage(sm, q, 0, c);
    float yacc = 0.f;
    bool dirty = false;
    // every pass through the loop's back edge has consumed and reissued all kChRing slots in order
    for (;;) {
#pragma unroll
        for (int i = 0; i < kChRing; ++i) {
            if (q.left == 0) {   // the stage's tiles are done: partial rows out, then stages until one has tiles
                if (dirty) ch_flush(sm, c, q.k - q.kfirst, lane, yacc);
                dirty = false;
                int s = q.s;
                for (;;) {
#ifdef P8X_TIMELINE
                    if (lane == 0 && c == 0) sm.tstamp = __builtin_amdgcn_s_memrealtime();
#endif
                    ch_barrier();   // B2: partial rows in LDS
                    if (++s >= nst) goto out;
                    ch_barrier();   // B1: the next stage's input in LDS
                    ch_stage(sm, q, s, c);
                    if (q.left > 0) break;
                }
            }
            ch_tile(sm, ring[i], q.s, q.k, q.bl, q.nbk, hs, j, bankbytes, yacc);
            dirty = true;
            ch_issue(sm, iq, nst, c, ring[i], vo);
            --q.left;
            if (++q.bl == q.nbk && q.left > 0) {   // the unit is complete and the stage goes on
                ch_flush(sm, c, q.k - q.kfirst, lane, yacc);
                dirty = false;
                q.bl = 0;
                ++q.k;
            }
        }
    }
out:;
}

// ------------------------------------------------------------------------------------------------ poller waves
// A poller wave takes its input four 256-blocks at a time (a quad): lane l holds columns 16 (l & 15) .. + 15 of block
// (l >> 4) of the quad, so the Hadamard stages h = 1 .. 8 are in-lane, h = 16 .. 128 cross lanes inside the lane's row
// of 16 (DPP moves, no LDS round trip), and each half-block's maximum is three DPP steps: four blocks' rotations and
// quantizations run side by side in one wave. The butterflies are the reference's (a + b, a - b on the same pairs,
// CPU.patch:533-554), so x' is bit-identical whatever lane computes it.

// the lane's 16 columns of one published vector part: 16 (value, tag) pairs in 8 16-byte loads
struct ChPart {
    u32x4_t q[8];
    __device__ __forceinline__ uint32_t value(int e) const { return q[e >> 1][2 * (e & 1)]; }
    __device__ __forceinline__ bool ok(unsigned run) const {
        bool r = true;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t v0 = q[i][0], t0 = q[i][1], v1 = q[i][2], t1 = q[i][3];
            r = r && ch_ok(v0, t0, run) && ch_ok(v1, t1, run);
        }
        return r;
    }
};

// a quad's input in registers: VP published parts (VP = parts x (1 + glu) <= 2; part i is vector i / parts, K-chunk
// i % parts), or the caller's activations (VP == 0); and the rotation ic
template <int VP>
struct ChQuad {
    ChPart p[VP > 0 ? VP : 1];
    f32x4 xe[4], c[4];
};

// lane's block within the quad and column in the block; blocks past the chunk read the chunk's last block (in bounds)
__device__ __forceinline__ uint32_t ch_quad_col(const ChPlan &p, int Q, int lane) {
    const int bl = min(4 * Q + (lane >> 4), p.nbk - 1);
    return 256u * (uint32_t)(p.kb0 + bl) + 16u * (uint32_t)(lane & 15);
}

template <int VP>
__device__ __forceinline__ void ch_quad_issue(kptr<const ChStage> st, const ChPlan &p, int Q, int lane, ChQuad<VP> &I) {
    const uint32_t col = ch_quad_col(p, Q, lane);
    const gptr<const f32x4> icv = as_global(reinterpret_cast<const f32x4 *>(st->ic + col));
#pragma unroll
    for (int i = 0; i < 4; ++i) I.c[i] = icv[i];
    if constexpr (VP == 0) {
        const gptr<const f32x4> xv = as_global(reinterpret_cast<const f32x4 *>(st->in.x + col));
#pragma unroll
        for (int i = 0; i < 4; ++i) I.xe[i] = xv[i];
    } else {
        const int parts = st->in.parts, K = st->K;
#pragma unroll
        for (int i = 0; i < VP; ++i) {
            const int v = i / parts, pp = i % parts;
            const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(v ? st->in.pub[1] : st->in.pub[0], (uint32_t)parts * (uint32_t)K * 8u);
            const uint32_t off = ((uint32_t)pp * (uint32_t)K + col) * 8u;
#pragma unroll
            for (int k = 0; k < 8; ++k) I.p[i].q[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16u * k, 0, kBufSC1);
        }
    }
}

// Readiness probe of a quad's blocks: 16 lanes per block, each reading one pair (8 bytes) of one part, evenly spaced
// over the block's 256 values, so that a wait costs little traffic; the quad is loaded whole once the probes pass (and
// every tag is checked again there).
template <int VP>
__device__ __forceinline__ bool ch_probe(kptr<const ChStage> st, const ChPlan &p, int Q, int lane, unsigned run) {
    constexpr int PER = 16 / (VP > 0 ? VP : 1), STRIDE = 256 / PER;   // probes per part of a block, rows between them
    const int i = lane >> 4, ip = (lane & 15) / PER, q = lane % PER;
    bool ok = true;
    if (4 * Q + i < p.nbk) {
        const int parts = st->in.parts, K = st->K;
        const int v = ip / parts, pp = ip % parts;
        const u64 *base = v ? st->in.pub[1] : st->in.pub[0];
        u64 *src = const_cast<u64 *>(base) + (size_t)pp * K + 256 * (p.kb0 + 4 * Q + i) + STRIDE * q + STRIDE - 1;
        const u64 pr = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = ch_ok((uint32_t)pr, (uint32_t)(pr >> 32), run);
    }
    return __all(ok);
}

__device__ __forceinline__ float ch_silu_mul(float gate, float up) { return gate / (1.0f + expf(-gate)) * up; }

// The workgroup's clamp-delta entries of the current stage: [e0, e1) of the LDS list.
struct ChDeltaRange {
    int e0, e1;
};

__device__ __forceinline__ void ch_delta_next(const ChSmem &sm, int s, int ndl, ChDeltaRange &dr) {
    dr.e0 = dr.e1;
    while (dr.e1 < ndl && (int)(rfl((int)sm.dl[dr.e1].skj) & 0xFFFF) == s) ++dr.e1;
}

// the lane's 16 rotated values x' = FWHT(x ic) / 16 of its block (butterflies h = 1 .. 128 in index order)
__device__ __forceinline__ void ch_rotate16(float (&v)[16], int lane) {
#pragma unroll
    for (int h = 1; h < 16; h <<= 1)
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if ((i & h) == 0) {
                const float a = v[i], b = v[i + h];
                v[i] = a + b;
                v[i + h] = a - b;
            }
    // h = 16, 32, 64, 128: lanes 1, 2, 4, 8 apart in the row of 16
    auto stage = [&](auto M) {
        constexpr int m = decltype(M)::value;
        const bool upper = (lane & m) != 0;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float q = lane_xor<m>(v[e], lane);
            v[e] = upper ? q - v[e] : v[e] + q;
        }
    };
    stage(std::integral_constant<int, 1>{});
    stage(std::integral_constant<int, 2>{});
    stage(std::integral_constant<int, 4>{});
    stage(std::integral_constant<int, 8>{});
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] *= 0.0625f;
}

// The quad's blocks of the workgroup's K-chunk: combined, the input values of this stage's clamp-delta entries in them
// saved (dxv), rotated and quantized into LDS (8 bits per 128 columns, the vrc_prep_block rule). A designated
// workgroup (block bl of its K-chunk when bl % nact == r) also writes the combined values to the caller's buffer: they
// wait in LDS for the publisher waves (stores would queue the poller's next loads behind them), or, past the LDS
// slots, are stored at once.
template <int VP>
__device__ __forceinline__ void ch_quad_store(ChSmem &sm, kptr<const ChStage> st, const ChQuad<VP> &I, int Q, const ChPlan &p,
                                              const ChDeltaRange &dr, int lane) {
    const int g = lane >> 4, l = lane & 15, bl = 4 * Q + g;
    const bool valid = bl < p.nbk;
    float x[16];
    if constexpr (VP == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[4 * i] = I.xe[i].x; x[4 * i + 1] = I.xe[i].y; x[4 * i + 2] = I.xe[i].z; x[4 * i + 3] = I.xe[i].w;
        }
    } else {
        const int parts = st->in.parts, glu = st->in.glu;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float a0 = __uint_as_float(I.p[0].value(e));
            if constexpr (VP == 1) {
                x[e] = a0;
            } else {
                const float a1 = __uint_as_float(I.p[1].value(e));
                x[e] = glu ? ch_silu_mul(a0, a1) : (parts > 1 ? a0 + a1 : a0);
            }
        }
    }
    for (int e = dr.e0; e < dr.e1; ++e) {
        const int lc = (int)sm.dl[e].lcol;
        if (valid && (lc >> 8) == bl && ((lc & 255) >> 4) == l) {
            float val = 0.f;
#pragma unroll
            for (int i = 0; i < 16; ++i) val = (lc & 15) == i ? x[i] : val;
            sm.dxv[e] = val;
        }
    }
    float *out = st->in.out;
    if (out && valid && bl % p.nact == p.r) {
        const int slot = (bl - p.r) / p.nact;
        f32x4 *dst = slot < kChMaxDes ? &sm.dsx[slot][4 * l] : nullptr;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f32x4 q4;
            q4.x = x[4 * i]; q4.y = x[4 * i + 1]; q4.z = x[4 * i + 2]; q4.w = x[4 * i + 3];
            if (dst) dst[i] = q4;
            else as_global_rw(reinterpret_cast<f32x4 *>(out + 256 * (p.kb0 + bl) + 16 * l))[i] = q4;
        }
        if (dst && l == 0) sm.dsb[slot] = p.kb0 + bl;
    }
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[4 * i] = x[4 * i] * I.c[i].x; v[4 * i + 1] = x[4 * i + 1] * I.c[i].y;
        v[4 * i + 2] = x[4 * i + 2] * I.c[i].z; v[4 * i + 3] = x[4 * i + 3] * I.c[i].w;
    }
    ch_rotate16(v, lane);
    float am = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) am = fmaxf(am, fabsf(v[e]));
    am = fmaxf(am, lane_xor<1>(am, lane));
    am = fmaxf(am, lane_xor<2>(am, lane));
    am = fmaxf(am, lane_xor<4>(am, lane));   // lanes 0-7 of the row hold half 0, lanes 8-15 half 1
    const float dd = div_rn(am, 127.f);
    const float id = dd > 0.f ? div_rn(1.f, dd) : 0.f;
    u32x4_t packed;
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) word |= (uint32_t)(uint8_t)__float2int_rn(v[4 * w4 + b] * id) << (8 * b);
        packed[w4] = word;
    }
    if (valid) {
        *reinterpret_cast<u32x4_t *>(&sm.xq[bl * 64 + 4 * l]) = packed;
        if ((l & 7) == 0) sm.xd[2 * bl + (l >> 3)] = dd;
    }
}

// The poller wave's quads Q = pw, pw + kChPoll, ... of the workgroup's K-chunk: load each whole and check every tag;
// while some are not from this run, probe (bounded) and load again once the probes pass.
template <int VP>
__device__ __forceinline__ void ch_prep_t(ChSmem &sm, kptr<const ChStage> st, const ChPlan &p, const ChDeltaRange &dr, int pw, int lane,
                                          unsigned run, unsigned *words, unsigned spin, bool &failed) {
    const int nq = (p.nbk + 3) / 4;
    for (int Q = pw; Q < nq; Q += kChPoll) {
        ChQuad<VP> I;
#ifdef P8X_TIMELINE
        const u64 tq0 = __builtin_amdgcn_s_memrealtime();
#endif
        ch_quad_issue<VP>(st, p, Q, lane, I);
        auto whole = [&]() {
            bool ok = true;
#pragma unroll
            for (int i = 0; i < VP; ++i) ok = ok && I.p[i].ok(run);
            return __all(ok) != 0;
        };
        bool ready = VP == 0 || whole();
#ifdef P8X_TIMELINE
        if (Q == pw) sm.tpoll = (__builtin_amdgcn_s_memrealtime() - tq0) | ((u64)ready << 63);
        unsigned probes = 0;
#endif
        if (!ready && !failed) {
            for (unsigned n = 0;; ++n) {
                __builtin_amdgcn_s_sleep(2);
#ifdef P8X_TIMELINE
                ++probes;
#endif
                if (ch_probe<VP>(st, p, Q, lane, run)) {
                    ch_quad_issue<VP>(st, p, Q, lane, I);
                    if (whole()) break;
                }
                if (n >= spin || ((n & 15) == 15 && ld_agent(words + kSwFail) != 0u)) {
                    if (lane == 0) st_agent(words + kSwFail, 1u);
                    failed = true;
                    break;
                }
            }
        }
#ifdef P8X_TIMELINE
        const u64 tq1 = __builtin_amdgcn_s_memrealtime();
#endif
        ch_quad_store<VP>(sm, st, I, Q, p, dr, lane);
#ifdef P8X_TIMELINE
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (Q == pw) sm.tprobes = probes | ((unsigned)(__builtin_amdgcn_s_memrealtime() - tq1) << 16);
#endif
    }
}

__device__ __forceinline__ void ch_prep(ChSmem &sm, kptr<const ChStage> st, const ChPlan &p, const ChDeltaRange &dr, int pw, int lane,
                                        unsigned run, unsigned *words, unsigned spin, bool &failed) {
    const int vp = st->in.parts * (1 + st->in.glu);
    if (vp == 0) ch_prep_t<0>(sm, st, p, dr, pw, lane, run, words, spin, failed);
    else if (vp == 1) ch_prep_t<1>(sm, st, p, dr, pw, lane, run, words, spin, failed);
    else ch_prep_t<2>(sm, st, p, dr, pw, lane, run, words, spin, failed);
}

constexpr int kChPub = kChSync - kChPoll;   // publisher waves
constexpr int kChUnitsPerPub = 8;           // units of a stage per publisher wave

// stage s's row scales into sc[s & 1]: unit k, block bl, row r at [(k nbk + bl) 32 + r], each unit's run
// Sg[g][kb0 .. kb0 + nbk - 1][32] copied by direct-to-LDS loads (publisher wave qw: units qw, qw + kChPub, ...)
__device__ __forceinline__ void ch_scales(ChSmem &sm, kptr<const ChStage> st, int s, const ChPlan &p, int qw, int lane) {
    const int n16 = 4 * p.nbk;   // 16-byte pieces of a unit's run
    for (int k = qw; k < p.nr; k += kChPub) {
        const int u = p.r + k * p.m;
        const int jb = (u >= st->ngo[0]) + (u >= st->ngo[1]) + (u >= st->ngo[2]);
        const int g = u - (jb == 0 ? 0 : jb == 1 ? st->ngo[0] : jb == 2 ? st->ngo[1] : st->ngo[2]);
        const uint16_t *src = st->job[jb].Sg + (size_t)(g * st->nb + p.kb0) * 32;
        uint16_t *dst = sm.sc[s & 1] + k * p.nbk * 32;
        for (int i0 = 0; i0 < n16; i0 += 64)
            if (i0 + lane < n16) __builtin_amdgcn_global_load_lds(src + 8 * (i0 + lane), dst + 8 * i0, 16, 0, 0);
    }
}

// the output rows of the publisher wave's units k = qw, qw + kChPub, ..., loaded during the compute phase
__device__ __forceinline__ void ch_rows(kptr<const ChStage> st, const ChPlan &p, int qw, int lane, int (&ro)[kChUnitsPerPub]) {
#pragma unroll
    for (int i = 0; i < kChUnitsPerPub; ++i) {
        const int k = qw + kChPub * i;
        ro[i] = 0;
        if (k < p.nr) {
            const int u = p.r + k * p.m;
            const int jb = (u >= st->ngo[0]) + (u >= st->ngo[1]) + (u >= st->ngo[2]);
            const int g = u - (jb == 0 ? 0 : jb == 1 ? st->ngo[0] : jb == 2 ? st->ngo[1] : st->ngo[2]);
            ro[i] = as_global(st->job[jb].prmd)[32 * g + (lane & 31)] & 0x7FFF;
        }
    }
}

// the publisher wave's units: the compute waves' partial rows summed in wave order, this K-chunk's clamp-delta entries
// (input values from LDS), then the row published and / or written at its original row
__device__ __forceinline__ void ch_epilogue(const ChSmem &sm, kptr<const ChStage> st, const ChPlan &p, const ChDeltaRange &dr, int qw,
                                            int lane, unsigned run, const int (&ro)[kChUnitsPerPub]) {
    const int T = p.nr * p.nbk, j = lane & 31;
    int c0[kChComp + 1], k0[kChComp];   // the compute waves' tile ranges and first units
#pragma unroll
    for (int c = 0; c <= kChComp; ++c) c0[c] = ch_t0(c, T);
#pragma unroll
    for (int c = 0; c < kChComp; ++c) k0[c] = p.nbk > 0 ? c0[c] / p.nbk : 0;
#pragma unroll
    for (int i = 0; i < kChUnitsPerPub; ++i) {
        const int k = qw + kChPub * i;
        if (k >= p.nr) break;
        const int u = p.r + k * p.m;
        const int jb = (u >= st->ngo[0]) + (u >= st->ngo[1]) + (u >= st->ngo[2]);
        const auto J = &st->job[jb];
        float v = 0.f;
#pragma unroll
        for (int c = 0; c < kChComp; ++c)
            if (c0[c + 1] > c0[c] && c0[c] < (k + 1) * p.nbk && c0[c + 1] > k * p.nbk) v += sm.red[c][k - k0[c]][j];
        for (int e = dr.e0; e < dr.e1; ++e) {
            const uint32_t skj = sm.dl[e].skj;
            if ((int)((skj >> 16) & 0xFF) == k && (int)(skj >> 24) == j) v += sm.dl[e].val * sm.dxv[e];
        }
        const int row = ro[i];
        if (lane < 32) {
            u64 *pub = J->pub;
            if (pub) __hip_atomic_store(pub + (size_t)p.ks * J->rows + row, ch_pack(v, run), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            float *y = J->y;
            if (y) as_global_rw(y)[row] = v;
        }
    }
}

// brings a stage record's cache lines into the scalar cache
__device__ __forceinline__ void ch_touch(kptr<const ChStage> st) {
    const kptr<const unsigned> w = (kptr<const unsigned>)st;
#pragma unroll
    for (unsigned o = 0; o < sizeof(ChStage) / 4; o += 16) {
        const unsigned v = w[o];
        __asm__ volatile("" ::"s"(v));
    }
}

__device__ __forceinline__ ChPlan ch_plan_of(const ChSmem &sm, int s) {
    const ChPlanRec &P = sm.pl[s];
    ChPlan p;
    p.nr = rfl(P.nr); p.kb0 = rfl(P.kb0); p.nbk = rfl(P.nbk); p.nact = rfl(P.nact);
    p.r = rfl(P.r); p.m = rfl(P.m); p.ks = rfl(P.ks);
    return p;
}

// Poller waves: each stage's input into LDS (polled, combined, quantized), then the two barriers of the stage.
__device__ __forceinline__ void chain_poll(ChSmem &sm, const ChStage *stages, int nst, unsigned *words, unsigned spin, int pw, int lane,
                                           int w, int G, unsigned run
#ifdef P8X_TIMELINE
                                           , u64 *tl
#endif
) {
    bool failed = false;
    ChDeltaRange dr;
    dr.e1 = 0;
    const int ndl = rfl(sm.ndl);
    for (int s = 0; s < nst; ++s) {
        const kptr<const ChStage> st = as_const(stages) + s;
        const ChPlan p = ch_plan_of(sm, s);
        ch_delta_next(sm, s, ndl, dr);
#ifdef P8X_TIMELINE
        const u64 t0 = __builtin_amdgcn_s_memrealtime();
#endif
        if (p.nr > 0) ch_prep(sm, st, p, dr, pw, lane, run, words, spin, failed);
#ifdef P8X_TIMELINE
        const u64 t1 = __builtin_amdgcn_s_memrealtime();
#endif
        ch_barrier();   // B1
#ifdef P8X_TIMELINE
        if (pw == 0 && lane == 0) {
            u64 *rec = tl + ((size_t)s * G + w) * 8;
            rec[0] = t0; rec[1] = t1; rec[2] = __builtin_amdgcn_s_memrealtime(); rec[6] = (u64)p.nr;
            rec[7] = (sm.tpoll & 0xFFFFFFFFull) | ((sm.tpoll >> 63) << 62) | ((u64)sm.tprobes << 32);
        }
#endif
        if (s + 1 < nst) ch_touch(st + 1);
        ch_barrier();   // B2
    }
}

// Publisher waves: the row scales of each stage one stage ahead, the caller's copies of combined inputs, and each
// stage's epilogue (after the barrier that ends its compute phase, while the pollers already wait for the next input).
__device__ __forceinline__ void chain_publish(ChSmem &sm, const ChStage *stages, int nst, int qw, int lane, int w, int G, unsigned run
#ifdef P8X_TIMELINE
                                              , u64 *tl
#endif
) {
    ChDeltaRange dr;
    dr.e1 = 0;
    const int ndl = rfl(sm.ndl);
    ch_scales(sm, as_const(stages), 0, ch_plan_of(sm, 0), qw, lane);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");   // stage 0's scales are in LDS
    for (int s = 0; s < nst; ++s) {
        const kptr<const ChStage> st = as_const(stages) + s;
        const ChPlan p = ch_plan_of(sm, s);
        ch_delta_next(sm, s, ndl, dr);
        ch_barrier();   // B1
        int ro[kChUnitsPerPub];
        ch_rows(st, p, qw, lane, ro);
        // the designated copies of this stage's input (their LDS slots free again for the next stage)
        if (qw == 0) {
            float *out = st->in.out;
#pragma unroll
            for (int i = 0; i < kChMaxDes; ++i) {
                const int b = sm.dsb[i];
                if (b >= 0) as_global_rw(reinterpret_cast<f32x4 *>(out + 256 * b))[lane] = sm.dsx[i][lane];
            }
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (lane < kChMaxDes) sm.dsb[lane] = -1;
        }
        if (s + 1 < nst) ch_scales(sm, st + 1, s + 1, ch_plan_of(sm, s + 1), qw, lane);
        ch_touch(st);
        ch_barrier();   // B2
#ifdef P8X_TIMELINE
        const u64 t3 = __builtin_amdgcn_s_memrealtime();
#endif
        if (p.nr > 0) ch_epilogue(sm, st, p, dr, qw, lane, run, ro);
#ifdef P8X_TIMELINE
        if (qw == 0 && lane == 0) {
            u64 *rec = tl + ((size_t)s * G + w) * 8;
            rec[3] = t3; rec[4] = __builtin_amdgcn_s_memrealtime(); rec[5] = sm.tstamp;
        }
#endif
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the next stage's scales are in LDS
    }
}

__global__ __launch_bounds__(64 * kChWaves) __attribute__((amdgpu_waves_per_eu(kChWaves / 4, kChWaves / 4)))
void k_chain(const ChStage *__restrict__ stages, const ChTileStage *__restrict__ tstages, const ChPlanRec *__restrict__ plans,
             const ChDelta *__restrict__ dlist, const int *__restrict__ dl_off, int nst, unsigned *words, unsigned spin,
             const uint32_t *__restrict__ a2
#ifdef P8X_TIMELINE
             , u64 *tl
#endif
) {
    __shared__ ChSmem sm;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = (int)gridDim.x, wg = (int)blockIdx.x;
    CosetTableFill<64 * kChWaves> fill;
    fill.load(a2, tid);
    // the stage records, this workgroup's plans and clamp-delta entries (16-byte pieces)
    for (int i = tid; i < nst * (int)(sizeof(ChTileStage) / 16); i += 64 * kChWaves)
        reinterpret_cast<u32x4_t *>(sm.ts)[i] = as_global(reinterpret_cast<const u32x4_t *>(tstages))[i];
    for (int i = tid; i < nst; i += 64 * kChWaves)
        reinterpret_cast<u32x4_t *>(sm.pl)[i] = as_global(reinterpret_cast<const u32x4_t *>(plans + (size_t)wg * nst))[i];
    const int d0 = as_global(dl_off)[wg], nd = as_global(dl_off)[wg + 1] - d0;
    for (int i = tid; i < nd; i += 64 * kChWaves)
        reinterpret_cast<u32x4_t *>(sm.dl)[i] = as_global(reinterpret_cast<const u32x4_t *>(dlist + d0))[i];
    if (tid == 0) {
        unsigned run = ld_agent(words + kSwRuns) + 1u;
        sm.run = run == 0u ? 1u : run;
        sm.ndl = nd;
    }
    if (tid < kChMaxDes) sm.dsb[tid] = -1;
    fill.store(sm.tab, tid);
    __syncthreads();
    const unsigned run = sm.run;
    if (w < kChPoll) {
        chain_poll(sm, stages, nst, words, spin, w, lane, wg, G, run
#ifdef P8X_TIMELINE
                   , tl
#endif
        );
    } else if (w < kChSync) {
        chain_publish(sm, stages, nst, w - kChPoll, lane, wg, G, run
#ifdef P8X_TIMELINE
                      , tl
#endif
        );
        if (w == kChPoll && lane == 0) run_exit(words, run, G);
    } else {
        chain_compute(sm, nst, w - kChSync, lane);
    }
}

// ================================================================================================ k_step (any class)
struct StepStage {
    RgJobs R;   // the stage's linears: activations and K plan (R.j0), tensor metadata (R.jt), outputs, swiglu
    int nvwg;   // virtual workgroups of the stage (row-group assignments), R.wgbase[kRgMaxJobs]
    int gc;     // row groups a workgroup streams together (teams of waves; 1 with K-chunks)
};

// 4 consecutive floats per lane, agent-coherent (the previous stage wrote them in this launch): one 16-byte load
__device__ __forceinline__ f32x4 load4_coherent(const float *p, int lane, uint32_t bytes) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(buffer_rsrc(p, bytes), 16u * (uint32_t)lane, 0, kBufSC1);
    const uint32_t a = v[0], b = v[1], c = v[2], d = v[3];
    f32x4 r;
    r.x = __uint_as_float(a); r.y = __uint_as_float(b); r.z = __uint_as_float(c); r.w = __uint_as_float(d);
    return r;
}

// One virtual workgroup v of stage *sp: the body of k_gemv_rg<CM, nks > 1, 1, gc > 1, multi> with one column, the
// variant chosen from the stage's plan at run time, inputs read and outputs written agent-coherently.
template <int CM>
__device__ __forceinline__ void step_stage(kptr<const StepStage> sp, int v, RgSmem<1> &sm, int tid) {
    constexpr int WAVES = rg_waves(1), RQ = kRgMaxBlocks / WAVES;
    // this workgroup's job, its index among the job's workgroups and their count
    const int jb = (v >= sp->R.wgbase[1]) + (v >= sp->R.wgbase[2]) + (v >= sp->R.wgbase[3]);
    const int wb = pick(jb, sp->R.wgbase[0], sp->R.wgbase[1], sp->R.wgbase[2], sp->R.wgbase[3]);
    const int wgl = v - wb;
    const int nwg = pick(jb, sp->R.wgbase[1], sp->R.wgbase[2], sp->R.wgbase[3], sp->R.wgbase[4]) - wb;
    GemvJob JL = *(const GemvJob *)pick(jb, sp->R.jt[0], sp->R.jt[1], sp->R.jt[2], sp->R.jt[3]);
    JL.x = sp->R.j0.x; JL.ldx = sp->R.j0.ldx; JL.nks = sp->R.j0.nks; JL.kchunk = sp->R.j0.kchunk;
    JL.y = pick(jb, sp->R.y[0], sp->R.y[1], sp->R.y[2], sp->R.y[3]);
    const GemvJob &J = JL;
    const int glu = sp->R.glu;
    const int nks = J.nks;
    const int gc = nks > 1 ? 1 : sp->gc;
    const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    TaskCtx<1, P8X_ACT_Q8_128> c;
    c.J = &J;
    c.hs = lane >> 5; c.j = lane & 31;
    c.bankbytes = (uint32_t)(c.j << 2) * 0x01010101u;
    c.xlane = c.hs * 64;
    const int ks = wgl % nks, nbk = min(J.kchunk, J.nb - ks * J.kchunk);
    c.b0 = ks * J.kchunk; c.nbl = nbk;
    const int wpg = WAVES / gc, team = w / wpg, wk = w % wpg;   // waves beyond gc teams stay idle
    const int per = nbk / wpg, rem = nbk % wpg;
    int b0 = c.b0 + wk * per + min(wk, rem), b1 = b0 + per + (wk < rem ? 1 : 0);   // the wave's K range
    if (team >= gc) b1 = b0;
    // the wave's activation blocks (agent-coherent loads), then, for a one-class chain, its first run of tiles
    BlockLane in[RQ];
    const uint32_t xbytes = 4u * (uint32_t)J.K;
#pragma unroll
    for (int i = 0; i < RQ; ++i) {
        const int it = w + i * WAVES, bk = c.b0 + it % nbk;
        if (it < nbk) {
            in[i].x = load4_coherent(J.x + 256 * bk, lane, xbytes - 1024u * (uint32_t)bk);
            in[i].c = as_global(reinterpret_cast<const f32x4 *>(J.ic + 256 * bk))[lane];
        } else {
            in[i] = BlockLane{};
        }
    }
    constexpr int PC = CM == kCmC3 ? 3 : CM == kCmC6 ? 6 : 0;
    GemvRun<1, P8X_ACT_Q8_128, false, PC ? PC : 3, gemv_nbuf(1, PC ? PC : 3), true> pre;
    const int gstep = nwg / nks;
    const int gfirst = wgl / nks + min(team, gc - 1) * gstep;
    const bool pre_on = PC != 0 && team < gc && gfirst < J.ng && b0 < b1;
    __asm__ volatile("" ::: "memory");
    if constexpr (PC != 0) {   // on every path, as in k_gemv_rg
        c.g = min(gfirst, J.ng - 1);
        const int bb = pre_on ? b0 : min(b0, J.nb - 1);
        pre.begin(c, bb, pre_on ? b1 : bb + 1);
    }
    __asm__ volatile("" ::: "memory");
    if (nbk <= WAVES) rg_quantize<1, 1>(nbk, sm, in, w, lane);
    else if (nbk <= 2 * WAVES) rg_quantize<2, 1>(nbk, sm, in, w, lane);
    else rg_quantize<4, 1>(nbk, sm, in, w, lane);
    __syncthreads();
    int set = 0;
    bool first = true;
    for (int g0 = wgl / nks; g0 < J.ng; g0 += gstep * gc, set ^= 1) {
        const int g = g0 + min(team, gc - 1) * gstep;   // this wave's row group
        const bool lead = wk == 0 && team < gc && g < J.ng;
        c.g = g;
        int ro = 0;
        if (lead && lane < 32) ro = as_global(J.prmd)[32 * g + lane];
        float yacc[1] = {0.f};
        int bstart = b0;
        if (PC != 0 && first && pre_on) bstart = pre.finish(c, sm, yacc);
        first = false;
        for (int b = bstart; b < (g < J.ng ? b1 : b0);) {
            if constexpr (PC != 0) {   // one class: no tile word to read
                b = gemv_run<1, P8X_ACT_Q8_128, false, PC, gemv_nbuf(1, PC), true>(c, sm, b, b1, yacc);
                continue;
            }
            const uint32_t mt = as_const(J.M)[(size_t)g * J.nb + b];
            switch (mt >> 29) {
                case 1: if constexpr ((CM >> 1) & 1) { b = gemv_run<1, P8X_ACT_Q8_128, false, 1, gemv_nbuf(1, 1), CM == (1 << 1)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                case 2: if constexpr ((CM >> 2) & 1) { b = gemv_run<1, P8X_ACT_Q8_128, false, 2, gemv_nbuf(1, 2), CM == (1 << 2)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                case 3: if constexpr ((CM >> 3) & 1) { b = gemv_run<1, P8X_ACT_Q8_128, false, 3, gemv_nbuf(1, 3), CM == (1 << 3)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                case 4: if constexpr ((CM >> 4) & 1) { b = gemv_run<1, P8X_ACT_Q8_128, false, 4, gemv_nbuf(1, 4), CM == (1 << 4)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                case 5: if constexpr ((CM >> 5) & 1) { b = gemv_run<1, P8X_ACT_Q8_128, false, 5, gemv_nbuf(1, 5), CM == (1 << 5)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                case 6: if constexpr ((CM >> 6) & 1) { b = gemv_run<1, P8X_ACT_Q8_128, false, 6, gemv_nbuf(1, 6), CM == (1 << 6)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                case 7: if constexpr ((CM >> 7) & 1) { b = gemv_run<1, P8X_ACT_Q8_128, false, 7, gemv_nbuf(1, 7), CM == (1 << 7)>(c, sm, b, b1, yacc); break; } [[fallthrough]];
                default: ++b; break;   // class 0: zero weights
            }
        }
        yacc[0] += __shfl_xor(yacc[0], 32);
        if (lane < 32) sm.red[set][w][0][lane] = yacc[0];
        __syncthreads();
        if (lead) {
            float vr = 0.f;
            if (lane < 32)
                for (int i = 0; i < wpg; ++i) vr += sm.red[set][w + i][0][lane];
            bool fin = lane < 32;   // lanes that finish their row here
            if (nks == 2) {   // two K-halves: each row's halves meet in its slot (pair_meet)
                int oi;
                float other;
                fin = fin && pair_meet(as_global_rw(J.wslot) + 32 * g + lane, ks, vr, oi, other);
                if (fin) vr = ks == 0 ? vr + other : other + vr;   // chunk 0 + chunk 1 either way
            } else if (nks > 2) {   // K-chunks: the last arrival sums them in chunk order
                const gptr<float> wpart = as_global_rw(J.wpart);
                const gptr<unsigned> wcnt = as_global_rw(J.wcnt);
                if (lane < 32) __hip_atomic_store(&wpart[(size_t)ks * J.rows + 32 * g + lane], vr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (arrive_after_stores(J.wcnt + g, lane) != (unsigned)(nks - 1)) continue;
                if (lane < 32) {
                    vr = 0.f;
                    for (int k = 0; k < nks; ++k)
                        vr += __hip_atomic_load(&wpart[(size_t)k * J.rows + 32 * g + lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                if (lane == 0) __hip_atomic_store(&wcnt[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            const int r = ro & 0x7FFF;
            float vo = vr;
            if (fin && (ro & 0x8000)) {
                float *xr = const_cast<float *>(J.x);
                for (int e = as_global(J.cp)[r]; e < as_global(J.cp)[r + 1]; ++e)
                    vo += as_global(J.cv)[e] * __hip_atomic_load(&xr[as_global(J.cc)[e]], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (glu) glu_meet(sp->R.glu_slot, sp->R.glu_out, jb, r, vo, fin);
            else if (fin) __hip_atomic_store(&as_global_rw(J.y)[r], vo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Grid barrier number `b` of run `run` (b = 1, 2, ... within the run): every wave's stores complete, one arrival per
// workgroup on its XCD's counter (workgroup i runs on XCD i % 8); the last arrival of an XCD arrives on the top
// counter, the last of those writes the barrier's number into every XCD's release word; thread 0 polls its XCD's
// release word. The counters only grow: an XCD counter gains nx per barrier (nx workgroups on that XCD), the top
// counter kXcds, so the targets follow from the number of barriers passed before this one, (run - 1) * per_run + b - 1
// (modulo 2^32). Bounded: a wait gives up after `spin` polls or when another has given up. Returns false when the
// launch must end.
__device__ __forceinline__ bool step_barrier(unsigned *words, unsigned spin, unsigned passed, unsigned tag, int *flag) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const int G = (int)gridDim.x, x = (int)blockIdx.x % kXcds, nx = (G - 1 - x) / kXcds + 1;
        int good = 1;
        if (add_agent(words + kSwXcd + 32 * x, 1u) == (passed + 1u) * (unsigned)nx - 1u &&
            add_agent(words + kSwTop, 1u) == (passed + 1u) * (unsigned)min(G, kXcds) - 1u)
            for (int k = 0; k < kXcds; ++k) st_agent(words + kSwRel + 32 * k, tag);
        for (unsigned n = 0; ld_agent(words + kSwRel + 32 * x) != tag; ++n) {
            if (n >= spin || ld_agent(words + kSwFail) != 0u) {
                st_agent(words + kSwFail, 1u);
                good = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        *flag = good;
    }
    __syncthreads();
    return *flag != 0;
}

template <int CM>
__global__ __launch_bounds__(64 * rg_waves(1)) __attribute__((amdgpu_waves_per_eu(rg_waves(1) / 4, rg_waves(1) / 4)))
void k_step(const StepStage *__restrict__ stages, int nst, unsigned *words, unsigned spin, const uint32_t *__restrict__ a2) {
    __shared__ RgSmem<1> sm;
    __shared__ int flag;
    __shared__ unsigned run_s;
    const int tid = threadIdx.x;
    if (tid == 0) run_s = ld_agent(words + kSwRuns) + 1u;
    // the table once for the whole chain (each stage's barrier after its quantization orders these writes
    // before the first lookup)
    build_coset_table<64 * rg_waves(1)>(sm.tab, a2, tid);
    __syncthreads();
    const unsigned run = run_s, per_run = (unsigned)(nst - 1);
    bool ok = true;
    for (int s = 0; s < nst; ++s) {
        const kptr<const StepStage> sp = as_const(stages) + s;
        const int nv = sp->nvwg;
        for (int v = blockIdx.x; v < nv; v += gridDim.x) {
            step_stage<CM>(sp, v, sm, tid);
            __syncthreads();   // the next virtual workgroup rewrites the activation buffer
        }
        // release tag: the barrier's number over all runs, never 0 (the words start at 0)
        if (s + 1 < nst && !step_barrier(words, spin, (run - 1u) * per_run + (unsigned)s, (run - 1u) * per_run + (unsigned)s + 1u, &flag)) {
            ok = false;
            break;
        }
    }
    (void)ok;
    if (tid == 0) run_exit(words, run, (int)gridDim.x);
}

template <int CM>
static int launch_step_t(const StepStage *stages, int nst, unsigned *words, unsigned spin, const uint32_t *a2, int grid, hipStream_t st) {
    void *args[] = {(void *)&stages, (void *)&nst, (void *)&words, (void *)&spin, (void *)&a2};
    return hip_check(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(&k_step<CM>), dim3(grid), dim3(64 * rg_waves(1)), args,
                                                0, st),
                     "k_step cooperative launch");
}

template <typename K>
static int occupancy_grid(K kern, int threads, int *grid, const char *what) {
    int per_cu = 0;
    const int rc = hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(kern), threads, 0), what);
    if (rc) return rc;
    if (per_cu < 1) return set_error(P8X_ERR_UNSUPPORTED, "%s: no workgroup fits a CU", what);
    *grid = num_cus();   // one workgroup per CU
    return P8X_OK;
}

}  // namespace p8x

using namespace p8x;

struct p8x_step {
    int nst = 0, cm = 0, grid = 0;
    bool chain = false;                  // k_chain (else k_step)
    StepStage *dstages = nullptr;        // k_step
    ChStage *dchain = nullptr;           // k_chain: stage records
    ChTileStage *dtiles = nullptr;       // and the compute waves' copies
    ChPlanRec *dplans = nullptr;         // each workgroup's share of each stage
    ChDelta *ddl = nullptr;              // clamp-delta entries per workgroup
    int *ddl_off = nullptr;
    std::vector<void *> pubs;            // published-output buffers
    unsigned *words = nullptr;           // kSyncWords device words
    bool broken = false;
    const uint32_t *a2 = nullptr;
    int device = 0;
    std::vector<const void *> keep;      // tensors and buffers the stages point to (identity only)
};

namespace {

// The k_chain plan of a chain, or a reason it does not apply (then k_step runs it).
struct ChainPlan {
    std::vector<ChStage> st;
    std::vector<ChTileStage> ts;
    std::vector<ChPlanRec> plans;                 // [workgroup][stage]
    std::vector<ChDelta> dl;                      // clamp-delta entries, workgroup-major
    std::vector<int> dl_off;                      // [workgroups + 1]
    std::vector<std::pair<int, int>> pub_jobs;   // (stage, job) whose output is published
    std::vector<size_t> pub_bytes;
};

// a tensor's row order and clamp-delta CSR, read back from the device (the step resolves delta entries per workgroup)
struct HostDelta {
    std::vector<int16_t> prm;
    std::vector<int> cp;
    std::vector<uint16_t> cc;
    std::vector<float> cv;
};

int host_delta(const p8x_tensor *t, HostDelta &h) {
    h.prm.resize(t->rows);
    h.cp.resize(t->rows + 1);
    h.cc.resize(std::max(1, t->nd));
    h.cv.resize(std::max(1, t->nd));
    int rc = hip_check(hipMemcpy(h.prm.data(), t->prm, 2 * (size_t)t->rows, hipMemcpyDeviceToHost), "p8x_step_create: prm");
    if (!rc) rc = hip_check(hipMemcpy(h.cp.data(), t->cp, 4 * (size_t)(t->rows + 1), hipMemcpyDeviceToHost), "p8x_step_create: delta");
    if (!rc && t->nd > 0) rc = hip_check(hipMemcpy(h.cc.data(), t->cc, 2 * (size_t)t->nd, hipMemcpyDeviceToHost), "p8x_step_create: delta");
    if (!rc && t->nd > 0) rc = hip_check(hipMemcpy(h.cv.data(), t->cv, 4 * (size_t)t->nd, hipMemcpyDeviceToHost), "p8x_step_create: delta");
    return rc;
}

const char *chain_plan(const p8x_step_stage *stages, int n, ChainPlan &P) {
    const int G = num_cus();
    if (n > kChMaxStages) return "more stages than the LDS stage table holds";
    if (G > 32767) return "too many workgroups";
    P.st.assign(n, ChStage{});
    P.ts.assign(n, ChTileStage{});
    P.plans.assign((size_t)G * n, ChPlanRec{});
    // producers of each buffer: (stage, job) for a plain output, (stage, -1) for a swiglu output
    struct Out { const void *p; int s, j; };
    std::vector<Out> outs;
    for (int s = 0; s < n; ++s) {
        const p8x_step_stage &S = stages[s];
        for (int i = 0; i < S.n; ++i) {
            const p8x_tensor *t = S.tensors[i];
            if (!(t->class_tiles[3] == t->nt && t->lin_words == 512u)) return "a tensor is not class 3 with its tiles in order";
        }
        if (S.glu_out) outs.push_back({S.glu_out, s, -1});
        else
            for (int i = 0; i < S.n; ++i) outs.push_back({S.y[i], s, i});
    }
    for (size_t a = 0; a < outs.size(); ++a)
        for (size_t b = a + 1; b < outs.size(); ++b)
            if (outs[a].p == outs[b].p) return "two outputs share a buffer";
    std::vector<int> consumed(outs.size(), 0);
    std::vector<int> src(n, -1);   // index into outs of each stage's input producer
    for (int s = 0; s < n; ++s) {
        for (size_t o = 0; o < outs.size(); ++o) {
            if (outs[o].p != (const void *)stages[s].x) continue;
            if (outs[o].s >= s) return "a stage reads an output of itself or of a later stage";
            src[s] = (int)o;
            consumed[o] = 1;
        }
    }
    // K plans: chunks of at most kChMaxBlk blocks; two when the row groups fill at most half the workgroups (not for a
    // swiglu stage: its consumers read gate and up halves, two parts already)
    std::vector<int> nks(n);
    for (int s = 0; s < n; ++s) {
        const p8x_step_stage &S = stages[s];
        const int nb = S.tensors[0]->nb;
        int U = 0;
        for (int i = 0; i < S.n; ++i) U += S.tensors[i]->ng;
        int k = (nb + kChMaxBlk - 1) / kChMaxBlk;
        if (k == 1 && 2 * U <= G / 2 && nb >= 16 && !S.glu_out) k = 2;
        const int kc = (nb + k - 1) / k;
        nks[s] = (nb + kc - 1) / kc;
        ChStage &C = P.st[s];
        C.nj = S.n; C.nks = nks[s]; C.kchunk = kc; C.nb = nb; C.K = S.tensors[0]->K;
        C.ic = S.tensors[0]->ic;
        int acc = 0;
        for (int i = 0; i < kRgMaxJobs; ++i) {
            if (i < S.n) acc += S.tensors[i]->ng;
            if (i < 3) C.ngo[i] = i + 1 < S.n ? acc : INT_MAX;
        }
        C.ngo[3] = U;
        // every compute wave's range within kChSlots units, and each workgroup's chunk within the LDS buffer
        for (int w = 0; w < G; ++w) {
            const ChPlan p = ch_plan(C.nks, C.kchunk, nb, U, w, G);
            if (p.nbk > kChMaxBlk || p.nbk < 1) return "a K-chunk does not fit the LDS activations";
            const int T = p.nr * p.nbk;
            if (T > kChMaxTiles) return "a workgroup's tiles of a stage exceed the LDS row-scale buffer";
            if (p.nr > kChPub * kChUnitsPerPub) return "a workgroup has more units in a stage than its publisher waves hold";
            ChPlanRec &R = P.plans[(size_t)w * n + s];
            R.nr = (int16_t)p.nr; R.kb0 = (int16_t)p.kb0; R.nbk = (int16_t)p.nbk; R.nact = (int16_t)p.nact;
            R.r = (int16_t)p.r; R.m = (int16_t)p.m; R.ks = (int16_t)p.ks; R.pad = 0;
            for (int c = 0; c < kChComp; ++c) {
                const int t0 = ch_t0(c, T), t1 = ch_t0(c + 1, T);
                if (t1 > t0 && (t1 - 1) / p.nbk - t0 / p.nbk >= kChSlots) return "a compute wave's tiles span too many units";
            }
        }
    }
    // outputs: plain one-chunk outputs are written by their producer; split or swiglu outputs only by the designated
    // readers of a later stage, so they must be read
    for (size_t o = 0; o < outs.size(); ++o) {
        const int s = outs[o].s;
        if ((nks[s] > 1 || outs[o].j < 0) && !consumed[o]) return "a split or swiglu output that no later stage reads";
    }
    // published buffers
    std::vector<std::vector<int>> pub_of(n, std::vector<int>(kRgMaxJobs, -1));
    for (size_t o = 0; o < outs.size(); ++o) {
        if (!consumed[o]) continue;
        const int s = outs[o].s;
        for (int i = 0; i < stages[s].n; ++i) {
            if (outs[o].j >= 0 && outs[o].j != i) continue;
            if (pub_of[s][i] >= 0) continue;
            pub_of[s][i] = (int)P.pub_jobs.size();
            P.pub_jobs.push_back({s, i});
            P.pub_bytes.push_back((size_t)nks[s] * stages[s].tensors[i]->rows * 8);
        }
    }
    for (int s = 0; s < n; ++s) {
        const p8x_step_stage &S = stages[s];
        ChStage &C = P.st[s];
        for (int i = 0; i < S.n; ++i) {
            const p8x_tensor *t = S.tensors[i];
            ChJob &J = C.job[i];
            J.D = t->D; J.Sg = t->Sg; J.prmd = t->prmd; J.cp = t->cp; J.cc = t->cc; J.cv = t->cv;
            J.rows = t->rows;
            J.dbytes = (unsigned)(t->nt * kChTileBytes);
            J.y = (!S.glu_out && nks[s] == 1) ? S.y[i] : nullptr;
            J.pub = nullptr;   // device address filled in by the caller
            ChTileJob &TJ = P.ts[s].job[i];
            TJ.D = t->D; TJ.dbytes = J.dbytes;
        }
        P.ts[s].nb = C.nb;
        for (int i = 0; i < kRgMaxJobs; ++i) P.ts[s].ngo[i] = C.ngo[i];
        C.in.x = S.x;
        if (src[s] >= 0) {
            const Out &o = outs[src[s]];
            if (nks[o.s] * (o.j < 0 ? 2 : 1) > 2) return "an input published in more than two parts (K-chunks x swiglu halves)";
            C.in.parts = nks[o.s];
            C.in.glu = o.j < 0;
            C.in.out = (o.j < 0 || nks[o.s] > 1) ? const_cast<float *>(S.x) : nullptr;
        }
    }
    (void)pub_of;
    return nullptr;
}

// each workgroup's clamp-delta entries (stage order; within a stage by unit, row and the row's entry order): the
// entries of its units' rows whose column lies in its K-chunk
int chain_deltas(const p8x_step_stage *stages, int n, ChainPlan &P, const char **why) {
    const int G = num_cus();
    std::vector<std::pair<const p8x_tensor *, HostDelta>> cache;
    auto host_of = [&](const p8x_tensor *t, const HostDelta **out) -> int {
        for (auto &c : cache)
            if (c.first == t) { *out = &c.second; return (int)P8X_OK; }
        cache.emplace_back(t, HostDelta{});
        *out = &cache.back().second;
        return host_delta(t, cache.back().second);
    };
    P.dl.clear();
    P.dl_off.assign(G + 1, 0);
    for (int w = 0; w < G; ++w) {
        P.dl_off[w] = (int)P.dl.size();
        for (int s = 0; s < n; ++s) {
            const ChPlanRec &R = P.plans[(size_t)w * n + s];
            const ChStage &C = P.st[s];
            for (int k = 0; k < R.nr; ++k) {
                const int u = R.r + k * R.m;
                const int jb = (u >= C.ngo[0]) + (u >= C.ngo[1]) + (u >= C.ngo[2]);
                const int g = u - (jb == 0 ? 0 : C.ngo[jb - 1]);
                const p8x_tensor *t = stages[s].tensors[jb];
                if (t->nd == 0) continue;
                const HostDelta *h = nullptr;
                const int rc = host_of(t, &h);
                if (rc) return rc;
                for (int j = 0; j < 32; ++j) {
                    const int ro = h->prm[32 * g + j];
                    for (int e = h->cp[ro]; e < h->cp[ro + 1]; ++e) {
                        const int lcol = (int)h->cc[e] - 256 * R.kb0;
                        if (lcol < 0 || lcol >= 256 * R.nbk) continue;
                        ChDelta d;
                        d.skj = (uint32_t)s | ((uint32_t)k << 16) | ((uint32_t)j << 24);
                        d.lcol = (uint32_t)lcol;
                        d.val = h->cv[e];
                        d.pad = 0;
                        P.dl.push_back(d);
                    }
                }
            }
        }
        if ((int)P.dl.size() - P.dl_off[w] > kChMaxDelta) {
            *why = "a workgroup has more clamp-delta entries than its LDS list holds";
            return P8X_OK;
        }
    }
    P.dl_off[G] = (int)P.dl.size();
    if (P.dl.empty()) P.dl.push_back(ChDelta{});   // a valid device array
    return P8X_OK;
}

}  // namespace

extern "C" {

int p8x_step_create(const p8x_step_stage *stages, int n, p8x_step **out) {
    if (!stages || n < 1 || !out) return set_error(P8X_ERR_ARG, "p8x_step_create: bad arguments");
    *out = nullptr;
    std::vector<StepStage> hs(n);
    size_t hist[8] = {0};
    bool in_order = true;
    const p8x_tensor *t0 = nullptr;
    for (int s = 0; s < n; ++s) {
        const p8x_step_stage &st = stages[s];
        if (st.n < 1 || st.n > kRgMaxJobs) return set_error(P8X_ERR_ARG, "p8x_step_create: stage %d has %d tensors (1..%d)", s, st.n, kRgMaxJobs);
        int rc = check_shared_input(st.tensors, st.n, st.x, st.x ? st.tensors[0]->K : 0, "p8x_step_create");
        if (rc) return rc;
        if (!t0) t0 = st.tensors[0];
        for (int i = 0; i < st.n; ++i) {
            const p8x_tensor *t = st.tensors[i];
            if (memcmp(t->a2_host, t0->a2_host, sizeof t->a2_host))
                return set_error(P8X_ERR_UNSUPPORTED, "p8x_step_create: stage %d tensor %d has a different codebook", s, i);
            for (int c = 0; c < 8; ++c) hist[c] += t->class_tiles[c];
            in_order = in_order && t->lin_words != 0;
        }
        const bool glu = st.glu_out != nullptr;
        if (glu && (st.n != 2 || st.tensors[0]->rows != st.tensors[1]->rows))
            return set_error(P8X_ERR_ARG, "p8x_step_create: stage %d: swiglu needs a gate and an up tensor of the same rows", s);
        size_t ldy[kRgMaxJobs];
        for (int i = 0; i < st.n; ++i) {
            if (!glu && !st.y[i]) return set_error(P8X_ERR_ARG, "p8x_step_create: stage %d output %d is null", s, i);
            ldy[i] = (size_t)st.tensors[i]->rows;
        }
        int cm = 0, ng = 0;
        rc = plan_gemv_multi(st.tensors, st.n, st.x, (size_t)st.tensors[0]->K, glu ? nullptr : st.y, glu ? nullptr : ldy,
                             glu ? st.glu_out : nullptr, hs[s].R, cm, ng);
        if (rc) return rc;
        hs[s].nvwg = hs[s].R.wgbase[kRgMaxJobs];
        const int per = (ng + num_cus() - 1) / num_cus();
        hs[s].gc = std::min(per, 4);
    }
    p8x_step *sp = new p8x_step();
    sp->nst = n;
    sp->cm = class_set(hist, in_order) == kCmC3 ? kCmC3 : kCmAll;
    sp->a2 = t0->a2;
    (void)hipGetDevice(&sp->device);
    for (int s = 0; s < n; ++s) {
        for (int i = 0; i < stages[s].n; ++i) sp->keep.push_back(stages[s].tensors[i]);
    }
    int rc = P8X_OK;
    ChainPlan P;
    const char *why = chain_plan(stages, n, P);
    if (!why) rc = chain_deltas(stages, n, P, &why);
    if (!rc && !why) {
        sp->chain = true;
        rc = occupancy_grid(&k_chain, 64 * kChWaves, &sp->grid, "k_chain occupancy");
        for (size_t i = 0; !rc && i < P.pub_jobs.size(); ++i) {
            void *b = nullptr;
            if (hipMalloc(&b, P.pub_bytes[i]) != hipSuccess) rc = set_error(P8X_ERR_NOMEM, "p8x_step_create: hipMalloc published output");
            else {
                sp->pubs.push_back(b);
                rc = hip_check(hipMemset(b, 0, P.pub_bytes[i]), "p8x_step_create: published output");
                P.st[P.pub_jobs[i].first].job[P.pub_jobs[i].second].pub = (u64 *)b;
            }
        }
        // each stage's input: the producer's published vectors
        for (int s = 0; !rc && s < n; ++s) {
            ChStage &C = P.st[s];
            if (C.in.parts == 0) continue;
            for (int t = 0; t < s; ++t) {
                const p8x_step_stage &S = stages[t];
                if (S.glu_out && S.glu_out == stages[s].x) { C.in.pub[0] = P.st[t].job[0].pub; C.in.pub[1] = P.st[t].job[1].pub; }
                if (!S.glu_out)
                    for (int i = 0; i < S.n; ++i)
                        if (S.y[i] == stages[s].x) C.in.pub[0] = C.in.pub[1] = P.st[t].job[i].pub;
            }
            if (!C.in.pub[0]) rc = set_error(P8X_ERR_HIP, "p8x_step_create: stage %d: producer not found", s);
        }
        if (!rc && hipMalloc((void **)&sp->dchain, sizeof(ChStage) * n) != hipSuccess) rc = set_error(P8X_ERR_NOMEM, "p8x_step_create: hipMalloc stages");
        if (!rc && hipMalloc((void **)&sp->dtiles, sizeof(ChTileStage) * n) != hipSuccess) rc = set_error(P8X_ERR_NOMEM, "p8x_step_create: hipMalloc stages");
        if (!rc && hipMalloc((void **)&sp->dplans, sizeof(ChPlanRec) * P.plans.size()) != hipSuccess) rc = set_error(P8X_ERR_NOMEM, "p8x_step_create: hipMalloc plans");
        if (!rc && hipMalloc((void **)&sp->ddl, sizeof(ChDelta) * P.dl.size()) != hipSuccess) rc = set_error(P8X_ERR_NOMEM, "p8x_step_create: hipMalloc delta");
        if (!rc && hipMalloc((void **)&sp->ddl_off, sizeof(int) * P.dl_off.size()) != hipSuccess) rc = set_error(P8X_ERR_NOMEM, "p8x_step_create: hipMalloc delta");
        if (!rc) rc = hip_check(hipMemcpy(sp->dchain, P.st.data(), sizeof(ChStage) * n, hipMemcpyHostToDevice), "p8x_step_create: stages");
        if (!rc) rc = hip_check(hipMemcpy(sp->dtiles, P.ts.data(), sizeof(ChTileStage) * n, hipMemcpyHostToDevice), "p8x_step_create: stages");
        if (!rc) rc = hip_check(hipMemcpy(sp->dplans, P.plans.data(), sizeof(ChPlanRec) * P.plans.size(), hipMemcpyHostToDevice), "p8x_step_create: plans");
        if (!rc) rc = hip_check(hipMemcpy(sp->ddl, P.dl.data(), sizeof(ChDelta) * P.dl.size(), hipMemcpyHostToDevice), "p8x_step_create: delta");
        if (!rc) rc = hip_check(hipMemcpy(sp->ddl_off, P.dl_off.data(), sizeof(int) * P.dl_off.size(), hipMemcpyHostToDevice), "p8x_step_create: delta");
    } else if (!rc) {
        rc = sp->cm == kCmC3 ? occupancy_grid(&k_step<kCmC3>, 64 * rg_waves(1), &sp->grid, "k_step occupancy")
                             : occupancy_grid(&k_step<kCmAll>, 64 * rg_waves(1), &sp->grid, "k_step occupancy");
        if (!rc && hipMalloc((void **)&sp->dstages, sizeof(StepStage) * n) != hipSuccess) rc = set_error(P8X_ERR_NOMEM, "p8x_step_create: hipMalloc stages");
        if (!rc) rc = hip_check(hipMemcpy(sp->dstages, hs.data(), sizeof(StepStage) * n, hipMemcpyHostToDevice), "p8x_step_create: stages");
    }
    if (!rc && hipMalloc((void **)&sp->words, kSyncWords * sizeof(unsigned)) != hipSuccess) rc = set_error(P8X_ERR_NOMEM, "p8x_step_create: hipMalloc sync");
    if (!rc) rc = hip_check(hipMemset(sp->words, 0, kSyncWords * sizeof(unsigned)), "p8x_step_create: sync");
    if (!rc) rc = hip_check(hipDeviceSynchronize(), "p8x_step_create");
    if (rc) { p8x_step_release(sp); return rc; }
    *out = sp;
    return P8X_OK;
}

int p8x_step_run(p8x_step *sp, void *stream) {
    if (!sp) return set_error(P8X_ERR_ARG, "p8x_step_run: null step");
    if (sp->broken) return set_error(P8X_ERR_HIP, "p8x_step_run: a previous launch gave up waiting (see p8x_step_check)");
    const unsigned spin = 1u << 20;
    hipStream_t st = (hipStream_t)stream;
    if (sp->chain) {
        const ChStage *a0 = sp->dchain;
        const ChTileStage *a1 = sp->dtiles;
        const ChPlanRec *a3 = sp->dplans;
        const ChDelta *a4 = sp->ddl;
        const int *a5 = sp->ddl_off;
        int nst = sp->nst;
        unsigned *words = sp->words;
        unsigned sp_ = spin;
        const uint32_t *a2 = sp->a2;
#ifdef P8X_TIMELINE
        u64 *tl = timeline_buf();
        void *args[] = {(void *)&a0, (void *)&a1, (void *)&a3, (void *)&a4, (void *)&a5, (void *)&nst, (void *)&words, (void *)&sp_,
                        (void *)&a2, (void *)&tl};
#else
        void *args[] = {(void *)&a0, (void *)&a1, (void *)&a3, (void *)&a4, (void *)&a5, (void *)&nst, (void *)&words, (void *)&sp_,
                        (void *)&a2};
#endif
        return hip_check(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(&k_chain), dim3(sp->grid), dim3(64 * kChWaves), args, 0, st),
                         "k_chain cooperative launch");
    }
    return sp->cm == kCmC3 ? launch_step_t<kCmC3>(sp->dstages, sp->nst, sp->words, spin, sp->a2, sp->grid, st)
                           : launch_step_t<kCmAll>(sp->dstages, sp->nst, sp->words, spin, sp->a2, sp->grid, st);
}

int p8x_step_check(p8x_step *sp) {
    if (!sp) return set_error(P8X_ERR_ARG, "p8x_step_check: null step");
    int rc = hip_check(hipDeviceSynchronize(), "p8x_step_check");
    if (rc) return rc;
    unsigned w[3] = {0, 0, 0};
    rc = hip_check(hipMemcpy(w, sp->words, sizeof w, hipMemcpyDeviceToHost), "p8x_step_check: read");
    if (rc) return rc;
    if (w[kSwFail]) {
        sp->broken = true;
        return set_error(P8X_ERR_HIP, "p8x_step: a wait gave up (workgroups not co-resident?)");
    }
    if (w[kSwExit] != 0u) {
        sp->broken = true;
        return set_error(P8X_ERR_HIP, "p8x_step: %u workgroups of the last run did not finish", w[kSwExit]);
    }
    return P8X_OK;
}

#ifdef P8X_TIMELINE
// timeline build only: the row-group kernel's records (first n bytes) and their count; reset sets the count to 0
// (call it before capturing launches: it allocates the buffer on first use). The chain kernel writes its per-stage
// records at [stage][workgroup][8] from the buffer's start.
int p8x_timeline_read(void *host, size_t n, unsigned *count) {
    if (!timeline_buf()) return set_error(P8X_ERR_NOMEM, "p8x_timeline_read: no buffer");
    int rc = hip_check(hipMemcpy(host, timeline_buf(), n, hipMemcpyDeviceToHost), "p8x_timeline_read");
    if (!rc) rc = hip_check(hipMemcpy(count, timeline_buf() + (size_t)kTimelineRecords * 8, 4, hipMemcpyDeviceToHost), "p8x_timeline_read");
    return rc;
}
int p8x_timeline_reset(void) {
    if (!timeline_buf()) return set_error(P8X_ERR_NOMEM, "p8x_timeline_reset: no buffer");
    return hip_check(hipMemset(timeline_buf() + (size_t)kTimelineRecords * 8, 0, 8), "p8x_timeline_reset");
}
#endif

int p8x_step_info(const p8x_step *sp, int *grid, int *stages, int *class_set_) {
    if (!sp) return set_error(P8X_ERR_ARG, "p8x_step_info: null step");
    if (grid) *grid = sp->grid;
    if (stages) *stages = sp->nst;
    if (class_set_) *class_set_ = sp->cm | (sp->chain ? 0x100 : 0);
    return P8X_OK;
}

void p8x_step_release(p8x_step *sp) {
    if (!sp) return;
    (void)hipDeviceSynchronize();
    if (sp->dstages) (void)hipFree(sp->dstages);
    if (sp->dchain) (void)hipFree(sp->dchain);
    if (sp->dtiles) (void)hipFree(sp->dtiles);
    if (sp->dplans) (void)hipFree(sp->dplans);
    if (sp->ddl) (void)hipFree(sp->ddl);
    if (sp->ddl_off) (void)hipFree(sp->ddl_off);
    for (void *b : sp->pubs) (void)hipFree(b);
    if (sp->words) (void)hipFree(sp->words);
    delete sp;
}

}  // extern "C"
