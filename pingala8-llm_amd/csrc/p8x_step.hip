// p8x_step.hip -- a batch-1 decode step's chain of linears in one persistent launch.
//
// The reference launches one kernel per MUL_MAT node (CPU.patch:2615-2631, :4466-4521), so a step of L layers runs
// 4 L + 1 dependent launches (q/k/v, o, gate/up, down, then the head), each paying the launch and the kernel-boundary
// cache work, and each rebuilding the 64 KB coset table in every workgroup. Here one cooperative launch (k_step, one
// workgroup per CU) walks the whole chain with the table built once per workgroup: each stage runs the row-group GEMV
// body of k_gemv_rg over the stage's virtual workgroups, then a grid barrier orders it before the next stage.
//
// The barrier: per-XCD arrival counters, one counter above them, and a release word per XCD (workgroup i runs on XCD
// i % 8, so each counter line is shared by the workgroups of one XCD only). Its targets derive from a device-side run
// counter, so a launch replays from a HIP graph unchanged. While thread 0 waits for the release, another wave brings
// the next stage's records into the scalar cache (the stage body reads them through dependent scalar loads).
//
// Cross-workgroup hand-off rules: a stage's outputs are agent-scope stores (sc1: written through the XCD's L2 to the
// coherence point), every wave waits vmcnt(0) before its workgroup's arrival, and the next stage's inputs are
// agent-scope loads (sc1) issued after the release was observed. Cache-wide release / acquire (buffer_wbl2 /
// buffer_inv) would allow plain accesses but cost tens of microseconds per barrier on this part, so each access
// carries its own scope instead.
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

// ================================================================================================ k_step (any class)
constexpr int kBufSC1 = 16;   // buffer-load cache policy: sc1 (agent-coherent, served from the coherence point)

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
__device__ __forceinline__ void step_stage(kptr<const StepStage> sp, int v, RgSmem<1> &sm, int tid
#ifdef P8X_TIMELINE
                                           , u64 *rec
#endif
) {
    constexpr int WAVES = rg_waves(1), RQ = kRgMaxBlocks / WAVES;
    // this workgroup's job, its index among the job's workgroups and their count
    const int jb = (v >= sp->R.wgbase[1]) + (v >= sp->R.wgbase[2]) + (v >= sp->R.wgbase[3]);
    const int wb = pick(jb, sp->R.wgbase[0], sp->R.wgbase[1], sp->R.wgbase[2], sp->R.wgbase[3]);
    const int wgl = v - wb;
    const int nwg = pick(jb, sp->R.wgbase[1], sp->R.wgbase[2], sp->R.wgbase[3], sp->R.wgbase[4]) - wb;
    GemvJob JL = *(const GemvJob *)pick(jb, sp->R.jt[0], sp->R.jt[1], sp->R.jt[2], sp->R.jt[3]);
    JL.x = sp->R.j0.x; JL.ldx = sp->R.j0.ldx; JL.nks = sp->R.j0.nks; JL.kchunk = sp->R.j0.kchunk;
    JL.ic = sp->R.j0.ic; JL.nb = sp->R.j0.nb;   // shared by the stage's jobs (checked on the host): no tensor record wait
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
#ifdef P8X_TIMELINE
    // timeline build: thread 0 waits for its activation loads here and records when they are in (rec[6] bits 16..31)
    if (rec && tid == 0) {
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        rec[6] |= min(__builtin_amdgcn_s_memrealtime() - rec[0], (u64)0xFFFF) << 16;
    }
#endif
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
#ifdef P8X_TIMELINE
    if (rec && tid == 0) rec[6] |= min(__builtin_amdgcn_s_memrealtime() - rec[0], (u64)0xFFFF) << 32;   // prefetch issued
#endif
    if (nbk <= WAVES) rg_quantize<1, 1>(nbk, sm, in, w, lane);
    else if (nbk <= 2 * WAVES) rg_quantize<2, 1>(nbk, sm, in, w, lane);
    else rg_quantize<4, 1>(nbk, sm, in, w, lane);
#ifdef P8X_TIMELINE
    // rec[7]: 16-bit tick counts of thread 0: its quantization done (from the stage start), then from the input in LDS
    // its first round's tiles done, the partial rows exchanged, the round's epilogue done
    u64 tq = 0;
    if (rec && tid == 0) tq = __builtin_amdgcn_s_memrealtime();
#endif
    __syncthreads();
#ifdef P8X_TIMELINE
    u64 tin = 0;
    if (rec && tid == 0) {
        tin = __builtin_amdgcn_s_memrealtime();
        rec[1] = tin;
        rec[7] = min(tq - rec[0], (u64)0xFFFF);
    }
    bool round0 = true;
#endif
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
#ifdef P8X_TIMELINE
        if (rec && round0 && tid == 0) rec[7] |= min(__builtin_amdgcn_s_memrealtime() - tin, (u64)0xFFFF) << 16;
#endif
        if (lane < 32) sm.red[set][w][0][lane] = yacc[0];
        __syncthreads();
#ifdef P8X_TIMELINE
        if (rec && round0 && tid == 0) rec[7] |= min(__builtin_amdgcn_s_memrealtime() - tin, (u64)0xFFFF) << 32;
#endif
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
#ifdef P8X_TIMELINE
        if (rec && round0 && tid == 0) rec[7] |= min(__builtin_amdgcn_s_memrealtime() - tin, (u64)0xFFFF) << 48;
        round0 = false;
#endif
    }
}

// Grid barrier number `b` of run `run` (b = 1, 2, ... within the run): every wave's stores complete, one arrival per
// workgroup on its XCD's counter (workgroup i runs on XCD i % 8); the last arrival of an XCD arrives on the top
// counter, the last of those writes the barrier's number into every XCD's release word; thread 0 polls its XCD's
// release word. The counters only grow: an XCD counter gains nx per barrier (nx workgroups on that XCD), the top
// counter kXcds, so the targets follow from the number of barriers passed before this one, (run - 1) * per_run + b - 1
// (modulo 2^32). Bounded: a wait gives up after `spin` polls or when another has given up. Returns false when the
// launch must end.
// The next stage's record and its jobs' tensor records brought into the scalar cache while the barrier completes
// (waves other than the one that arrives and polls): the stage body reads them through dependent scalar loads.
__device__ __forceinline__ void step_touch(kptr<const StepStage> sp) {
    const kptr<const unsigned> w = (kptr<const unsigned>)sp;
#pragma unroll
    for (unsigned o = 0; o < sizeof(StepStage) / 4; o += 16) {
        const unsigned v = w[o];
        __asm__ volatile("" ::"s"(v));
    }
    const int nj = sp->R.njobs;
    for (int j = 0; j < nj; ++j) {
        const kptr<const unsigned> jw = (kptr<const unsigned>)pick(j, sp->R.jt[0], sp->R.jt[1], sp->R.jt[2], sp->R.jt[3]);
#pragma unroll
        for (unsigned o = 0; o < sizeof(GemvJob) / 4; o += 16) {
            const unsigned v = jw[o];
            __asm__ volatile("" ::"s"(v));
        }
    }
}

__device__ __forceinline__ bool step_barrier(unsigned *words, unsigned spin, unsigned passed, unsigned tag, int *flag,
                                             kptr<const StepStage> next
#ifdef P8X_TIMELINE
                                             , u64 *rec
#endif
) {
#ifdef P8X_TIMELINE
    if (threadIdx.x == 0) rec[2] = __builtin_amdgcn_s_memrealtime();
#endif
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (next && threadIdx.x >= 64 && threadIdx.x < 128) step_touch(next);
    if (threadIdx.x == 0) {
#ifdef P8X_TIMELINE
        rec[3] = __builtin_amdgcn_s_memrealtime();
#endif
        const int G = (int)gridDim.x, x = (int)blockIdx.x % kXcds, nx = (G - 1 - x) / kXcds + 1;
        int good = 1;
        if (add_agent(words + kSwXcd + 32 * x, 1u) == (passed + 1u) * (unsigned)nx - 1u &&
            add_agent(words + kSwTop, 1u) == (passed + 1u) * (unsigned)min(G, kXcds) - 1u)
            for (int k = 0; k < kXcds; ++k) st_agent(words + kSwRel + 32 * k, tag);
#ifdef P8X_TIMELINE
        rec[4] = __builtin_amdgcn_s_memrealtime();
#endif
        for (unsigned n = 0; ld_agent(words + kSwRel + 32 * x) != tag; ++n) {
            if (n >= spin || ld_agent(words + kSwFail) != 0u) {
                st_agent(words + kSwFail, 1u);
                good = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        *flag = good;
#ifdef P8X_TIMELINE
        rec[5] = __builtin_amdgcn_s_memrealtime();
#endif
    }
    __syncthreads();
    return *flag != 0;
}

template <int CM>
__global__ __launch_bounds__(64 * rg_waves(1)) __attribute__((amdgpu_waves_per_eu(rg_waves(1) / 4, rg_waves(1) / 4)))
void k_step(const StepStage *__restrict__ stages, int nst, unsigned *words, unsigned spin, const uint32_t *__restrict__ a2
#ifdef P8X_TIMELINE
            , u64 *tl
#endif
) {
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
#ifdef P8X_TIMELINE
        // timeline build: thread 0 records per stage: its start, the first virtual workgroup's input in LDS, the end
        // of its virtual workgroups, its stores complete, its arrival done, the release seen, and the count of its
        // virtual workgroups
        u64 *rec = tl + ((size_t)s * gridDim.x + blockIdx.x) * 8;
        if (tid == 0) {
            rec[0] = __builtin_amdgcn_s_memrealtime();
            rec[6] = (u64)((nv - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x);
        }
#endif
        for (int v = blockIdx.x; v < nv; v += gridDim.x) {
            step_stage<CM>(sp, v, sm, tid
#ifdef P8X_TIMELINE
                           , v == (int)blockIdx.x ? rec : nullptr
#endif
            );
            __syncthreads();   // the next virtual workgroup rewrites the activation buffer
        }
        if (s + 1 == nst) break;
        // release tag: the barrier's number over all runs, never 0 (the words start at 0)
        const unsigned passed = (run - 1u) * per_run + (unsigned)s;
        ok = step_barrier(words, spin, passed, passed + 1u, &flag, sp + 1
#ifdef P8X_TIMELINE
                          , rec
#endif
        );
        if (!ok) break;
    }
    (void)ok;
    if (tid == 0) run_exit(words, run, (int)gridDim.x);
}

template <int CM>
static int launch_step_t(const StepStage *stages, int nst, unsigned *words, unsigned spin, const uint32_t *a2, int grid, hipStream_t st) {
#ifdef P8X_TIMELINE
    u64 *tl = timeline_buf();
    void *args[] = {(void *)&stages, (void *)&nst, (void *)&words, (void *)&spin, (void *)&a2, (void *)&tl};
#else
    void *args[] = {(void *)&stages, (void *)&nst, (void *)&words, (void *)&spin, (void *)&a2};
#endif
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
    StepStage *dstages = nullptr;        // stage records
    unsigned *words = nullptr;           // kSyncWords device words
    bool broken = false;
    const uint32_t *a2 = nullptr;
    int device = 0;
    std::vector<const void *> keep;      // tensors and buffers the stages point to (identity only)
    int act = P8X_ACT_Q8_128;            // block_q8_1 / x16: the stages run as their per-node launches
    std::vector<p8x_step_stage> host;    // the stages of that form
};

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
    int rc = sp->cm == kCmC3 ? occupancy_grid(&k_step<kCmC3>, 64 * rg_waves(1), &sp->grid, "k_step occupancy")
                             : occupancy_grid(&k_step<kCmAll>, 64 * rg_waves(1), &sp->grid, "k_step occupancy");
    if (!rc && hipMalloc((void **)&sp->dstages, sizeof(StepStage) * n) != hipSuccess) rc = set_error(P8X_ERR_NOMEM, "p8x_step_create: hipMalloc stages");
    if (!rc) rc = hip_check(hipMemcpy(sp->dstages, hs.data(), sizeof(StepStage) * n, hipMemcpyHostToDevice), "p8x_step_create: stages");
    if (!rc && hipMalloc((void **)&sp->words, kSyncWords * sizeof(unsigned)) != hipSuccess) rc = set_error(P8X_ERR_NOMEM, "p8x_step_create: hipMalloc sync");
    if (!rc) rc = hip_check(hipMemset(sp->words, 0, kSyncWords * sizeof(unsigned)), "p8x_step_create: sync");
    if (!rc) rc = hip_check(hipDeviceSynchronize(), "p8x_step_create");
    if (rc) { p8x_step_release(sp); return rc; }
    *out = sp;
    return P8X_OK;
}

// block_q8_1 or x16 activations: each stage is the per-node call of its kind (p8x_mul_mat_vec_multi_act for one or
// several tensors on one input, p8x_mul_mat_vec_glu_act for a swiglu pair), enqueued in stage order on the stream;
// the cooperative launch quantizes its stages' inputs per 128 columns in the stage body and stays q8/128-only.
int p8x_step_create_act(const p8x_step_stage *stages, int n, int act, p8x_step **out) {
    if (act == P8X_ACT_Q8_128) return p8x_step_create(stages, n, out);
    if (act != P8X_ACT_Q8_1 && act != P8X_ACT_X16) return set_error(P8X_ERR_ARG, "p8x_step_create_act: act %d", act);
    if (!stages || n < 1 || !out) return set_error(P8X_ERR_ARG, "p8x_step_create_act: bad arguments");
    *out = nullptr;
    size_t hist[8] = {0};
    bool in_order = true;
    for (int s = 0; s < n; ++s) {
        const p8x_step_stage &st = stages[s];
        if (st.n < 1 || st.n > kRgMaxJobs) return set_error(P8X_ERR_ARG, "p8x_step_create_act: stage %d has %d tensors (1..%d)", s, st.n, kRgMaxJobs);
        int rc = check_shared_input(st.tensors, st.n, st.x, st.x ? st.tensors[0]->K : 0, "p8x_step_create_act");
        if (rc) return rc;
        const bool glu = st.glu_out != nullptr;
        if (glu && (st.n != 2 || st.tensors[0]->rows != st.tensors[1]->rows))
            return set_error(P8X_ERR_ARG, "p8x_step_create_act: stage %d: swiglu needs a gate and an up tensor of the same rows", s);
        for (int i = 0; i < st.n; ++i) {
            if (!glu && !st.y[i]) return set_error(P8X_ERR_ARG, "p8x_step_create_act: stage %d output %d is null", s, i);
            for (int c = 0; c < 8; ++c) hist[c] += st.tensors[i]->class_tiles[c];
            in_order = in_order && st.tensors[i]->lin_words != 0;
        }
    }
    p8x_step *sp = new p8x_step();
    sp->nst = n;
    sp->act = act;
    sp->cm = class_set(hist, in_order) == kCmC3 ? kCmC3 : kCmAll;
    (void)hipGetDevice(&sp->device);
    sp->host.assign(stages, stages + n);
    for (int s = 0; s < n; ++s)
        for (int i = 0; i < stages[s].n; ++i) sp->keep.push_back(stages[s].tensors[i]);
    *out = sp;
    return P8X_OK;
}

static int run_per_node(const p8x_step *sp, void *stream) {
    for (const p8x_step_stage &st : sp->host) {
        const size_t K = (size_t)st.tensors[0]->K;
        int rc;
        if (st.glu_out) {
            rc = p8x_mul_mat_vec_glu_act(st.tensors[0], st.tensors[1], sp->act, st.x, K, st.glu_out, stream);
        } else {
            size_t ldy[kRgMaxJobs];
            for (int i = 0; i < st.n; ++i) ldy[i] = (size_t)st.tensors[i]->rows;
            rc = p8x_mul_mat_vec_multi_act(st.tensors, st.n, sp->act, st.x, K, st.y, ldy, stream);
        }
        if (rc) return rc;
    }
    return P8X_OK;
}

int p8x_step_run(p8x_step *sp, void *stream) {
    if (!sp) return set_error(P8X_ERR_ARG, "p8x_step_run: null step");
    if (sp->act != P8X_ACT_Q8_128) return run_per_node(sp, stream);
    if (sp->broken) return set_error(P8X_ERR_HIP, "p8x_step_run: a previous launch gave up waiting (see p8x_step_check)");
    const unsigned spin = 1u << 20;
    hipStream_t st = (hipStream_t)stream;
    return sp->cm == kCmC3 ? launch_step_t<kCmC3>(sp->dstages, sp->nst, sp->words, spin, sp->a2, sp->grid, st)
                           : launch_step_t<kCmAll>(sp->dstages, sp->nst, sp->words, spin, sp->a2, sp->grid, st);
}

int p8x_step_check(p8x_step *sp) {
    if (!sp) return set_error(P8X_ERR_ARG, "p8x_step_check: null step");
    int rc = hip_check(hipDeviceSynchronize(), "p8x_step_check");
    if (rc || !sp->words) return rc;   // the per-node form has no barrier words
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
// (call it before capturing launches: it allocates the buffer on first use). The step kernel writes its per-stage
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
    if (class_set_) *class_set_ = sp->cm;
    return P8X_OK;
}

void p8x_step_release(p8x_step *sp) {
    if (!sp) return;
    (void)hipDeviceSynchronize();
    if (sp->dstages) (void)hipFree(sp->dstages);
    if (sp->words) (void)hipFree(sp->words);
    delete sp;
}

}  // extern "C"
