// p8x_step.hip -- a batch-1 decode step's chain of linears in one persistent launch.
//
// The reference launches one kernel per MUL_MAT node (CPU.patch:2615-2631, :4466-4521), so a step of L layers runs
// 4 L + 1 dependent launches (q/k/v, o, gate/up, down, then the head), each paying the launch and the kernel-boundary
// cache work, and each rebuilding the 64 KB coset table in every workgroup. Here one cooperative launch walks the
// whole chain: the table is built once per workgroup, the stages run the row-group GEMV body of k_gemv_rg (whole
// 32-row groups per workgroup, K-chunks with the fixed-order fix-up, teams of waves, several linears on one input,
// the swiglu meet), and a grid barrier separates each stage from the next, whose input is its output.
//
// Cross-workgroup hand-off. A stage's outputs are agent-scope atomic stores (sc1: written through the XCD's L2 to the
// agent's coherence point); every wave waits for its stores (vmcnt(0)) before the workgroup counts its arrival on the
// barrier counter; the next stage reads its input with agent-scope atomic loads issued after the barrier observed every
// arrival. This is the split-K fix-up's publication rule (p8x_gemv.h, arrive_after_stores) applied to whole stages.
//
// Termination. All workgroups are resident together (cooperative launch, one workgroup per CU, the grid sized from the
// kernel's occupancy); a barrier wait polls at most `spin` times, and a workgroup that gives up raises the shared fail
// flag, which every other waiting workgroup also polls, so every wave leaves the kernel in any case. The host reads
// the flag in p8x_step_check. The barrier counter only grows (each launch starts from the value the previous one left;
// comparisons are modulo 2^32).
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

struct StepStage {
    RgJobs R;   // the stage's linears: activations and K plan (R.j0), tensor metadata (R.jt), outputs, swiglu
    int nvwg;   // virtual workgroups of the stage (row-group assignments), R.wgbase[kRgMaxJobs]
    int gc;     // row groups a workgroup streams together (teams of waves; 1 with K-chunks)
};

struct StepSync {
    unsigned *bar;    // arrival counter
    unsigned *fail;   // nonzero once a wait gave up
    unsigned base;    // counter value at the launch's start
    unsigned spin;    // polls before a wait gives up
};

// 4 consecutive floats per lane, agent-coherent (the previous stage wrote them in this launch)
__device__ __forceinline__ f32x4 load4_coherent(const float *p, int lane) {
    float *q = const_cast<float *>(p) + 4 * lane;
    f32x4 v;
    v.x = __hip_atomic_load(q + 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    v.y = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    v.z = __hip_atomic_load(q + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    v.w = __hip_atomic_load(q + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return v;
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
#pragma unroll
    for (int i = 0; i < RQ; ++i) {
        const int it = w + i * WAVES, bk = c.b0 + it % nbk;
        if (it < nbk) {
            in[i].x = load4_coherent(J.x + 256 * bk, lane);
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

// Every wave's stores complete, one arrival per workgroup, then thread 0 polls until all gridDim.x arrivals of this
// barrier are in (or gives up, or sees another workgroup give up). Returns false when the launch must end.
__device__ __forceinline__ bool step_barrier(const StepSync &sy, unsigned target, int *flag) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(sy.bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned want = sy.base + target;
        int good = 1;
        for (unsigned n = 0;; ++n) {
            const unsigned cnt = __hip_atomic_load(sy.bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((int)(cnt - want) >= 0) break;
            if (__hip_atomic_load(sy.fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u || n >= sy.spin) {
                __hip_atomic_store(sy.fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
void k_step(const StepStage *__restrict__ stages, int nst, StepSync sync, const uint32_t *__restrict__ a2) {
    __shared__ RgSmem<1> sm;
    __shared__ int flag;
    const int tid = threadIdx.x;
    // the table once for the whole chain (each stage's barrier after its quantization orders these writes
    // before the first lookup)
    build_coset_table<64 * rg_waves(1)>(sm.tab, a2, tid);
    for (int s = 0; s < nst; ++s) {
        const kptr<const StepStage> sp = as_const(stages) + s;
        const int nv = sp->nvwg;
        for (int v = blockIdx.x; v < nv; v += gridDim.x) {
            step_stage<CM>(sp, v, sm, tid);
            __syncthreads();   // the next virtual workgroup rewrites the activation buffer
        }
        if (s + 1 < nst && !step_barrier(sync, (unsigned)(s + 1) * gridDim.x, &flag)) return;
    }
}

template <int CM>
static int launch_step_t(const StepStage *stages, int nst, const StepSync &sync, const uint32_t *a2, int grid, hipStream_t st) {
    void *args[] = {(void *)&stages, (void *)&nst, (void *)&sync, (void *)&a2};
    return hip_check(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(&k_step<CM>), dim3(grid), dim3(64 * rg_waves(1)), args,
                                                0, st),
                     "k_step cooperative launch");
}

template <int CM>
static int step_grid(int *grid) {
    int per_cu = 0;
    const int rc = hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(&k_step<CM>),
                                                                          64 * rg_waves(1), 0),
                             "k_step occupancy");
    if (rc) return rc;
    if (per_cu < 1) return set_error(P8X_ERR_UNSUPPORTED, "k_step: no workgroup fits a CU");
    *grid = per_cu * num_cus();
    return P8X_OK;
}

}  // namespace p8x

using namespace p8x;

struct p8x_step {
    StepStage *dstages = nullptr;
    int nst = 0, cm = 0, grid = 0;
    unsigned *sync_words = nullptr;   // [0] barrier counter, [1] fail flag
    unsigned base = 0;
    bool broken = false;
    const uint32_t *a2 = nullptr;
    int device = 0;
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
    int rc = sp->cm == kCmC3 ? step_grid<kCmC3>(&sp->grid) : step_grid<kCmAll>(&sp->grid);
    if (!rc && hipMalloc((void **)&sp->dstages, sizeof(StepStage) * n) != hipSuccess) rc = set_error(P8X_ERR_NOMEM, "p8x_step_create: hipMalloc stages");
    if (!rc && hipMalloc((void **)&sp->sync_words, 2 * sizeof(unsigned)) != hipSuccess) rc = set_error(P8X_ERR_NOMEM, "p8x_step_create: hipMalloc sync");
    if (!rc) rc = hip_check(hipMemcpy(sp->dstages, hs.data(), sizeof(StepStage) * n, hipMemcpyHostToDevice), "p8x_step_create: stages");
    if (!rc) rc = hip_check(hipMemset(sp->sync_words, 0, 2 * sizeof(unsigned)), "p8x_step_create: sync");
    if (!rc) rc = hip_check(hipDeviceSynchronize(), "p8x_step_create");
    if (rc) { p8x_step_release(sp); return rc; }
    *out = sp;
    return P8X_OK;
}

int p8x_step_run(p8x_step *sp, void *stream) {
    if (!sp) return set_error(P8X_ERR_ARG, "p8x_step_run: null step");
    if (sp->broken) return set_error(P8X_ERR_HIP, "p8x_step_run: a previous launch gave up at a barrier (see p8x_step_check)");
    StepSync sy;
    sy.bar = sp->sync_words;
    sy.fail = sp->sync_words + 1;
    sy.base = sp->base;
    sy.spin = 1u << 20;
    const int rc = sp->cm == kCmC3 ? launch_step_t<kCmC3>(sp->dstages, sp->nst, sy, sp->a2, sp->grid, (hipStream_t)stream)
                                   : launch_step_t<kCmAll>(sp->dstages, sp->nst, sy, sp->a2, sp->grid, (hipStream_t)stream);
    if (rc) return rc;
    sp->base += (unsigned)(sp->nst - 1) * (unsigned)sp->grid;
    return P8X_OK;
}

int p8x_step_check(p8x_step *sp) {
    if (!sp) return set_error(P8X_ERR_ARG, "p8x_step_check: null step");
    int rc = hip_check(hipDeviceSynchronize(), "p8x_step_check");
    if (rc) return rc;
    unsigned w[2] = {0, 0};
    rc = hip_check(hipMemcpy(w, sp->sync_words, sizeof w, hipMemcpyDeviceToHost), "p8x_step_check: read");
    if (rc) return rc;
    if (w[1]) {
        sp->broken = true;
        return set_error(P8X_ERR_HIP, "p8x_step: a barrier wait gave up (workgroups not co-resident?)");
    }
    if (w[0] != sp->base) {
        sp->broken = true;
        return set_error(P8X_ERR_HIP, "p8x_step: barrier count %u, expected %u", w[0], sp->base);
    }
    return P8X_OK;
}

#ifdef P8X_TIMELINE
// timeline build only: the row-group kernel's records (first n bytes) and their count; reset sets the count to 0
// (call it before capturing launches: it allocates the buffer on first use)
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
    if (sp->sync_words) (void)hipFree(sp->sync_words);
    delete sp;
}

}  // extern "C"
