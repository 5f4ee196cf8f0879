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

#include "p8x_internal.h"
#include "p8x_lane.h"

namespace p8x {

constexpr int kGemvWaves = 8;
constexpr int kGemvThreads = 64 * kGemvWaves;

// ------------------------------------------------------------------------------------------------ activation prep
// correctly rounded f32 quotient via f64 (53 >= 2*24 + 2 bits: no double-rounding error)
__device__ __forceinline__ float div_rn(float a, float b) { return (float)((double)a / (double)b); }

// x' for one 256-block: lane holds 4 consecutive elements
__device__ __forceinline__ void rotate_block_lane(const float *__restrict__ x, const float *__restrict__ ic, int lane, float (&v)[4]) {
    const float4 xv = *reinterpret_cast<const float4 *>(x + 4 * lane);
    const float4 cv = *reinterpret_cast<const float4 *>(ic + 4 * lane);
    v[0] = xv.x * cv.x; v[1] = xv.y * cv.y; v[2] = xv.z * cv.z; v[3] = xv.w * cv.w;
    // h = 1, 2 inside the lane
    { const float a0 = v[0], b0 = v[1], a1 = v[2], b1 = v[3]; v[0] = a0 + b0; v[1] = a0 - b0; v[2] = a1 + b1; v[3] = a1 - b1; }
    { const float a0 = v[0], b0 = v[2], a1 = v[1], b1 = v[3]; v[0] = a0 + b0; v[2] = a0 - b0; v[1] = a1 + b1; v[3] = a1 - b1; }
    // h = 4 .. 128 across lanes: the lower index gets a + b, the upper a - b, with a the lower operand
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const bool upper = (lane & m) != 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float p = __shfl_xor(v[e], m);
            v[e] = upper ? p - v[e] : v[e] + p;
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] *= 0.0625f;
}

__device__ __forceinline__ float half_wave_max(float v) {
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}

__device__ __forceinline__ int half_wave_sum(int v) {
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) v += __shfl_xor(v, m);
    return v;
}

// grid (nb, ncols), block 64
__global__ __launch_bounds__(64) void k_act_q8_128(const float *__restrict__ x, size_t ldx, const float *__restrict__ ic, int K,
                                                   int8_t *__restrict__ q, float *__restrict__ d, int32_t *__restrict__ sum) {
    const int b = blockIdx.x, n = blockIdx.y, lane = threadIdx.x;
    float v[4];
    rotate_block_lane(x + (size_t)n * ldx + 256 * b, ic + 256 * b, lane, v);
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = half_wave_max(am);
    const float dd = div_rn(am, 127.f);
    const float id = dd > 0.f ? div_rn(1.f, dd) : 0.f;
    int qi[4], s = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) { qi[e] = __float2int_rn(v[e] * id); s += qi[e]; }
    const uint32_t packed = (uint32_t)(uint8_t)qi[0] | ((uint32_t)(uint8_t)qi[1] << 8) | ((uint32_t)(uint8_t)qi[2] << 16) | ((uint32_t)(uint8_t)qi[3] << 24);
    reinterpret_cast<uint32_t *>(q + (size_t)n * K + 256 * b)[lane] = packed;
    s = half_wave_sum(s);
    const int nsl = K / 128;
    if ((lane & 31) == 0) {
        d[(size_t)n * nsl + 2 * b + (lane >> 5)] = dd;
        if (sum) sum[(size_t)n * nsl + 2 * b + (lane >> 5)] = s;
    }
}

// block_q8_1 over x' (ggml layout: fp16 d, fp16 s = d * sum q, 32 int8). 8 lanes per 32-column block.
__global__ __launch_bounds__(64) void k_act_q8_1(const float *__restrict__ x, size_t ldx, const float *__restrict__ ic, int K,
                                                 uint8_t *__restrict__ blocks) {
    const int b = blockIdx.x, n = blockIdx.y, lane = threadIdx.x;
    float v[4];
    rotate_block_lane(x + (size_t)n * ldx + 256 * b, ic + 256 * b, lane, v);
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) am = fmaxf(am, __shfl_xor(am, m));
    const float dd = div_rn(am, 127.f);
    const float id = dd != 0.f ? div_rn(1.f, dd) : 0.f;
    int qi[4], s = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) { qi[e] = (int)roundf(v[e] * id); s += qi[e]; }
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) s += __shfl_xor(s, m);
    uint8_t *blk = blocks + ((size_t)n * (K / 32) + 8 * b + (lane >> 3)) * 36;
    const uint32_t packed = (uint32_t)(uint8_t)qi[0] | ((uint32_t)(uint8_t)qi[1] << 8) | ((uint32_t)(uint8_t)qi[2] << 16) | ((uint32_t)(uint8_t)qi[3] << 24);
    reinterpret_cast<uint32_t *>(blk + 4)[lane & 7] = packed;
    if ((lane & 7) == 0) {
        const uint32_t ds = (uint32_t)float_to_half(dd) | ((uint32_t)float_to_half((float)s * dd) << 16);
        *reinterpret_cast<uint32_t *>(blk) = ds;
    }
}

// ------------------------------------------------------------------------------------------------ fused decode + GEMV
struct GemvArgs {
    const uint32_t *M; const uint16_t *S; const uint32_t *D; const uint32_t *a2; const int16_t *prm;
    const int *cp; const uint16_t *cc; const float *cv;
    const int8_t *q;          // Q8_128: [ncol][K] int8
    const float *d;           // Q8_128: [ncol][nsl]
    const uint8_t *q81;       // Q8_1: [ncol][K/32] blocks
    const float *x; size_t ldx;   // original activations for the clamp delta (nullptr: no delta)
    float *y; size_t ldy;
    int32_t *partials;        // optional integer partials (sorted rows)
    float *wpart; unsigned *wcnt;
    int rows, K, nb, ng, nsl, bpk, nks, items;
};

template <int NCOL, int ACT>
struct GemvSmem {
    static constexpr int kXBytes = NCOL * 8 * 256;   // activation bytes of one item (bpk <= 8)
    static constexpr int kScales = ACT == P8X_ACT_Q8_128 ? 16 : 64;   // scales per column per item
    uint32_t tab[kTabWords];
    uint32_t xq[kXBytes / 4];
    float xd[NCOL * kScales];
    float red[kGemvWaves * NCOL * 32];
};

template <int NCOL, int ACT, bool PARTIALS, int C>
__device__ __forceinline__ void gemv_tile(const GemvArgs &a, const GemvSmem<NCOL, ACT> &sm, const uint32_t *__restrict__ payload,
                                          int lane, int bl, int b, int g, uint32_t bankbytes, float (&yacc)[NCOL]) {
    constexpr int NST = nstage_of(C), SH1 = sh1_of(C), SH2 = sh2_of(C), NW = nw_of(C);
    const int hs = lane >> 5, j = lane & 31;
    LaneSlice<C> ls;
    ls.load(payload + hs * NW * 32, j);
    const float sc = half_to_float(a.S[(size_t)b * a.rows + 32 * g + j]);
    ls.prepare(bankbytes);
    constexpr int NSUB = ACT == P8X_ACT_Q8_128 ? 1 : 4;   // integer sums per lane-slice
    int acc[NST][NCOL][NSUB];
#pragma unroll
    for (int s = 0; s < NST; ++s)
#pragma unroll
        for (int n = 0; n < NCOL; ++n)
#pragma unroll
            for (int u = 0; u < NSUB; ++u) acc[s][n][u] = 0;
    const uint32_t *xbase = sm.xq + (bl * 256 + hs * 128) / 4;
#pragma unroll
    for (int t4 = 0; t4 < 8; ++t4) {
        uint4 xv[NCOL];
#pragma unroll
        for (int n = 0; n < NCOL; ++n) xv[n] = *reinterpret_cast<const uint4 *>(xbase + n * (GemvSmem<NCOL, ACT>::kXBytes / 4 / NCOL) + 4 * t4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = 4 * t4 + e;
            constexpr int dummy = 0; (void)dummy;
            const int u = NSUB == 1 ? 0 : (t >> 3);
            uint32_t w[3];
            w[0] = lds_word(sm.tab, ls.template addr<0>(t));
            if constexpr (NST > 1) w[1] = lds_word(sm.tab, ls.template addr<1>(t));
            if constexpr (NST > 2) w[2] = lds_word(sm.tab, ls.template addr<2>(t));
#pragma unroll
            for (int n = 0; n < NCOL; ++n) {
                const uint32_t xc = e == 0 ? xv[n].x : e == 1 ? xv[n].y : e == 2 ? xv[n].z : xv[n].w;
#pragma unroll
                for (int s = 0; s < NST; ++s) acc[s][n][u] = __builtin_amdgcn_sdot4((int)w[s], (int)xc, acc[s][n][u], false);
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NCOL; ++n) {
#pragma unroll
        for (int u = 0; u < NSUB; ++u) {
            int isum = acc[0][n][u] * (1 << SH1);
            if constexpr (NST > 1) isum += acc[1][n][u] * (1 << SH2);
            if constexpr (NST > 2) isum += acc[2][n][u];
            if constexpr (PARTIALS) {
                const int r = 32 * g + j;
                if constexpr (ACT == P8X_ACT_Q8_128) a.partials[((size_t)n * a.rows + r) * a.nsl + 2 * b + hs] = isum;
                else a.partials[((size_t)n * a.rows + r) * (a.K / 32) + 8 * b + 4 * hs + u] = isum;
            }
            const float dsc = ACT == P8X_ACT_Q8_128 ? sm.xd[n * GemvSmem<NCOL, ACT>::kScales + 2 * bl + hs]
                                                    : sm.xd[n * GemvSmem<NCOL, ACT>::kScales + 8 * bl + 4 * hs + u];
            yacc[n] += ((float)isum * dsc) * sc;
        }
    }
}

template <int NCOL, int ACT, bool PARTIALS>
__global__ __launch_bounds__(kGemvThreads) void k_gemv(const GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    auto &sm = *reinterpret_cast<GemvSmem<NCOL, ACT> *>(smem_raw);
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t bankbytes = (uint32_t)((lane & 31) << 2) * 0x01010101u;
    build_coset_table(sm.tab, a.a2, tid, kGemvThreads);
    for (int item = blockIdx.x; item < a.items; item += gridDim.x) {
        const int g = item / a.nks, ks = item % a.nks;
        const int b0 = ks * a.bpk, nbl = min(a.bpk, a.nb - b0);
        // stage this item's activations (NCOL x nbl blocks of 256 bytes) and scales
        __syncthreads();
        constexpr int XW = GemvSmem<NCOL, ACT>::kXBytes / 4 / NCOL;   // words per column
        if constexpr (ACT == P8X_ACT_Q8_128) {
            for (int i = tid; i < NCOL * nbl * 64; i += kGemvThreads) {
                const int n = i / (nbl * 64), wi = i % (nbl * 64);
                sm.xq[n * XW + wi] = reinterpret_cast<const uint32_t *>(a.q + (size_t)n * a.K + 256 * b0)[wi];
            }
            for (int i = tid; i < NCOL * 2 * nbl; i += kGemvThreads) {
                const int n = i / (2 * nbl), si = i % (2 * nbl);
                sm.xd[n * GemvSmem<NCOL, ACT>::kScales + si] = a.d[(size_t)n * a.nsl + 2 * b0 + si];
            }
        } else {
            const int nq = a.K / 32;
            for (int i = tid; i < NCOL * nbl * 64; i += kGemvThreads) {
                const int n = i / (nbl * 64), wi = i % (nbl * 64);   // word wi: block wi / 8, word wi % 8 of its 32 ints
                const uint8_t *blk = a.q81 + ((size_t)n * nq + 8 * b0 + wi / 8) * 36;
                sm.xq[n * XW + wi] = reinterpret_cast<const uint32_t *>(blk + 4)[wi % 8];
            }
            for (int i = tid; i < NCOL * 8 * nbl; i += kGemvThreads) {
                const int n = i / (8 * nbl), si = i % (8 * nbl);
                const uint8_t *blk = a.q81 + ((size_t)n * nq + 8 * b0 + si) * 36;
                sm.xd[n * GemvSmem<NCOL, ACT>::kScales + si] = half_to_float(*reinterpret_cast<const uint16_t *>(blk));
            }
        }
        __syncthreads();
        float yacc[NCOL];
#pragma unroll
        for (int n = 0; n < NCOL; ++n) yacc[n] = 0.f;
        for (int bl = w; bl < nbl; bl += kGemvWaves) {
            const int b = b0 + bl;
            const uint32_t mt = a.M[(size_t)g * a.nb + b];
            const uint32_t *payload = a.D + (mt & 0x1FFFFFFFu);
            switch (mt >> 29) {
                case 1: gemv_tile<NCOL, ACT, PARTIALS, 1>(a, sm, payload, lane, bl, b, g, bankbytes, yacc); break;
                case 2: gemv_tile<NCOL, ACT, PARTIALS, 2>(a, sm, payload, lane, bl, b, g, bankbytes, yacc); break;
                case 3: gemv_tile<NCOL, ACT, PARTIALS, 3>(a, sm, payload, lane, bl, b, g, bankbytes, yacc); break;
                case 4: gemv_tile<NCOL, ACT, PARTIALS, 4>(a, sm, payload, lane, bl, b, g, bankbytes, yacc); break;
                case 5: gemv_tile<NCOL, ACT, PARTIALS, 5>(a, sm, payload, lane, bl, b, g, bankbytes, yacc); break;
                case 6: gemv_tile<NCOL, ACT, PARTIALS, 6>(a, sm, payload, lane, bl, b, g, bankbytes, yacc); break;
                case 7: gemv_tile<NCOL, ACT, PARTIALS, 7>(a, sm, payload, lane, bl, b, g, bankbytes, yacc); break;
                default:
                    if constexpr (PARTIALS) {   // class 0: zero weights
                        const int r = 32 * g + (lane & 31), hs = lane >> 5;
                        for (int n = 0; n < NCOL; ++n) {
                            if constexpr (ACT == P8X_ACT_Q8_128) a.partials[((size_t)n * a.rows + r) * a.nsl + 2 * b + hs] = 0;
                            else for (int u = 0; u < 4; ++u) a.partials[((size_t)n * a.rows + r) * (a.K / 32) + 8 * b + 4 * hs + u] = 0;
                        }
                    }
                    break;
            }
        }
        // half-slice 1 joins half-slice 0, then the waves meet in LDS
#pragma unroll
        for (int n = 0; n < NCOL; ++n) {
            const float o = __shfl_xor(yacc[n], 32);
            if (lane < 32) sm.red[(w * NCOL + n) * 32 + lane] = yacc[n] + o;
        }
        __syncthreads();
        float ysum = 0.f;
        int n = 0, j = 0;
        if (tid < 32 * NCOL) {
            n = tid >> 5; j = tid & 31;
            for (int ww = 0; ww < kGemvWaves; ++ww) ysum += sm.red[(ww * NCOL + n) * 32 + j];
        }
        bool final_rows = a.nks == 1;
        if (a.nks > 1) {
            if (tid < 32 * NCOL) a.wpart[((size_t)ks * NCOL + n) * a.rows + 32 * g + j] = ysum;
            __threadfence();
            __syncthreads();
            __shared__ unsigned last;
            if (tid == 0) last = atomicAdd(&a.wcnt[g], 1u) == (unsigned)(a.nks - 1);
            __syncthreads();
            final_rows = last != 0;
            if (final_rows) {
                __threadfence();
                if (tid < 32 * NCOL) {
                    ysum = 0.f;
                    for (int k2 = 0; k2 < a.nks; ++k2)
                        ysum += __hip_atomic_load(&a.wpart[((size_t)k2 * NCOL + n) * a.rows + 32 * g + j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                if (tid == 0) a.wcnt[g] = 0u;
            }
        }
        if (final_rows && tid < 32 * NCOL) {
            const int ro = a.prm[32 * g + j];
            if (a.x) {
                const float *xr = a.x + (size_t)n * a.ldx;
                for (int e = a.cp[ro]; e < a.cp[ro + 1]; ++e) ysum += a.cv[e] * xr[a.cc[e]];
            }
            a.y[(size_t)n * a.ldy + ro] = ysum;
        }
    }
}

GemvPlan gemv_plan(const p8x_tensor *t, int ncols) {
    (void)ncols;
    GemvPlan p;
    p.bpk = t->nb < 8 ? t->nb : 8;
    p.nks = (t->nb + p.bpk - 1) / p.bpk;
    p.items = t->ng * p.nks;
    p.grid = p.items;
    return p;
}

template <int NCOL, int ACT, bool PARTIALS>
static int launch_gemv_t(const GemvArgs &a, int items, hipStream_t st) {
    const size_t smem = sizeof(GemvSmem<NCOL, ACT>);
    auto kern = k_gemv<NCOL, ACT, PARTIALS>;
    static bool attr_set = false;
    if (!attr_set) {
        int rc = hip_check(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem), "gemv smem attribute");
        if (rc) return rc;
        attr_set = true;
    }
    const int per_cu = smem <= 80 * 1024 ? 2 : 1;
    const int grid = std::min(items, num_cus() * per_cu);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kGemvThreads), smem, st, a);
    return hip_check(hipGetLastError(), "k_gemv launch");
}

template <int ACT, bool PARTIALS>
static int launch_gemv_cols(const GemvArgs &a, int ncols, int items, hipStream_t st) {
    switch (ncols) {
        case 1: return launch_gemv_t<1, ACT, PARTIALS>(a, items, st);
        case 2: return launch_gemv_t<2, ACT, PARTIALS>(a, items, st);
        case 3: return launch_gemv_t<3, ACT, PARTIALS>(a, items, st);
        case 4: return launch_gemv_t<4, ACT, PARTIALS>(a, items, st);
        case 5: return launch_gemv_t<5, ACT, PARTIALS>(a, items, st);
        case 6: return launch_gemv_t<6, ACT, PARTIALS>(a, items, st);
        case 7: return launch_gemv_t<7, ACT, PARTIALS>(a, items, st);
        case 8: return launch_gemv_t<8, ACT, PARTIALS>(a, items, st);
        default: return set_error(P8X_ERR_ARG, "gemv: ncols %d", ncols);
    }
}

int launch_gemv(const p8x_tensor *t, int act, const void *q, const float *d, int ncols, const float *x, size_t ldx,
                float *y, size_t ldy, int32_t *partials, hipStream_t st) {
    GemvArgs a{};
    a.M = t->M; a.S = t->S; a.D = t->D; a.a2 = t->a2; a.prm = t->prm;
    a.cp = t->cp; a.cc = t->cc; a.cv = t->cv;
    if (act == P8X_ACT_Q8_128) { a.q = (const int8_t *)q; a.d = d; }
    else a.q81 = (const uint8_t *)q;
    a.x = x; a.ldx = ldx; a.y = y; a.ldy = ldy; a.partials = partials;
    a.wpart = t->wpart; a.wcnt = t->wcnt;
    a.rows = t->rows; a.K = t->K; a.nb = t->nb; a.ng = t->ng; a.nsl = t->nsl;
    a.bpk = t->gemv_bpk; a.nks = t->gemv_nks; a.items = t->ng * t->gemv_nks;
    if (act == P8X_ACT_Q8_128) {
        return partials ? launch_gemv_cols<P8X_ACT_Q8_128, true>(a, ncols, a.items, st) : launch_gemv_cols<P8X_ACT_Q8_128, false>(a, ncols, a.items, st);
    }
    return partials ? launch_gemv_cols<P8X_ACT_Q8_1, true>(a, ncols, a.items, st) : launch_gemv_cols<P8X_ACT_Q8_1, false>(a, ncols, a.items, st);
}

int launch_act_q8_128(const p8x_tensor *t, const float *x, int ncols, size_t ldx, int8_t *q, float *d, int32_t *sum, hipStream_t st) {
    hipLaunchKernelGGL(k_act_q8_128, dim3(t->nb, ncols), dim3(64), 0, st, x, ldx, (const float *)t->ic, t->K, q, d, sum);
    return hip_check(hipGetLastError(), "k_act_q8_128 launch");
}

int launch_act_q8_1(const p8x_tensor *t, const float *x, int ncols, size_t ldx, void *blocks, hipStream_t st) {
    hipLaunchKernelGGL(k_act_q8_1, dim3(t->nb, ncols), dim3(64), 0, st, x, ldx, (const float *)t->ic, t->K, (uint8_t *)blocks);
    return hip_check(hipGetLastError(), "k_act_q8_1 launch");
}

}  // namespace p8x
