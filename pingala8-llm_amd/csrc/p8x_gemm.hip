// p8x_gemm.hip -- prompt-processing GEMM: Y [N][rows] = X [N][K] W^T for a Pingala-8 tensor W.
//
// The 256-point Hadamard rotation of every weight block moves onto the activations:
//   W[prm[r], 256b + c] = (FWHT(v[r, 256b + :] S[b][r]) / 16)[c] ic[256b + c]   (+ clamp delta)
// so  Y[n, prm[r]] = sum_b S[b][r] sum_i v[r, 256b + i] x'[n, 256b + i] + delta terms, with
//   x' = FWHT(x ic) / 16 per 256-block (the GEMV's activation prep, CPU.patch:559-571, kept in fp16 here).
// Pass 1 (k_mm_act) writes x' as fp16 [N][K]. Pass 2 (k_mm) gives each wave two 32-row tiles of a 256-row
// workgroup tile: per 256-block it decodes the tiles in chunk order (rotated loads, p8x_lane.h) from a
// 2 KB LDS copy of the coset table straight into fp16 MFMA operands (v S, one rounding), and multiplies them
// with x' staged in LDS by v_mfma_f32_32x32x16_f16 with fp32 accumulation. Tokens are the MFMA rows and weight
// rows its columns, so each lane's outputs run along 32 consecutive sorted rows. Deep-K shapes split K over
// workgroups into fp32 partial planes summed in a fixed order by k_mm_reduce (deterministic). The sparse
// clamp delta (CPU.patch:1193) is added last on the original activations by k_mm_delta.
//
// Reference role: ggml_cuda_f44_mul_mat_q8 (CPU.patch:2303-2343), which instead dequantizes the tensor to a
// Q8_0 slab (k_r51_k1, CPU.patch:2138-2235) and calls the stock integer MMQ.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "p8x_internal.h"
#include "p8x_lane.h"

namespace p8x {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int kMmRows = 256;     // weight rows per workgroup tile (4 waves x 2 row groups)
constexpr int kMmTok = 128;      // tokens per workgroup tile (4 MFMA row tiles of 32)
constexpr int kMmThreads = 256;
constexpr int kMmXStride = 136;  // halfs per staged token row (128 + 8 pad: 16-byte reads spread over the banks)

// ------------------------------------------------------------------------------------------------ pass 1
// x' = FWHT(x ic) / 16 per 256-block, fp16. Lane holds 4 consecutive elements; butterflies h = 1, 2 in the
// lane, 4 .. 128 across lanes.
template <typename XT>
__global__ __launch_bounds__(64) void k_mm_act(const XT *__restrict__ x, size_t ldx, const float *__restrict__ ic, int K,
                                               _Float16 *__restrict__ xr) {
    const int b = blockIdx.x, n = blockIdx.y, lane = threadIdx.x;
    const XT *xp = x + (size_t)n * ldx + 256 * b + 4 * lane;
    const float4 cv = *reinterpret_cast<const float4 *>(ic + 256 * b + 4 * lane);
    float v[4];
    if constexpr (sizeof(XT) == 4) {
        v[0] = xp[0]; v[1] = xp[1]; v[2] = xp[2]; v[3] = xp[3];
    } else {
        const uint2 raw = *reinterpret_cast<const uint2 *>(xp);
        v[0] = bf16_to_float((uint16_t)raw.x); v[1] = bf16_to_float((uint16_t)(raw.x >> 16));
        v[2] = bf16_to_float((uint16_t)raw.y); v[3] = bf16_to_float((uint16_t)(raw.y >> 16));
    }
    v[0] *= cv.x; v[1] *= cv.y; v[2] *= cv.z; v[3] *= cv.w;
    { const float a0 = v[0], b0 = v[1], a1 = v[2], b1 = v[3]; v[0] = a0 + b0; v[1] = a0 - b0; v[2] = a1 + b1; v[3] = a1 - b1; }
    { const float a0 = v[0], b0 = v[2], a1 = v[1], b1 = v[3]; v[0] = a0 + b0; v[2] = a0 - b0; v[1] = a1 + b1; v[3] = a1 - b1; }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const bool upper = (lane & m) != 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float p = __shfl_xor(v[e], m);
            v[e] = upper ? p - v[e] : v[e] + p;
        }
    }
    half2v lo, hi;
    lo.x = (_Float16)(v[0] * 0.0625f); lo.y = (_Float16)(v[1] * 0.0625f);
    hi.x = (_Float16)(v[2] * 0.0625f); hi.y = (_Float16)(v[3] * 0.0625f);
    uint2 out;
    out.x = __builtin_bit_cast(uint32_t, lo);
    out.y = __builtin_bit_cast(uint32_t, hi);
    *reinterpret_cast<uint2 *>(xr + (size_t)n * K + 256 * b + 4 * lane) = out;
}

// ------------------------------------------------------------------------------------------------ pass 2
struct MmJob {
    const uint32_t *M; const uint16_t *S; const uint32_t *D; const int16_t *prm;
    const _Float16 *xr;     // x' [N][K]
    float *y; unsigned ldy;
    float *ws;              // partial planes [nsplit][N][rows] (sorted rows), nsplit > 1
    const uint32_t *a2;     // [2][256] coset table words (A[f] + h c), h-major
    int N, rows, K, nb, ng;
    int tiles_m, tiles_n, nsplit, kper;
};

// Rotated lane-slice words of any class up to NWMAX words (chunk order after the per-lane rotation), plus the
// coset bits in chunk order. Region layout as stored: [label word if W1 < 8] stage-1 fields, stage 2, stage 3.
template <int NWMAX>
struct MmSlice {
    uint32_t r[NWMAX];
    uint32_t H;
    uint16_t s;

    template <int C>
    __device__ __forceinline__ void load(const uint32_t *__restrict__ p, int j, const uint16_t *__restrict__ srow) {
        constexpr int W1 = w1_of(C), W2 = w2_of(C), W3 = w3_of(C);
        uint32_t z;
        if constexpr (W1 == 8) {
            uint32_t R[8];
            load_region<8, 0>(p, j, R);
#pragma unroll
            for (int i = 0; i < 8; ++i) r[i] = R[i];
            z = labels_from_bytes(R);
        } else {
            const uint32_t w0 = __builtin_nontemporal_load(p + lane_word_offset(0, j));
            r[0] = __builtin_amdgcn_alignbit(w0, w0, (32 - j) & 31);
            z = r[0];
            uint32_t R[W1 - 1];
            load_region<W1 - 1, 1>(p, j, R);
#pragma unroll
            for (int i = 0; i < W1 - 1; ++i) r[1 + i] = R[i];
        }
        if constexpr (W2 > 0) {
            uint32_t R[W2];
            load_region<W2, W1>(p, j, R);
#pragma unroll
            for (int i = 0; i < W2; ++i) r[W1 + i] = R[i];
        }
        if constexpr (W3 > 0) {
            uint32_t R[W3];
            load_region<W3, W1 + W2>(p, j, R);
#pragma unroll
            for (int i = 0; i < W3; ++i) r[W1 + W2 + i] = R[i];
        }
        H = trellis_coset_bits(z);
        s = srow[j];
    }

    // stage-S field of chunk t
    template <int C, int S>
    __device__ __forceinline__ uint32_t field(int t) const {
        constexpr int W1 = w1_of(C), W2 = w2_of(C);
        if constexpr (S == 0) {
            if constexpr (W1 == 8) return __builtin_amdgcn_ubfe(r[t >> 2], 8 * (t & 3), 8);
            else {
                constexpr int W = W1 - 1;
                const int pos = W * t, wi = 1 + (pos >> 5), bb = pos & 31;
                uint32_t f;
                if (bb + W <= 32) f = __builtin_amdgcn_ubfe(r[wi], bb, W);
                else f = __builtin_amdgcn_alignbit(r[1 + ((wi - 1 + 1) % W)], r[wi], bb) & ((1u << W) - 1u);
                return f | (__builtin_amdgcn_ubfe(r[0], t, 1) << W);
            }
        } else if constexpr (S == 1) {
            if constexpr (W2 == 8) return __builtin_amdgcn_ubfe(r[W1 + (t >> 2)], 8 * (t & 3), 8);
            else {
                const int pos = W2 * t, wi = pos >> 5, bb = pos & 31;
                if (bb + W2 <= 32) return __builtin_amdgcn_ubfe(r[W1 + wi], bb, W2);
                return __builtin_amdgcn_alignbit(r[W1 + (wi + 1) % W2], r[W1 + wi], bb) & ((1u << W2) - 1u);
            }
        } else {
            return __builtin_amdgcn_ubfe(r[W1 + W2 + (t >> 2)], 8 * (t & 3), 8);
        }
    }
};

// offset-binary int8x4 (v + 128 per byte) -> two fp16 pairs holding 1152 + v exactly
__device__ __forceinline__ half2v ob_lo(uint32_t w) { return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u)); }
__device__ __forceinline__ half2v ob_hi(uint32_t w) { return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u)); }

// chunk t of class C -> 4 fp16 weights v S (v exact in fp16, |v| <= 1596; one rounding for the product)
template <int C, int NWMAX>
__device__ __forceinline__ void decode_chunk(const MmSlice<NWMAX> &ls, const uint32_t *tab, int t, half2v s2, half2v &lo, half2v &hi) {
    constexpr int NST = nstage_of(C), SH1 = sh1_of(C), SH2 = sh2_of(C);
    const uint32_t h4 = __builtin_amdgcn_ubfe(ls.H, t, 1) << 2;
    const half2v bias = {(_Float16)-1152.f, (_Float16)-1152.f};
    uint32_t w[3];
    w[0] = lds_word(tab, (ls.template field<C, 0>(t) << 3) | h4);
    if constexpr (NST > 1) w[1] = lds_word(tab, (ls.template field<C, 1>(t) << 3) | h4);
    if constexpr (NST > 2) w[2] = lds_word(tab, (ls.template field<C, 2>(t) << 3) | h4);
    half2v vl = ob_lo(w[0]) + bias, vh = ob_hi(w[0]) + bias;
    if constexpr (NST > 1) {
        const half2v m1 = {(_Float16)(float)(1 << SH1), (_Float16)(float)(1 << SH1)};
        const half2v m2 = {(_Float16)(float)(1 << SH2), (_Float16)(float)(1 << SH2)};
        half2v al = (ob_lo(w[1]) + bias) * m2, ah = (ob_hi(w[1]) + bias) * m2;
        if constexpr (NST > 2) { al += ob_lo(w[2]) + bias; ah += ob_hi(w[2]) + bias; }
        vl = vl * m1 + al;
        vh = vh * m1 + ah;
    }
    lo = vl * s2;
    hi = vh * s2;
}

template <int C, int NWMAX>
__device__ __forceinline__ half8v decode_pair(const MmSlice<NWMAX> &ls, const uint32_t *tab, int s) {
    const half2v s2 = {__builtin_bit_cast(_Float16, ls.s), __builtin_bit_cast(_Float16, ls.s)};
    half2v a, b, c, d;
    decode_chunk<C>(ls, tab, 2 * s, s2, a, b);
    decode_chunk<C>(ls, tab, 2 * s + 1, s2, c, d);
    half8v o;
    o[0] = a.x; o[1] = a.y; o[2] = b.x; o[3] = b.y; o[4] = c.x; o[5] = c.y; o[6] = d.x; o[7] = d.y;
    return o;
}

// classes decoded by an instantiation: the tensor's class set (class 0 decodes as zeros in all of them)
constexpr int kMmCmC3 = 1 << 3, kMmCmAll = 0xFE;
__host__ __device__ constexpr int mm_nwmax(int cm) { return cm == kMmCmC3 ? 8 : 24; }

template <int CM, int NWMAX>
__device__ __forceinline__ half8v decode_any(const MmSlice<NWMAX> &ls, int c, const uint32_t *tab, int s) {
    switch (c) {
        case 1: if constexpr ((CM >> 1) & 1) return decode_pair<1>(ls, tab, s); break;
        case 2: if constexpr ((CM >> 2) & 1) return decode_pair<2>(ls, tab, s); break;
        case 3: if constexpr ((CM >> 3) & 1) return decode_pair<3>(ls, tab, s); break;
        case 4: if constexpr ((CM >> 4) & 1) return decode_pair<4>(ls, tab, s); break;
        case 5: if constexpr ((CM >> 5) & 1) return decode_pair<5>(ls, tab, s); break;
        case 6: if constexpr ((CM >> 6) & 1) return decode_pair<6>(ls, tab, s); break;
        case 7: if constexpr ((CM >> 7) & 1) return decode_pair<7>(ls, tab, s); break;
        default: break;
    }
    return half8v{};
}

template <int CM, int NWMAX>
__device__ __forceinline__ void load_any(MmSlice<NWMAX> &ls, int c, const uint32_t *p, int j, const uint16_t *srow) {
    switch (c) {
        case 1: if constexpr ((CM >> 1) & 1) ls.template load<1>(p, j, srow); break;
        case 2: if constexpr ((CM >> 2) & 1) ls.template load<2>(p, j, srow); break;
        case 3: if constexpr ((CM >> 3) & 1) ls.template load<3>(p, j, srow); break;
        case 4: if constexpr ((CM >> 4) & 1) ls.template load<4>(p, j, srow); break;
        case 5: if constexpr ((CM >> 5) & 1) ls.template load<5>(p, j, srow); break;
        case 6: if constexpr ((CM >> 6) & 1) ls.template load<6>(p, j, srow); break;
        case 7: if constexpr ((CM >> 7) & 1) ls.template load<7>(p, j, srow); break;
        default: break;
    }
}

template <int CM>
__global__ __launch_bounds__(kMmThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_mm(MmJob J) {
    constexpr int NWMAX = mm_nwmax(CM);
    __shared__ uint32_t tab[512];                          // (f << 1 | h): A[f] + h c, bytes offset by 128
    __shared__ __attribute__((aligned(16))) _Float16 xs[kMmTok * kMmXStride];   // x' part: [token][kh * 64 + 8 (s & 7) + i]
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31, kh = lane >> 5;
    int wg = blockIdx.x;
    const int ks = wg % J.nsplit; wg /= J.nsplit;
    const int tn = wg % J.tiles_n, tm = wg / J.tiles_n;
    for (int i = tid; i < 512; i += kMmThreads) tab[i] = J.a2[(i & 1) * 256 + (i >> 1)] ^ 0x80808080u;
    const int tok0 = tn * kMmTok;
    const int b0 = ks * J.kper, b1 = min(J.nb, b0 + J.kper);
    int g[2];
    g[0] = (tm * kMmRows) / 32 + 2 * w;
    g[1] = g[0] + 1;
    float16v acc[4][2];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj) acc[ti][tj] = float16v{};
    // staging map: thread -> (token, kh): 128 contiguous bytes of x' per part
    const int st_tok = tid >> 1, st_kh = tid & 1;
    const bool st_ok = tok0 + st_tok < J.N;
    const _Float16 *xsrc = J.xr + (size_t)(tok0 + st_tok) * J.K + 128 * st_kh;
    for (int b = b0; b < b1; ++b) {
        MmSlice<NWMAX> ls[2];
        int cl[2];
#pragma unroll
        for (int tj = 0; tj < 2; ++tj) {
            cl[tj] = 0;
            if (g[tj] < J.ng) {
                const uint32_t mt = J.M[(size_t)g[tj] * J.nb + b];
                cl[tj] = (int)(mt >> 29);
                const int nw = nw_of(cl[tj]);
                load_any<CM>(ls[tj], cl[tj], J.D + (mt & 0x1FFFFFFFu) + kh * nw * 32, j, J.S + (size_t)b * J.rows + 32 * g[tj]);
            }
        }
#pragma unroll
        for (int sh = 0; sh < 2; ++sh) {
            uint4 v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = st_ok ? reinterpret_cast<const uint4 *>(xsrc + 256 * b + 64 * sh)[i] : make_uint4(0, 0, 0, 0);
            __syncthreads();   // the previous part's reads are done
#pragma unroll
            for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4 *>(xs + st_tok * kMmXStride + 64 * st_kh + 8 * i) = v[i];
            __syncthreads();
#pragma unroll
            for (int s8 = 0; s8 < 8; ++s8) {
                const int s = 8 * sh + s8;
                half8v A[4], B[2];
#pragma unroll
                for (int ti = 0; ti < 4; ++ti) A[ti] = *reinterpret_cast<const half8v *>(xs + (32 * ti + j) * kMmXStride + 64 * kh + 8 * s8);
#pragma unroll
                for (int tj = 0; tj < 2; ++tj) B[tj] = decode_any<CM>(ls[tj], cl[tj], tab, s);
#pragma unroll
                for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                    for (int tj = 0; tj < 2; ++tj) acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[ti], B[tj], acc[ti][tj], 0, 0, 0);
            }
        }
    }
    // acc[ti][tj] lane l, reg q: token 32 ti + 8 (q >> 2) + 4 kh + (q & 3), sorted row 32 g[tj] + j
#pragma unroll
    for (int tj = 0; tj < 2; ++tj) {
        if (g[tj] >= J.ng) continue;
        const int r = 32 * g[tj] + j;
        const int ro = J.nsplit == 1 ? J.prm[r] : r;
        float *dst = J.nsplit == 1 ? J.y : J.ws + (size_t)ks * J.N * J.rows;
        const size_t ld = J.nsplit == 1 ? J.ldy : (size_t)J.rows;
#pragma unroll
        for (int ti = 0; ti < 4; ++ti)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int tok = tok0 + 32 * ti + 8 * (q >> 2) + 4 * kh + (q & 3);
                if (tok < J.N) dst[(size_t)tok * ld + ro] = acc[ti][tj][q];
            }
    }
}

// y[n][prm[r]] = sum over K splits in split order
__global__ __launch_bounds__(256) void k_mm_reduce(const float *__restrict__ ws, int nsplit, int N, int rows, const int16_t *__restrict__ prm,
                                                   float *__restrict__ y, size_t ldy) {
    const int r = blockIdx.x * 256 + threadIdx.x, n = blockIdx.y;
    if (r >= rows) return;
    float s = 0.f;
    for (int k = 0; k < nsplit; ++k) s += ws[((size_t)k * N + n) * rows + r];
    y[(size_t)n * ldy + prm[r]] = s;
}

// clamp delta on the original activations: y[n][row] += sum_e cv[e] x[n][cc[e]] for the rows that have entries
template <typename XT>
__global__ __launch_bounds__(256) void k_mm_delta(const int *__restrict__ drows, const int *__restrict__ cp, const uint16_t *__restrict__ cc,
                                                  const float *__restrict__ cv, const XT *__restrict__ x, size_t ldx, int N, float *__restrict__ y, size_t ldy) {
    const int ro = drows[blockIdx.x];
    const int n = blockIdx.y * 256 + threadIdx.x;
    if (n >= N) return;
    const XT *xr = x + (size_t)n * ldx;
    float v = y[(size_t)n * ldy + ro];
    for (int e = cp[ro]; e < cp[ro + 1]; ++e) {
        float xv;
        if constexpr (sizeof(XT) == 4) xv = xr[cc[e]];
        else xv = bf16_to_float((uint16_t)xr[cc[e]]);
        v += cv[e] * xv;
    }
    y[(size_t)n * ldy + ro] = v;
}

static int grow(void **p, size_t *have, size_t need, const char *what) {
    if (*have >= need) return P8X_OK;
    if (*p) {
        int rc = hip_check(hipDeviceSynchronize(), what);
        if (rc) return rc;
        (void)hipFree(*p);
        *p = nullptr;
        *have = 0;
    }
    if (hipMalloc(p, need) != hipSuccess) return set_error(P8X_ERR_NOMEM, "%s: hipMalloc %zu bytes", what, need);
    *have = need;
    return P8X_OK;
}

struct MmPlan {
    int tiles_m, tiles_n, nsplit, kper;
};

static MmPlan mm_plan(const p8x_tensor *t, int N) {
    MmPlan p;
    p.tiles_m = (t->rows + kMmRows - 1) / kMmRows;
    p.tiles_n = (N + kMmTok - 1) / kMmTok;
    const int base = p.tiles_m * p.tiles_n, slots = 2 * num_cus();
    int ns = (slots + base - 1) / base;
    ns = std::max(1, std::min(ns, t->nb / 4));
    p.kper = (t->nb + ns - 1) / ns;
    p.nsplit = (t->nb + p.kper - 1) / p.kper;
    return p;
}

int launch_mul_mat(const p8x_tensor *t, const void *x, int x_dtype, int N, size_t ldx, float *y, size_t ldy, hipStream_t st) {
    if (((uintptr_t)x & 15) || (ldx % 8)) return set_error(P8X_ERR_ARG, "p8x_mul_mat: x must be 16-byte aligned with ldx %% 8 == 0");
    p8x_tensor *tw = const_cast<p8x_tensor *>(t);
    const MmPlan p = mm_plan(t, N);
    int rc;
    if ((rc = grow((void **)&tw->wx16, &tw->wx16_elems, (size_t)N * t->K * sizeof(_Float16), "p8x_mul_mat: activation workspace"))) return rc;
    if (p.nsplit > 1 && (rc = grow((void **)&tw->wmm, &tw->wmm_bytes, (size_t)p.nsplit * N * t->rows * 4, "p8x_mul_mat: split workspace"))) return rc;
    _Float16 *xr = reinterpret_cast<_Float16 *>(tw->wx16);
    if (x_dtype == P8X_F32) hipLaunchKernelGGL(k_mm_act<float>, dim3(t->nb, N), dim3(64), 0, st, (const float *)x, ldx, t->ic, t->K, xr);
    else hipLaunchKernelGGL(k_mm_act<uint16_t>, dim3(t->nb, N), dim3(64), 0, st, (const uint16_t *)x, ldx, t->ic, t->K, xr);
    if ((rc = hip_check(hipGetLastError(), "k_mm_act launch"))) return rc;
    MmJob J;
    J.M = t->M; J.S = t->S; J.D = t->D; J.prm = t->prm; J.xr = xr;
    J.y = y; J.ldy = (unsigned)ldy; J.ws = tw->wmm; J.a2 = t->a2;
    J.N = N; J.rows = t->rows; J.K = t->K; J.nb = t->nb; J.ng = t->ng;
    J.tiles_m = p.tiles_m; J.tiles_n = p.tiles_n; J.nsplit = p.nsplit; J.kper = p.kper;
    const int grid = p.tiles_m * p.tiles_n * p.nsplit;
    bool only_c3 = true;
    for (int c = 1; c < 8; ++c) if (c != 3 && t->class_tiles[c]) only_c3 = false;
    if (only_c3) hipLaunchKernelGGL(k_mm<kMmCmC3>, dim3(grid), dim3(kMmThreads), 0, st, J);
    else hipLaunchKernelGGL(k_mm<kMmCmAll>, dim3(grid), dim3(kMmThreads), 0, st, J);
    if ((rc = hip_check(hipGetLastError(), "k_mm launch"))) return rc;
    if (p.nsplit > 1) {
        hipLaunchKernelGGL(k_mm_reduce, dim3((t->rows + 255) / 256, N), dim3(256), 0, st, (const float *)tw->wmm, p.nsplit, N, t->rows, t->prm, y, ldy);
        if ((rc = hip_check(hipGetLastError(), "k_mm_reduce launch"))) return rc;
    }
    if (t->ndrows) {
        if (x_dtype == P8X_F32)
            hipLaunchKernelGGL(k_mm_delta<float>, dim3(t->ndrows, (N + 255) / 256), dim3(256), 0, st, t->drows, t->cp, t->cc, t->cv, (const float *)x, ldx, N, y, ldy);
        else
            hipLaunchKernelGGL(k_mm_delta<uint16_t>, dim3(t->ndrows, (N + 255) / 256), dim3(256), 0, st, t->drows, t->cp, t->cc, t->cv, (const uint16_t *)x, ldx, N, y, ldy);
        if ((rc = hip_check(hipGetLastError(), "k_mm_delta launch"))) return rc;
    }
    return P8X_OK;
}

}  // namespace p8x
