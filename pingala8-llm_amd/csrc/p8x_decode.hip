// p8x_decode.hip -- block decode (exact tile ints, rotated f32) and dequantize_row (original domain).
//
// Exact ints: v = sum_s (A[f_s] + h c)_e << SH_s (vrc_decode_tile_int, CPU.patch:992-1010).
// Original domain (vrc_dequant_f32, CPU.patch:1012-1027): per sorted row r and block b,
// t = FWHT256(v * S[b][r]) with butterflies h = 1..128 then * 0.0625, t *= ic, row prm[r], + delta.
// A lane owns one half-row (128 values) in registers: stages h = 1..64 stay in the lane, stage 128 pairs
// lane j with lane j + 32. Every output is the same a + b / a - b of the same operands as the reference,
// so the f32 result is bit-identical (no contraction: built with -ffp-contract=off); f16/bf16 are the
// hardware round-to-nearest-even conversions of that f32.
//
// Each wave walks tiles with the next tile's payload already in flight (rotated loads into registers), so
// the decode of one tile overlaps the memory latency of the next.
#include <hip/hip_runtime.h>

#include "p8x_internal.h"
#include "p8x_lane.h"

namespace p8x {

constexpr int kDecWaves = 4;
constexpr int kDecThreads = 64 * kDecWaves;
constexpr int kDecNW = 24;   // raw words held per lane: the largest class

struct DecodeArgs {
    const uint32_t *M; const uint16_t *S; const uint32_t *D; const uint32_t *a2; const int16_t *prm;
    const float *ic; const int *cp; const uint16_t *cc; const float *cv;
    void *out; size_t ld;
    int rows, K, nb, ng;
    size_t nt;
};

// exact ints of a decoded lane-slice of class C -> v[128] (chunk-major, element e), as float times sc
// (FP = true) or as ints (FP = false, written through the float array's bits)
template <int C, bool FP>
__device__ __forceinline__ void lane_values(const AnySlice<kDecNW> &ls, const uint32_t *tab, uint32_t bankbytes, float sc, float (&v)[128]) {
    constexpr int NST = nstage_of(C), SH1 = sh1_of(C), SH2 = sh2_of(C);
#pragma unroll
    for (int t = 0; t < 32; ++t) {
        const uint32_t hq = coset_bytes(ls.H, bankbytes, t >> 2);
        const uint32_t w0 = lds_word(tab, ls.template addr<C, 0>(t, hq));
        uint32_t w1 = 0, w2 = 0;
        if constexpr (NST > 1) w1 = lds_word(tab, ls.template addr<C, 1>(t, hq));
        if constexpr (NST > 2) w2 = lds_word(tab, ls.template addr<C, 2>(t, hq));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            int x = sext8(w0, e) * (1 << SH1);
            if constexpr (NST > 1) x += sext8(w1, e) * (1 << SH2);
            if constexpr (NST > 2) x += sext8(w2, e);
            v[4 * t + e] = FP ? (float)x * sc : __builtin_bit_cast(float, x);
        }
    }
}

template <bool FP>
__device__ __forceinline__ void lane_values_any(int c, const AnySlice<kDecNW> &ls, const uint32_t *tab, uint32_t bankbytes, float sc, float (&v)[128]) {
    switch (c) {
        case 1: lane_values<1, FP>(ls, tab, bankbytes, sc, v); break;
        case 2: lane_values<2, FP>(ls, tab, bankbytes, sc, v); break;
        case 3: lane_values<3, FP>(ls, tab, bankbytes, sc, v); break;
        case 4: lane_values<4, FP>(ls, tab, bankbytes, sc, v); break;
        case 5: lane_values<5, FP>(ls, tab, bankbytes, sc, v); break;
        case 6: lane_values<6, FP>(ls, tab, bankbytes, sc, v); break;
        case 7: lane_values<7, FP>(ls, tab, bankbytes, sc, v); break;
        default:
#pragma unroll
            for (int i = 0; i < 128; ++i) v[i] = 0.f;   // class 0: zero weights (0.0f and int 0 share bits)
            break;
    }
}

// The wave's walk over tiles tile0, tile0 + stride, ...: body(tile, g, b, class, slice) runs on each tile
// while the next tile's raw payload loads.
template <typename Body>
__device__ __forceinline__ void walk_tiles(const DecodeArgs &a, size_t tile0, size_t stride, int hs, int j, Body body) {
    if (tile0 >= a.nt) return;
    constexpr int CM = 0xFE;
    AnyRaw<kDecNW> raw;
    auto issue = [&](size_t tile, int &c) {
        const int g = (int)(tile / a.nb), b = (int)(tile % a.nb);
        const uint32_t mt = a.M[tile];
        c = (int)(mt >> 29);
        load_any<CM>(raw, c, a.D + (mt & 0x1FFFFFFFu) + hs * nw_of(c) * 32, j, a.S + (size_t)b * a.rows + 32 * g);
    };
    int c;
    issue(tile0, c);
    for (size_t tile = tile0; tile < a.nt; tile += stride) {
        AnySlice<kDecNW> ls;
        prepare_any<CM>(ls, c, raw, j);   // consumes the words of this tile
        const int cur = c;
        if (tile + stride < a.nt) issue(tile + stride, c);   // the next tile's words load during this tile
        body(tile, (int)(tile / a.nb), (int)(tile % a.nb), cur, ls);
    }
}

// DT: P8X_I16 (exact ints) or P8X_F32 (int * S), sorted rows, rotated domain
template <int DT>
__global__ __launch_bounds__(kDecThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_decode_rotated(const DecodeArgs a) {
    __shared__ __align__(16) uint32_t tab[kTabWords];
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), hs = lane >> 5, j = lane & 31;
    const uint32_t bankbytes = (uint32_t)(j << 2) * 0x01010101u;
    build_coset_table(tab, a.a2, tid, kDecThreads);
    __syncthreads();
    walk_tiles(a, (size_t)blockIdx.x * kDecWaves + w, (size_t)gridDim.x * kDecWaves, hs, j,
               [&](size_t, int g, int b, int c, const AnySlice<kDecNW> &ls) {
        float v[128];
        lane_values_any<DT == P8X_F32>(c, ls, tab, bankbytes, half_to_float(ls.s), v);
        const size_t o = (size_t)(32 * g + j) * a.ld + 256 * b + 128 * hs;
        if constexpr (DT == P8X_I16) {
            uint2 *dst = reinterpret_cast<uint2 *>((int16_t *)a.out + o);
#pragma unroll
            for (int t = 0; t < 32; ++t) {
                const int *vi = reinterpret_cast<const int *>(v) + 4 * t;
                dst[t] = make_uint2((uint32_t)(uint16_t)vi[0] | ((uint32_t)(uint16_t)vi[1] << 16),
                                    (uint32_t)(uint16_t)vi[2] | ((uint32_t)(uint16_t)vi[3] << 16));
            }
        } else {
            float4 *dst = reinterpret_cast<float4 *>((float *)a.out + o);
#pragma unroll
            for (int t = 0; t < 32; ++t) dst[t] = make_float4(v[4 * t], v[4 * t + 1], v[4 * t + 2], v[4 * t + 3]);
        }
    });
}

// original-domain weights, DT = P8X_F32 / P8X_F16 / P8X_BF16
template <int DT>
__global__ __launch_bounds__(kDecThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_dequant(const DecodeArgs a) {
    __shared__ __align__(16) uint32_t tab[kTabWords];
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), hs = lane >> 5, j = lane & 31;
    const uint32_t bankbytes = (uint32_t)(j << 2) * 0x01010101u;
    build_coset_table(tab, a.a2, tid, kDecThreads);
    __syncthreads();
    walk_tiles(a, (size_t)blockIdx.x * kDecWaves + w, (size_t)gridDim.x * kDecWaves, hs, j,
               [&](size_t, int g, int b, int c, const AnySlice<kDecNW> &ls) {
        float v[128];
        lane_values_any<true>(c, ls, tab, bankbytes, half_to_float(ls.s), v);
#pragma unroll
        for (int h = 1; h < 128; h <<= 1)
#pragma unroll
            for (int i = 0; i < 128; ++i)
                if (!(i & h)) { const float x0 = v[i], x1 = v[i + h]; v[i] = x0 + x1; v[i + h] = x0 - x1; }
#pragma unroll
        for (int i = 0; i < 128; ++i) {   // h = 128: half-slice 0 holds the lower operand
            const float p = __shfl_xor(v[i], 32);
            v[i] = hs ? p - v[i] : v[i] + p;
        }
        const float *icb = a.ic + 256 * b + 128 * hs;
#pragma unroll
        for (int i = 0; i < 128; i += 4) {
            const float4 c4 = *reinterpret_cast<const float4 *>(icb + i);
            v[i] = (v[i] * 0.0625f) * c4.x; v[i + 1] = (v[i + 1] * 0.0625f) * c4.y;
            v[i + 2] = (v[i + 2] * 0.0625f) * c4.z; v[i + 3] = (v[i + 3] * 0.0625f) * c4.w;
        }
        const int ro = a.prm[32 * g + j];
        for (int e = a.cp[ro]; e < a.cp[ro + 1]; ++e) {   // clamp delta (original row, column)
            const int col = (int)a.cc[e] - 256 * b - 128 * hs;
            if (col >= 0 && col < 128) {
                const float dv = a.cv[e];
#pragma unroll
                for (int i = 0; i < 128; ++i) v[i] = i == col ? v[i] + dv : v[i];
            }
        }
        const size_t o = (size_t)ro * a.ld + 256 * b + 128 * hs;
        if constexpr (DT == P8X_F32) {
            float4 *dst = reinterpret_cast<float4 *>((float *)a.out + o);
#pragma unroll
            for (int t = 0; t < 32; ++t) dst[t] = make_float4(v[4 * t], v[4 * t + 1], v[4 * t + 2], v[4 * t + 3]);
        } else {
            uint2 *dst = reinterpret_cast<uint2 *>((uint16_t *)a.out + o);
#pragma unroll
            for (int t = 0; t < 32; ++t) {
                uint16_t hv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (DT == P8X_F16) hv[e] = __builtin_bit_cast(uint16_t, (_Float16)v[4 * t + e]);   // v_cvt_f16_f32, RNE
                    else hv[e] = __builtin_bit_cast(uint16_t, (__bf16)v[4 * t + e]);                            // v_cvt_pk_bf16_f32, RNE
                }
                dst[t] = make_uint2((uint32_t)hv[0] | ((uint32_t)hv[1] << 16), (uint32_t)hv[2] | ((uint32_t)hv[3] << 16));
            }
        }
    });
}

static DecodeArgs decode_args(const p8x_tensor *t, void *out, size_t ld) {
    DecodeArgs a{};
    a.M = t->M; a.S = t->S; a.D = t->D; a.a2 = t->a2; a.prm = t->prm;
    a.ic = t->ic; a.cp = t->cp; a.cc = t->cc; a.cv = t->cv;
    a.out = out; a.ld = ld;
    a.rows = t->rows; a.K = t->K; a.nb = t->nb; a.ng = t->ng; a.nt = t->nt;
    return a;
}

// two 4-wave workgroups per CU (the 64 KB table each), persistent
static int decode_grid(const p8x_tensor *t) {
    const size_t wgs = (t->nt + kDecWaves - 1) / kDecWaves;
    return (int)std::min<size_t>(wgs, (size_t)num_cus() * 2);
}

int launch_decode_rotated(const p8x_tensor *t, int dtype, void *out, size_t ld, hipStream_t st) {
    if (ld % 4) return set_error(P8X_ERR_ARG, "decode: ld %zu must be a multiple of 4", ld);
    const DecodeArgs a = decode_args(t, out, ld);
    if (dtype == P8X_I16) hipLaunchKernelGGL(k_decode_rotated<P8X_I16>, dim3(decode_grid(t)), dim3(kDecThreads), 0, st, a);
    else hipLaunchKernelGGL(k_decode_rotated<P8X_F32>, dim3(decode_grid(t)), dim3(kDecThreads), 0, st, a);
    return hip_check(hipGetLastError(), "k_decode_rotated launch");
}

int launch_dequant(const p8x_tensor *t, int dtype, void *out, size_t ld, hipStream_t st) {
    if (ld % 4) return set_error(P8X_ERR_ARG, "dequantize: ld %zu must be a multiple of 4", ld);
    const DecodeArgs a = decode_args(t, out, ld);
    if (dtype == P8X_F32) hipLaunchKernelGGL(k_dequant<P8X_F32>, dim3(decode_grid(t)), dim3(kDecThreads), 0, st, a);
    else if (dtype == P8X_F16) hipLaunchKernelGGL(k_dequant<P8X_F16>, dim3(decode_grid(t)), dim3(kDecThreads), 0, st, a);
    else hipLaunchKernelGGL(k_dequant<P8X_BF16>, dim3(decode_grid(t)), dim3(kDecThreads), 0, st, a);
    return hip_check(hipGetLastError(), "k_dequant launch");
}

}  // namespace p8x
