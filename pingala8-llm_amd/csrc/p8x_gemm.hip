// p8x_gemm.hip -- prompt-processing GEMM: Y [N][rows] = X [N][K] W^T for a Pingala-8 tensor W.
//
// The 256-point Hadamard rotation of every weight block moves onto the activations:
//   W[prm[r], 256b + c] = (FWHT(v[r, 256b + :] S[b][r]) / 16)[c] ic[256b + c]   (+ clamp delta)
// so  Y[n, prm[r]] = sum_b S[b][r] sum_i v[r, 256b + i] x'[n, 256b + i] + delta terms, with
//   x' = FWHT(x ic) / 16 per 256-block (the GEMV's activation prep, CPU.patch:559-571, kept in fp16 here).
// Pass 1 (k_mm_act) writes x' as fp16 [N][K]. Pass 2 (k_mm): one workgroup of four waves per CU, one wave per
// SIMD; a wave holds NTI x 2 MFMA tiles (32 NTI tokens x 64 weight rows; NTI = 8 or 4 for class-3 tensors, the
// plan's choice, 4 for the every-class kernel). Per 256-block it decodes its two row tiles in chunk order (rotated
// loads, p8x_lane.h) through the LDS coset table straight into MFMA operands (v S, one rounding), each B operand
// feeding NTI v_mfma_f32_32x32x16_f16 with fp32 accumulation, software-pipelined two steps deep with counted LDS
// waits; the block's x' goes through registers into two LDS half-block buffers, written while the other half is
// multiplied. Tokens are the MFMA rows and weight rows its columns, so each lane's outputs run along 32 consecutive
// sorted rows (coalesced buffer stores). Sorted-row planes (one per K split) are then summed in a fixed order,
// un-permuted and given the sparse clamp delta (CPU.patch:1193) on the original activations by k_mm_finish; a
// tensor with identity rows and one K range writes y directly and only adds the delta.
//
// Reference role: ggml_cuda_f44_mul_mat_q8 (CPU.patch:2303-2343), which instead dequantizes the tensor to a
// Q8_0 slab (k_r51_k1, CPU.patch:2138-2235) and calls the stock integer MMQ.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "p8x_internal.h"
#include "p8x_act.h"
#include "p8x_lane.h"

namespace p8x {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));


// ------------------------------------------------------------------------------------------------ pass 1
// x' = FWHT(x ic) / 16 per 256-block, fp16. Lane holds 4 consecutive elements; butterflies h = 1, 2 in the
// lane, 4 .. 128 across lanes (DPP row moves for distances 1-8, lane swaps for 16 and 32). One wave per block,
// kMmActWaves blocks of one token per workgroup.
constexpr int kMmActWaves = 4;
template <typename XT>
__global__ __launch_bounds__(64 * kMmActWaves) void k_mm_act(const XT *__restrict__ x, size_t ldx, const float *__restrict__ ic, int K,
                                                             _Float16 *__restrict__ xr) {
    const int lane = threadIdx.x & 63, b = kMmActWaves * (int)blockIdx.x + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = blockIdx.y;
    if (256 * b >= K) return;
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
    fwht_lane_stage<1>(v, lane);
    fwht_lane_stage<2>(v, lane);
    fwht_lane_stage<4>(v, lane);
    fwht_lane_stage<8>(v, lane);
    fwht_lane_stage<16>(v, lane);
    fwht_lane_stage<32>(v, lane);
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
    const uint32_t *M; const uint16_t *S; const uint32_t *D;
    const _Float16 *xr;     // x' [N][K]
    float *y; unsigned ldy; // direct output (original rows = sorted rows, one K range)
    float *ws;              // sorted-row planes [nsplit][N][rows] otherwise
    const uint32_t *a2;     // [2][256] coset table words (A[f] + h c), h-major, then the same as fp16: entry 2 f + h,
                            // 4 halves
    int N, rows, K, nb, ng;
    int tiles_m, tiles_n, nsplit, kper, direct;
#ifdef P8X_TIMELINE
    unsigned long long *tl;
#endif
};

// offset-binary int8x4 (v + 128 per byte) -> two fp16 pairs holding 1152 + v exactly
__device__ __forceinline__ half2v ob_lo(uint32_t w) { return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u)); }
__device__ __forceinline__ half2v ob_hi(uint32_t w) { return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u)); }

// LDS words of chunk t, all stages (table bytes are A[f] + h c offset by 128)
template <int C, int NWMAX>
__device__ __forceinline__ void lookup_chunk(const AnySlice<NWMAX> &ls, const uint32_t *tab, int t, uint32_t hq, uint32_t (&w)[3]) {
    constexpr int NST = nstage_of(C);
    w[0] = lds_word(tab, ls.template addr<C, 0>(t, hq));
    if constexpr (NST > 1) w[1] = lds_word(tab, ls.template addr<C, 1>(t, hq));
    if constexpr (NST > 2) w[2] = lds_word(tab, ls.template addr<C, 2>(t, hq));
}

// table words of one chunk -> 4 fp16 weights v S (v exact in fp16, |v| <= 1596; one rounding for the product)
template <int C>
__device__ __forceinline__ void weights_chunk(const uint32_t (&w)[3], half2v s2, half2v &lo, half2v &hi) {
    constexpr int NST = nstage_of(C), SH1 = sh1_of(C), SH2 = sh2_of(C);
    const half2v bias = {(_Float16)-1152.f, (_Float16)-1152.f};
    half2v vl = ob_lo(w[0]) + bias, vh = ob_hi(w[0]) + bias;
    if constexpr (NST > 1) {
        const half2v m1 = {(_Float16)(float)(1 << SH1), (_Float16)(float)(1 << SH1)};
        const half2v m2 = {(_Float16)(float)(1 << SH2), (_Float16)(float)(1 << SH2)};
        half2v al = (ob_lo(w[1]) + bias) * m2, ah = (ob_hi(w[1]) + bias) * m2;
        if constexpr (NST > 2) { al += ob_lo(w[2]) + bias; ah += ob_hi(w[2]) + bias; }
        vl = vl * m1 + al;   // integers below 2048: exact in fp16
        vh = vh * m1 + ah;
    }
    lo = vl * s2;
    hi = vh * s2;
}

// classes decoded by an instantiation: the tensor's class set (class 0 decodes as zeros in all of them)
constexpr int kMmCmC3 = 1 << 3, kMmCmAll = 0xFE;
constexpr int kMmMain = 3;   // the class with a branch-free path in every instantiation (the 2-bit bulk)
__host__ __device__ constexpr int mm_nwmax(int cm) { return cm == kMmCmC3 ? 8 : 24; }
// Tile shape (one wave per SIMD, four per workgroup): a wave holds NTI x NTJ MFMA tiles of 32 tokens x 32 weight
// rows, 16 NTI NTJ fp32 accumulators per lane, for all the workgroup's tokens and its own 32 NTJ rows. Each decoded
// B operand feeds NTI MFMAs, so the decode work per MFMA falls as 1 / NTI: the class-3 kernel takes 8 x 2 (256
// tokens x 64 rows, 256 registers, held in the accumulation registers); the every-class kernel, whose decode needs
// more registers, 4 x 2.
// The class-3 kernel comes in two tile shapes, 8 x 2 and 4 x 2 (256 x 256 and 128 x 256 workgroup tiles); the plan
// picks the one with the lower modelled time (the smaller tile halves the K-split planes a shape may need).
__host__ __device__ constexpr int mm_waves() { return 4; }
__host__ __device__ constexpr int mm_ntj() { return 2; }
__host__ __device__ constexpr int mm_rows() { return 32 * mm_ntj() * mm_waves(); }
__host__ __device__ constexpr int mm_tok(int nti) { return 32 * nti; }
// Coset table copies in LDS: the every-class kernel's decode reads 32, one per lane of a half-wave (conflict-free);
// the class-3 kernels keep 16 (lane j reads copy j & 15: word f 32 + h 16 + (j & 15), the 32-copy byte address with
// the lane field doubled, halved), half the table to build per workgroup, and room next to the 8 x 2 shape's two
// 64 KB x' buffers (160 KB of LDS in all).
__host__ __device__ constexpr int mm_tab_words(int cm) { return cm == kMmCmC3 ? kTabWords / 2 : kTabWords; }
__host__ __device__ constexpr int mm_tab_shift(int cm) { return cm == kMmCmC3 ? 1 : 0; }
// The class-3 kernel of the 128-token tile keeps its 16 copies as fp16 instead: entry (f, h, c) = the four weights
// A[f] + h c as fp16 (8 bytes) at byte f 256 + h 128 + 8 c, the 32-copy byte address with the lane field doubled,
// so a lookup is one 8-byte read and the decode of a 4-weight chunk two packed multiplies by S (the offset-binary
// conversion moves into the table build). 64 KB, beside the 128-token tile's two 32 KB x' buffers; the 256-token
// tile's 64 KB buffers leave no room for it.
__host__ __device__ constexpr bool mm_f16_tab(int cm, int nti) { return cm == kMmCmC3 && nti == 4; }
__host__ __device__ constexpr int mm_tab_words(int cm, int nti) { return mm_f16_tab(cm, nti) ? kTabWords : mm_tab_words(cm); }


// x' half-block tile in LDS: half sh of block b holds, per token, columns 128 kh + 64 sh + 8 c8 + (0..7) as
// chunk c = 8 kh + c8 at position c ^ (t & 15) of the token's 256-byte row, so the 16-byte operand reads of
// 16 consecutive tokens cover all 64 banks once. TOK tokens: TOK x 128 halves per buffer.

// Stage half sh of block b in two parts: mm_fetch loads it into registers, mm_put writes it to LDS. With IPW =
// TOK / (4 NWAVES) rows of four tokens per wave, row i of wave w holds token rows 4 (IPW w + i) + (0..3); lane l
// carries token row + (l >> 4), position l & 15 and writes it at the row's LDS base + 16 l bytes. (Direct-to-LDS loads
// would save the registers, but while one may be in flight the compiler waits for every LDS read to finish
// before using any, which serializes the operand reads of consecutive MFMA steps.)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <int NWAVES, int TOK>
struct XStage {
    static constexpr int IPW = TOK / (4 * NWAVES);
    u32x4 v[IPW];   // a native vector type: kept in registers (HIP's uint4 struct made the array a stack object)
};

template <int NWAVES, int TOK>
__device__ __forceinline__ void mm_fetch(const MmJob &J, XStage<NWAVES, TOK> &xs, int tok0, int b, int sh, int w, int lane) {
    constexpr int IPW = XStage<NWAVES, TOK>::IPW;
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
        const int row = 4 * (IPW * w + i), t = row + (lane >> 4);
        const int ts = min(tok0 + t, J.N - 1);   // rows past N repeat the last token (never written out)
        const int c = (lane & 15) ^ (t & 15);
        xs.v[i] = *reinterpret_cast<const u32x4 *>(J.xr + (size_t)ts * J.K + 256 * b + 128 * (c >> 3) + 64 * sh + 8 * (c & 7));
    }
    __asm__ volatile("" ::: "memory");   // issued here, ahead of the products they overlap
}

// rows I0 .. I1 - 1 of the wave's share
template <int NWAVES, int TOK, int I0 = 0, int I1 = XStage<NWAVES, TOK>::IPW>
__device__ __forceinline__ void mm_put(const XStage<NWAVES, TOK> &xs, _Float16 *xb, int w, int lane) {
    constexpr int IPW = XStage<NWAVES, TOK>::IPW;
#pragma unroll
    for (int i = I0; i < I1; ++i) *reinterpret_cast<u32x4 *>(xb + 4 * (IPW * w + i) * 128 + 8 * lane) = xs.v[i];
}

// issue the raw payload loads of the wave's NTJ tiles at block b
template <int CM, int NWMAX, int NTJ>
__device__ __forceinline__ void mm_issue(const MmJob &J, AnyRaw<NWMAX> (&raw)[NTJ], int (&cl)[NTJ], const int (&g)[NTJ], int b, int j, int kh) {
#pragma unroll
    for (int tj = 0; tj < NTJ; ++tj) {
        cl[tj] = 0;
        if constexpr (CM == kMmCmC3) {   // the class-3-only path decodes every tile; zero weights through S = 0
#pragma unroll
            for (int i = 0; i < NWMAX; ++i) raw[tj].w[i] = 0;
            raw[tj].s = 0;
        }
        if (g[tj] < J.ng) {
            const uint32_t mt = as_const(J.M)[(size_t)g[tj] * J.nb + b];   // scalar load: not counted with the x' loads
            cl[tj] = (int)(mt >> 29);
            load_any<CM>(raw[tj], cl[tj], J.D + (mt & 0x1FFFFFFFu) + kh * nw_of(cl[tj]) * 32, j, J.S + (size_t)b * J.rows + 32 * g[tj]);
        }
    }
}

// decode the raw words into the slices the products read (after the loads have landed)
template <int CM, int NWMAX, int NTJ>
__device__ __forceinline__ void mm_prepare(AnySlice<NWMAX> (&ls)[NTJ], const int (&cl)[NTJ], const AnyRaw<NWMAX> (&raw)[NTJ]) {
#pragma unroll
    for (int tj = 0; tj < NTJ; ++tj) {
        if constexpr (CM == kMmCmC3) ls[tj].template from_raw<3>(raw[tj]);   // zero raw words, S = 0: zero weights
        else prepare_any<CM>(ls[tj], cl[tj], raw[tj]);
    }
}

// The 8 steps of one half-block for row tile TJ alone, its class C fixed: the same two-deep pipeline as the both-tiles
// path of mm_half (table words two steps ahead, B one step ahead), NTI MFMAs per step. Every-class kernel, for a
// half-block whose two tiles are not both class 3: one compact loop per (class, tile) instead of a class switch in
// every step (whose code for all classes exceeded the instruction cache).
template <int C, int TJ, int NWMAX, int NTI, int NTJ>
__device__ __forceinline__ void mm_tile_pass(const _Float16 *__restrict__ xb, const AnySlice<NWMAX> &ls, const uint32_t *tab, uint32_t bankbytes,
                                             int sh, int j, int kh, float16v (&acc)[NTI][NTJ]) {
    const half2v s2 = {__builtin_bit_cast(_Float16, (uint16_t)ls.s), __builtin_bit_cast(_Float16, (uint16_t)ls.s)};
    auto read_a = [&](int s8, half8v (&A)[NTI]) {
#pragma unroll
        for (int ti = 0; ti < NTI; ++ti)
            A[ti] = *reinterpret_cast<const half8v *>(xb + (32 * ti + j) * 128 + 8 * ((8 * kh + s8) ^ (j & 15)));
    };
    auto lookups = [&](int s, uint32_t (&W)[2][3]) {
        const uint32_t hq = coset_bytes(ls.H, bankbytes, s >> 1);
        lookup_chunk<C>(ls, tab, 2 * s, hq, W[0]);
        lookup_chunk<C>(ls, tab, 2 * s + 1, hq, W[1]);
    };
    auto decode = [&](const uint32_t (&W)[2][3]) {
        half2v a, b, c, d;
        weights_chunk<C>(W[0], s2, a, b);
        weights_chunk<C>(W[1], s2, c, d);
        half8v o;
        o[0] = a.x; o[1] = a.y; o[2] = b.x; o[3] = b.y; o[4] = c.x; o[5] = c.y; o[6] = d.x; o[7] = d.y;
        return o;
    };
    uint32_t W[2][3];
    lookups(8 * sh, W);
    half8v B = decode(W), A[NTI];
    read_a(0, A);
    lookups(8 * sh + 1, W);
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) {
        half8v An[NTI], Bn;
        uint32_t Wn[2][3];
        if (s8 < 7) { Bn = decode(W); read_a(s8 + 1, An); }
        if (s8 < 6) lookups(8 * sh + s8 + 2, Wn);
#pragma unroll
        for (int ti = 0; ti < NTI; ++ti) acc[ti][TJ] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[ti], B, acc[ti][TJ], 0, 0, 0);
        if (s8 < 7) {
            B = Bn;
#pragma unroll
            for (int ti = 0; ti < NTI; ++ti) A[ti] = An[ti];
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int q = 0; q < 3; ++q) W[u][q] = Wn[u][q];
        }
    }
}

// row tile TJ's half-block in the pass for its class (class 0: zero weights, nothing to add)
template <int CM, int TJ, int NWMAX, int NTI, int NTJ>
__device__ __forceinline__ void mm_tile_any(int c, const _Float16 *__restrict__ xb, const AnySlice<NWMAX> &ls, const uint32_t *tab, uint32_t bankbytes,
                                            int sh, int j, int kh, float16v (&acc)[NTI][NTJ]) {
    switch (c) {
        case 1: if constexpr ((CM >> 1) & 1) mm_tile_pass<1, TJ>(xb, ls, tab, bankbytes, sh, j, kh, acc); break;
        case 2: if constexpr ((CM >> 2) & 1) mm_tile_pass<2, TJ>(xb, ls, tab, bankbytes, sh, j, kh, acc); break;
        case 3: if constexpr ((CM >> 3) & 1) mm_tile_pass<3, TJ>(xb, ls, tab, bankbytes, sh, j, kh, acc); break;
        case 4: if constexpr ((CM >> 4) & 1) mm_tile_pass<4, TJ>(xb, ls, tab, bankbytes, sh, j, kh, acc); break;
        case 5: if constexpr ((CM >> 5) & 1) mm_tile_pass<5, TJ>(xb, ls, tab, bankbytes, sh, j, kh, acc); break;
        case 6: if constexpr ((CM >> 6) & 1) mm_tile_pass<6, TJ>(xb, ls, tab, bankbytes, sh, j, kh, acc); break;
        case 7: if constexpr ((CM >> 7) & 1) mm_tile_pass<7, TJ>(xb, ls, tab, bankbytes, sh, j, kh, acc); break;
        default: break;
    }
}

// The 8 MFMA steps of one half-block (steps s = 8 sh .. 8 sh + 7) from x' buffer xb; the staged x' of the next
// half-block goes to the other buffer xn during them (no wave reads xn between the barriers around this call).
template <int CM, int NWMAX, int NTI, int NTJ, int NWAVES, int TOK>
__device__ __forceinline__ void mm_half(const _Float16 *__restrict__ xb, const AnySlice<NWMAX> (&ls)[NTJ], const int (&cl)[NTJ], const uint32_t *tab,
                                        uint32_t bankbytes, int sh, int j, int kh, float16v (&acc)[NTI][NTJ],
                                        const XStage<NWAVES, TOK> &xq, _Float16 *xn, int w, int lane) {
    constexpr int IPW = XStage<NWAVES, TOK>::IPW, PPS = IPW / 4;   // x' rows written per step, in the last 4 steps
    static_assert(IPW % 4 == 0, "x' rows per wave split over 4 steps");
    auto read_a = [&](int s8, half8v (&A)[NTI]) {
#pragma unroll
        for (int ti = 0; ti < NTI; ++ti)
            A[ti] = *reinterpret_cast<const half8v *>(xb + (32 * ti + j) * 128 + 8 * ((8 * kh + s8) ^ (j & 15)));
    };
    bool main_only = true;
    if constexpr (CM != kMmCmC3) {
#pragma unroll
        for (int tj = 0; tj < NTJ; ++tj) main_only = main_only && cl[tj] == kMmMain;
    }
    if (main_only) {
        // Software-pipelined in two depths. While the NTI NTJ MFMAs of step s run, the first half of them interleaved
        // with the decode of step s + 1's B operands (table words read one step earlier), the second half with the
        // x' reads of step s + 1 and the table reads of step s + 2. At most NTI + 2 NTJ = 12 LDS reads are in
        // flight, within what the wait counter tracks, so each wait is counted: the MFMAs wait only for their own
        // x' operands.
        half2v s2[NTJ];
#pragma unroll
        for (int tj = 0; tj < NTJ; ++tj) s2[tj] = half2v{__builtin_bit_cast(_Float16, (uint16_t)ls[tj].s), __builtin_bit_cast(_Float16, (uint16_t)ls[tj].s)};
        constexpr bool F16T = mm_f16_tab(CM, NTI);
        auto lookups = [&](int s, uint32_t (&W)[NTJ][2][3]) {
#pragma unroll
            for (int tj = 0; tj < NTJ; ++tj) {
                const uint32_t hq = coset_bytes(ls[tj].H, bankbytes, s >> 1);
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const uint32_t a = ls[tj].template addr<kMmMain, 0>(2 * s + u, hq);
                    if constexpr (F16T) {   // the chunk's four fp16 weights
                        const uint2 v = *reinterpret_cast<const uint2 *>(reinterpret_cast<const char *>(tab) + a);
                        W[tj][u][0] = v.x;
                        W[tj][u][1] = v.y;
                    } else {
                        W[tj][u][0] = lds_word(tab, a >> mm_tab_shift(CM));
                    }
                }
            }
        };
        auto decode = [&](const uint32_t (&W)[NTJ][2][3], half8v (&B)[NTJ]) {
#pragma unroll
            for (int tj = 0; tj < NTJ; ++tj) {
                half2v a, b, c, d;
                if constexpr (F16T) {
                    a = __builtin_bit_cast(half2v, W[tj][0][0]) * s2[tj];
                    b = __builtin_bit_cast(half2v, W[tj][0][1]) * s2[tj];
                    c = __builtin_bit_cast(half2v, W[tj][1][0]) * s2[tj];
                    d = __builtin_bit_cast(half2v, W[tj][1][1]) * s2[tj];
                } else {
                    weights_chunk<kMmMain>(W[tj][0], s2[tj], a, b);
                    weights_chunk<kMmMain>(W[tj][1], s2[tj], c, d);
                }
                B[tj][0] = a.x; B[tj][1] = a.y; B[tj][2] = b.x; B[tj][3] = b.y;
                B[tj][4] = c.x; B[tj][5] = c.y; B[tj][6] = d.x; B[tj][7] = d.y;
            }
        };
        static_assert(nstage_of(kMmMain) == 1, "the main path reads one table word per chunk");
        half8v A[NTI], B[NTJ];
        uint32_t W[NTJ][2][3];
        lookups(8 * sh, W);
        decode(W, B);
        read_a(0, A);
        lookups(8 * sh + 1, W);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8) {
            half8v An[NTI], Bn[NTJ];
            uint32_t Wn[NTJ][2][3];
            if (s8 < 7) decode(W, Bn);
            if (s8 < 7) read_a(s8 + 1, An);
            if (s8 < 6) lookups(8 * sh + s8 + 2, Wn);
#pragma unroll
            for (int tj = 0; tj < NTJ; ++tj)
#pragma unroll
                for (int ti = 0; ti < NTI; ++ti) acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[ti], B[tj], acc[ti][tj], 0, 0, 0);
            if (s8 >= 4) {
                // the next half-block's x' rows (loaded since the start of this half-block) go to the other buffer
#pragma unroll
                for (int i = 0; i < PPS; ++i)
                    *reinterpret_cast<u32x4 *>(xn + 4 * (IPW * w + (s8 - 4) * PPS + i) * 128 + 8 * lane) = xq.v[(s8 - 4) * PPS + i];
            }
            if (s8 < 7) {
                constexpr int HM = NTI * NTJ / 2;                          // MFMAs per half of the step
                constexpr int DV = ((F16T ? 4 : 12) * NTJ + HM - 1) / HM;  // decode VALU per MFMA
                constexpr int RD = (NTI + 2 * NTJ + HM - 1) / HM;          // LDS reads per MFMA
#pragma unroll
                for (int i = 0; i < HM; ++i) {   // decode
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, DV, 0);
                }
#pragma unroll
                for (int i = 0; i < HM; ++i) {   // x' and table reads, table addresses, x' writes
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                    if (s8 >= 4 && i < PPS) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
                }
#pragma unroll
                for (int ti = 0; ti < NTI; ++ti) A[ti] = An[ti];
#pragma unroll
                for (int tj = 0; tj < NTJ; ++tj) {
                    B[tj] = Bn[tj];
#pragma unroll
                    for (int u = 0; u < 2; ++u)
#pragma unroll
                        for (int q = 0; q < 3; ++q) W[tj][u][q] = Wn[tj][u][q];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    } else if constexpr (CM != kMmCmC3) {
        static_assert(NTJ == 2, "one pass per row tile");
        mm_tile_any<CM, 0>(cl[0], xb, ls[0], tab, bankbytes, sh, j, kh, acc);
        mm_tile_any<CM, 1>(cl[1], xb, ls[1], tab, bankbytes, sh, j, kh, acc);
        mm_put<NWAVES, TOK>(xq, xn, w, lane);
    }
}

// One workgroup per CU of mm_waves() waves, one per SIMD (each: 32 NTJ weight rows x all 32 NTI tokens of the
// workgroup tile). K advances by half-blocks; the x' of the next half-block and the next block's payload are in flight
// while the current half-block is multiplied.
template <int CM, int NTI>
__global__ __launch_bounds__(64 * mm_waves()) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_mm(MmJob J) {
    constexpr int NWMAX = mm_nwmax(CM), NWAVES = mm_waves(), NTJ = mm_ntj(), kMmThreads = 64 * NWAVES;
    constexpr int kMmRows = mm_rows(), TOK = mm_tok(NTI), TABW = mm_tab_words(CM, NTI);
    constexpr bool F16T = mm_f16_tab(CM, NTI);
    __shared__ uint32_t tab[TABW];   // first: LDS address 0, replicated coset table (bytes offset by 128, or fp16)
    __shared__ __attribute__((aligned(16))) _Float16 xs0[TOK * 128];   // half 0 of a block
    __shared__ __attribute__((aligned(16))) _Float16 xs1[TOK * 128];   // half 1
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31, kh = lane >> 5;
    // lane field of the table byte addresses: the lane's copy, at the 32-copy spacing (halved on read for 16 copies)
    const uint32_t bankbytes = (uint32_t)((TABW == kTabWords && !F16T ? j : (j & 15) << 1) << 2) * 0x01010101u;
#ifdef P8X_TIMELINE
    const unsigned long long tl_start = __builtin_amdgcn_s_memrealtime();
#endif
    // Workgroups are dealt to the 8 XCDs round-robin (XCD = blockIdx % 8). Linear tile order is x'-slice-major
    // (slice = token tile x K split, then row tile), and each XCD takes one contiguous run of it, so the
    // workgroups that read one x' slice share an L2.
    const int per = (J.tiles_m * J.tiles_n * J.nsplit + kXcds - 1) / kXcds;
    const int lin = (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
    if (lin >= J.tiles_m * J.tiles_n * J.nsplit) return;
    const int tm = lin % J.tiles_m, slice = lin / J.tiles_m;
    const int ks = slice % J.nsplit, tn = slice / J.nsplit;
    const int tok0 = tn * TOK;
    const int b0 = ks * J.kper, b1 = min(J.nb, b0 + J.kper);
    int g[NTJ];
#pragma unroll
    for (int tj = 0; tj < NTJ; ++tj) g[tj] = (tm * kMmRows) / 32 + NTJ * w + tj;
    float16v acc[NTI][NTJ];
#pragma unroll
    for (int ti = 0; ti < NTI; ++ti)
#pragma unroll
        for (int tj = 0; tj < NTJ; ++tj) acc[ti][tj] = float16v{};
    AnySlice<NWMAX> ls[NTJ];
    AnyRaw<NWMAX> raw[NTJ];
    int cl[NTJ], ncl[NTJ];
    // the first half-block and payload loads go out first; the table is built while they are in flight
    XStage<NWAVES, TOK> xq;
    mm_fetch<NWAVES, TOK>(J, xq, tok0, b0, 0, w, lane);
    mm_issue<CM>(J, raw, cl, g, b0, j, kh);
    // the table build: every thread's loads first, then its stores (one memory round trip, not one per piece)
    constexpr int TPT = TABW / 4 / kMmThreads;   // 16-byte pieces per thread
    static_assert(TABW / 4 % kMmThreads == 0, "whole pieces per thread");
    uint4 *t4 = reinterpret_cast<uint4 *>(tab);
    if constexpr (F16T) {
        // 16-byte piece i = copies 2 (i % 8), 2 (i % 8) + 1 of entry 2 f + h = i / 8: the four A[f] + h c as fp16
        // (the fp16 entries the tensor's tables carry after the words)
        const uint2 *e16 = reinterpret_cast<const uint2 *>(J.a2 + 512);
        uint2 v[TPT];
#pragma unroll
        for (int k = 0; k < TPT; ++k) v[k] = e16[(tid + k * kMmThreads) >> 3];
#pragma unroll
        for (int k = 0; k < TPT; ++k) t4[tid + k * kMmThreads] = make_uint4(v[k].x, v[k].y, v[k].x, v[k].y);
    } else {
        // word (f, h, c) = A[f] + h c bytes (offset by 128) at f (TABW / 256) + h (TABW / 512) + c, c < TABW / 512
        constexpr int CPS = TABW / 512;   // copies
        uint32_t v[TPT];
#pragma unroll
        for (int k = 0; k < TPT; ++k) {
            const int i = tid + k * kMmThreads, f = (4 * i) / (2 * CPS), h = ((4 * i) / CPS) & 1;
            v[k] = J.a2[h * 256 + f] ^ 0x80808080u;
        }
#pragma unroll
        for (int k = 0; k < TPT; ++k) t4[tid + k * kMmThreads] = make_uint4(v[k], v[k], v[k], v[k]);
    }
    mm_put<NWAVES, TOK>(xq, xs0, w, lane);
    mm_prepare<CM>(ls, cl, raw);
    __syncthreads();   // table and the first half-block's x' are in LDS
#ifdef P8X_TIMELINE
    // Timeline build: s_memrealtime (100 MHz) per wave at its start, after the prologue, summed over the
    // half-blocks (products; x' write and barrier), at the loop's end and after its stores have completed:
    // record [8] = {lin << 32 | wave << 16 | blocks, start, prologue, products, barriers, loop end, end, grid}
    unsigned long long tl_t = __builtin_amdgcn_s_memrealtime(), tl_cmp = 0, tl_bar = 0;
    const unsigned long long tl_pro = tl_t;
#define P8X_MM_LAP(sum) do { const unsigned long long t_ = __builtin_amdgcn_s_memrealtime(); sum += t_ - tl_t; tl_t = t_; } while (0)
#else
#define P8X_MM_LAP(sum) do {} while (0)
#endif
    // Half h + 1 is fetched into registers while half h is multiplied, then written to the other buffer (which no
    // wave reads since the last barrier); the next block's payload stays in flight through the second half.
    // The loads are unconditional (the last block's successor is the last block again, never used), so the wait
    // counts the compiler derives for the x' writes inside mm_half are exact.
    for (int b = b0; b < b1; ++b) {
        const int bn = min(b + 1, b1 - 1);
        mm_fetch<NWAVES, TOK>(J, xq, tok0, b, 1, w, lane);
        mm_issue<CM>(J, raw, ncl, g, bn, j, kh);
        mm_half<CM>(xs0, ls, cl, tab, bankbytes, 0, j, kh, acc, xq, xs1, w, lane);
        P8X_MM_LAP(tl_cmp);
        __syncthreads();
        P8X_MM_LAP(tl_bar);
        mm_fetch<NWAVES, TOK>(J, xq, tok0, bn, 0, w, lane);
        mm_half<CM>(xs1, ls, cl, tab, bankbytes, 1, j, kh, acc, xq, xs0, w, lane);
        P8X_MM_LAP(tl_cmp);
#pragma unroll
        for (int tj = 0; tj < NTJ; ++tj) cl[tj] = ncl[tj];
        mm_prepare<CM>(ls, cl, raw);
        __syncthreads();
        P8X_MM_LAP(tl_bar);
    }
#ifdef P8X_TIMELINE
    const unsigned long long tl_loop = tl_t;
#endif
    // acc[ti][tj] lane l, reg q: token 32 ti + 8 (q >> 2) + 4 kh + (q & 3), sorted row 32 g[tj] + j: 32 lanes
    // store 32 consecutive rows of one token (planes, or y with identity rows; scattered 4-byte stores to the
    // original rows measured 5x slower than a plane and k_mm_finish)
    float *dst = J.direct ? J.y : J.ws + (size_t)ks * J.N * J.rows;
    const size_t ld = J.direct ? (size_t)J.ldy : (size_t)J.rows;
    if ((size_t)J.N * ld * 4 < 0xFFFFFFFFull) {
        // Buffer stores with 32-bit offsets, no branches. In a tile that runs past N, a token at or past N is
        // stored to token N - 1, whose value it holds bit for bit (its x' row repeats row N - 1, and each MFMA
        // output element is computed alike), so every store stays inside the N ld floats of the resource.
        const __amdgpu_buffer_rsrc_t rd = buffer_rsrc(dst, (uint32_t)((size_t)J.N * ld * 4));
        const uint32_t ld4 = (uint32_t)ld * 4u;
        const bool whole = tok0 + TOK <= J.N;
#pragma unroll
        for (int tj = 0; tj < NTJ; ++tj) {
            if (g[tj] >= J.ng) continue;
            const uint32_t r4 = (uint32_t)(32 * g[tj] + j) * 4u;
#pragma unroll
            for (int ti = 0; ti < NTI; ++ti)
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int tok = tok0 + 32 * ti + 8 * (q >> 2) + 4 * kh + (q & 3);
                    const uint32_t off = (uint32_t)(whole ? tok : min(tok, J.N - 1)) * ld4 + r4;
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[ti][tj][q]), rd, off, 0, 0);
                }
        }
    } else {
#pragma unroll
        for (int tj = 0; tj < NTJ; ++tj) {
            if (g[tj] >= J.ng) continue;
            const int r = 32 * g[tj] + j;
#pragma unroll
            for (int ti = 0; ti < NTI; ++ti)
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int tok = tok0 + 32 * ti + 8 * (q >> 2) + 4 * kh + (q & 3);
                    if (tok < J.N) dst[(size_t)tok * ld + r] = acc[ti][tj][q];
                }
        }
    }
#ifdef P8X_TIMELINE
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const unsigned long long tl_end = __builtin_amdgcn_s_memrealtime();
    if (lane == 0 && (unsigned)(4 * blockIdx.x + w) < kTimelineRecords) {
        const unsigned slot = __hip_atomic_fetch_add((unsigned *)(J.tl + kTimelineRecords * 8), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (slot < kTimelineRecords) {
            unsigned long long *o = J.tl + (size_t)slot * 8;
            o[0] = ((unsigned long long)lin << 32) | ((unsigned)w << 16) | (unsigned)(b1 - b0);
            o[1] = tl_start; o[2] = tl_pro; o[3] = tl_cmp; o[4] = tl_bar; o[5] = tl_loop; o[6] = tl_end; o[7] = gridDim.x;
        }
    }
#endif
}
#undef P8X_MM_LAP

// y[n][ro] = sum over K splits (split order) of the sorted planes at row pinv[ro], plus the clamp delta on the
// original activations. One workgroup per token: the planes are read coalesced into LDS (sorted order), the
// un-permute gathers from LDS, the stores are coalesced.
template <typename XT>
__global__ __launch_bounds__(1024) void k_mm_finish(const float *__restrict__ ws, int nsplit, int N, int rows, const int16_t *__restrict__ pinv,
                                                    const int *__restrict__ cp, const uint16_t *__restrict__ cc, const float *__restrict__ cv,
                                                    const XT *__restrict__ x, size_t ldx, float *__restrict__ y, size_t ldy) {
    extern __shared__ float srow[];   // [rows]
    const int n = blockIdx.x;
    for (int r = threadIdx.x; r < rows; r += 1024) {
        float v = 0.f;
        for (int k = 0; k < nsplit; ++k) v += ws[((size_t)k * N + n) * rows + r];
        srow[r] = v;
    }
    __syncthreads();
    const XT *xr = x + (size_t)n * ldx;
    for (int ro = threadIdx.x; ro < rows; ro += 1024) {
        float v = srow[pinv[ro]];
        for (int e = cp[ro]; e < cp[ro + 1]; ++e) {
            float xv;
            if constexpr (sizeof(XT) == 4) xv = xr[cc[e]];
            else xv = bf16_to_float((uint16_t)xr[cc[e]]);
            v += cv[e] * xv;
        }
        y[(size_t)n * ldy + ro] = v;
    }
}

// clamp delta alone (direct output): y[n][row] += sum_e cv[e] x[n][cc[e]] for the rows that have entries
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
    int nti;   // token tiles per wave: the workgroup tile is 256 rows x 32 nti tokens
    int tiles_m, tiles_n, nsplit, kper;
};

// One workgroup per CU. Estimated time = rounds of workgroups x (the measured prologue + blocks per workgroup x the
// measured time of one K block of a workgroup tile of the shape) + when planes are used (K split, or rows to
// un-permute) their traffic (written by k_mm, read by k_mm_finish at ~5 TB/s) and k_mm_finish's launch.
static bool mm_only_c3(const p8x_tensor *t) {
    for (int c = 1; c < 8; ++c) if (c != 3 && t->class_tiles[c]) return false;
    return true;
}

static MmPlan mm_plan(const p8x_tensor *t, int N) {
    const bool c3 = mm_only_c3(t);
    const long slots = num_cus();
    const double plane_us = 2.0 * 4.0 * N * t->rows / 5e6, finish_us = 3.0;
    // a split's planes stay within what the no-allocation entry point holds next to x', so that it runs the same
    // plan (and returns the same bits) as p8x_mul_mat wherever it runs at all
    const size_t xb = ((size_t)N * t->K * sizeof(_Float16) + 255) & ~(size_t)255;
    const size_t cap = xb < (size_t)P8X_NOALLOC_SCRATCH_BYTES ? (size_t)P8X_NOALLOC_SCRATCH_BYTES - xb : 0;
    MmPlan best{4, 0, 0, 1, t->nb};
    double best_cost = -1.0;
    for (int nti = 8; nti >= 4; nti -= 4) {
        if (nti == 8 && !c3) continue;   // the every-class decode needs the registers of the 4 x 2 shape
        // one K block of one workgroup tile and the prologue, us (class 3: 256 x 256 and 256 x 128 measured; every
        // class: 256 x 128)
        const double block_us = nti == 8 ? 7.5 : c3 ? 3.9 : 4.4, pro_us = c3 ? 3.7 : 5.0;
        const int tiles_m = (t->rows + mm_rows() - 1) / mm_rows(), tiles_n = (N + mm_tok(nti) - 1) / mm_tok(nti);
        const long base = (long)tiles_m * tiles_n;
        for (int ns = 1; ns <= std::min(t->nb, 16); ++ns) {
            const int kper = (t->nb + ns - 1) / ns, nsr = (t->nb + kper - 1) / kper;
            if (nsr > 1 && (size_t)nsr * N * t->rows * 4 > cap) continue;
            const bool planes = nsr > 1 || !t->prm_identity;
            const double cost = (double)((base * nsr + slots - 1) / slots) * (pro_us + kper * block_us) + (planes ? nsr * plane_us + finish_us : 0.0);
            if (best_cost < 0 || cost < best_cost) { best_cost = cost; best = MmPlan{nti, tiles_m, tiles_n, nsr, kper}; }
        }
    }
    return best;
}

int reserve_mul_mat(const p8x_tensor *t, int n_max) {
    p8x_tensor *tw = const_cast<p8x_tensor *>(t);
    int rc;
    if ((rc = grow((void **)&tw->wx16, &tw->wx16_elems, (size_t)n_max * t->K * sizeof(_Float16), "p8x_mul_mat_reserve: activation workspace"))) return rc;
    size_t planes = 0;   // the largest plane need over every N <= n_max (the split count depends on N)
    for (int n = 1; n <= n_max; ++n) {
        const MmPlan p = mm_plan(t, n);
        if (!(p.nsplit == 1 && t->prm_identity)) planes = std::max(planes, (size_t)p.nsplit * n * t->rows * 4);
    }
    if (planes && (rc = grow((void **)&tw->wmm, &tw->wmm_bytes, planes, "p8x_mul_mat_reserve: output planes"))) return rc;
    return P8X_OK;
}

// workspace bytes of one prompt GEMM call: rotated fp16 activations [N][K], and (K split or rows to un-permute) the
// sorted-row output planes [nsplit][N][rows] f32
static void mm_workspace(const p8x_tensor *t, int N, size_t *x_bytes, size_t *plane_bytes) {
    const MmPlan p = mm_plan(t, N);
    *x_bytes = (size_t)N * t->K * sizeof(_Float16);
    *plane_bytes = p.nsplit == 1 && t->prm_identity ? 0 : (size_t)p.nsplit * N * t->rows * 4;
}

// k_mm_finish keeps a row of the output (up to 128 KB) in dynamic LDS. The attribute that allows it is per device:
// set once on each device this process launches on (callers on several threads serialize here).
static int finish_lds_attribute() {
    int dev = 0;
    int rc = hip_check(hipGetDevice(&dev), "k_mm_finish attribute: hipGetDevice");
    if (rc) return rc;
    static std::mutex mu;
    static std::vector<char> done;
    std::lock_guard<std::mutex> lock(mu);
    if ((size_t)dev >= done.size()) done.resize((size_t)dev + 1, 0);
    if (done[dev]) return P8X_OK;
    if ((rc = hip_check(hipFuncSetAttribute((const void *)k_mm_finish<float>, hipFuncAttributeMaxDynamicSharedMemorySize, 131072), "k_mm_finish attribute")) ||
        (rc = hip_check(hipFuncSetAttribute((const void *)k_mm_finish<uint16_t>, hipFuncAttributeMaxDynamicSharedMemorySize, 131072), "k_mm_finish attribute")))
        return rc;
    done[dev] = 1;
    return P8X_OK;
}

// the launches of one prompt GEMM with its workspace given: xr >= N K fp16, wmm >= the plane bytes (unused when the
// output is written directly)

static int launch_mul_mat_ws(const p8x_tensor *t, const void *x, int x_dtype, int N, size_t ldx, float *y, size_t ldy, _Float16 *xr,
                             float *wmm, hipStream_t st) {
    const MmPlan p = mm_plan(t, N);
    const bool direct = p.nsplit == 1 && t->prm_identity;
    int rc;
    const dim3 agrid((t->nb + kMmActWaves - 1) / kMmActWaves, N);
    if (x_dtype == P8X_F32) hipLaunchKernelGGL(k_mm_act<float>, agrid, dim3(64 * kMmActWaves), 0, st, (const float *)x, ldx, t->ic, t->K, xr);
    else hipLaunchKernelGGL(k_mm_act<uint16_t>, agrid, dim3(64 * kMmActWaves), 0, st, (const uint16_t *)x, ldx, t->ic, t->K, xr);
    if ((rc = hip_check(hipGetLastError(), "k_mm_act launch"))) return rc;
    MmJob J;
    J.M = t->M; J.S = t->S; J.D = t->D; J.xr = xr;
    J.y = y; J.ldy = (unsigned)ldy; J.ws = wmm; J.a2 = t->a2;
    J.N = N; J.rows = t->rows; J.K = t->K; J.nb = t->nb; J.ng = t->ng;
    J.tiles_m = p.tiles_m; J.tiles_n = p.tiles_n; J.nsplit = p.nsplit; J.kper = p.kper; J.direct = direct;
#ifdef P8X_TIMELINE
    J.tl = timeline_buf();
#endif
    const int grid = ((p.tiles_m * p.tiles_n * p.nsplit + kXcds - 1) / kXcds) * kXcds;
    if (!mm_only_c3(t)) hipLaunchKernelGGL((k_mm<kMmCmAll, 4>), dim3(grid), dim3(64 * mm_waves()), 0, st, J);
    else if (p.nti == 8) hipLaunchKernelGGL((k_mm<kMmCmC3, 8>), dim3(grid), dim3(64 * mm_waves()), 0, st, J);
    else hipLaunchKernelGGL((k_mm<kMmCmC3, 4>), dim3(grid), dim3(64 * mm_waves()), 0, st, J);
    if ((rc = hip_check(hipGetLastError(), "k_mm launch"))) return rc;
    if (!direct) {
        const size_t lds = 4 * (size_t)t->rows;   // rows < 32768: at most 128 KB
        if ((rc = finish_lds_attribute())) return rc;
        if (x_dtype == P8X_F32)
            hipLaunchKernelGGL(k_mm_finish<float>, dim3(N), dim3(1024), lds, st, (const float *)wmm, p.nsplit, N, t->rows, t->pinv, t->cp, t->cc, t->cv,
                               (const float *)x, ldx, y, ldy);
        else
            hipLaunchKernelGGL(k_mm_finish<uint16_t>, dim3(N), dim3(1024), lds, st, (const float *)wmm, p.nsplit, N, t->rows, t->pinv, t->cp, t->cc, t->cv,
                               (const uint16_t *)x, ldx, y, ldy);
        return hip_check(hipGetLastError(), "k_mm_finish launch");
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

int launch_mul_mat(const p8x_tensor *t, const void *x, int x_dtype, int N, size_t ldx, float *y, size_t ldy, hipStream_t st) {
    if (((uintptr_t)x & 15) || (ldx % 8)) return set_error(P8X_ERR_ARG, "p8x_mul_mat: x must be 16-byte aligned with ldx %% 8 == 0");
    p8x_tensor *tw = const_cast<p8x_tensor *>(t);
    size_t xb, pb;
    mm_workspace(t, N, &xb, &pb);
    int rc;
    if ((rc = grow((void **)&tw->wx16, &tw->wx16_elems, xb, "p8x_mul_mat: activation workspace"))) return rc;
    if (pb && (rc = grow((void **)&tw->wmm, &tw->wmm_bytes, pb, "p8x_mul_mat: output planes"))) return rc;
    return launch_mul_mat_ws(t, x, x_dtype, N, ldx, y, ldy, reinterpret_cast<_Float16 *>(tw->wx16), tw->wmm, st);
}

// ------------------------------------------------------------------------------------------------ no-allocation variant
// Workspace of p8x_mul_mat_noalloc: one file-scope device array per GPU, held until the process ends. In host code
// `scratch` names a host-side stand-in; the device address of each GPU's copy comes from hipGetSymbolAddress with
// that GPU current, resolved once per device (scratch_resolve) and used everywhere host code passes the array on.
static __device__ __align__(256) uint8_t scratch[P8X_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch[kMaxDevices];

int scratch_resolve(int device) {
    if (device < 0 || device >= kMaxDevices) return set_error(P8X_ERR_UNSUPPORTED, "scratch: device %d beyond %d", device, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch[device]) return P8X_OK;
    int cur = 0, rc;
    if ((rc = hip_check(hipGetDevice(&cur), "scratch: hipGetDevice"))) return rc;
    if (cur != device && (rc = hip_check(hipSetDevice(device), "scratch: hipSetDevice"))) return rc;
    void *ptr = nullptr;
    rc = hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "scratch: hipGetSymbolAddress");
    if (cur != device) (void)hipSetDevice(cur);
    if (rc) return rc;
    g_scratch[device] = ptr;
    return P8X_OK;
}

static void *scratch_ptr(int device) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return device >= 0 && device < kMaxDevices ? g_scratch[device] : nullptr;
}

}  // namespace p8x

extern "C" int p8x_mul_mat_noalloc(const p8x_tensor *t, const void *x, int x_dtype, int N, size_t ldx, float *y, size_t ldy, void *stream) {
    using namespace p8x;
    if (!t || !x || !y) return set_error(P8X_ERR_ARG, "p8x_mul_mat_noalloc: null pointer");
    if (x_dtype != P8X_F32 && x_dtype != P8X_BF16) return set_error(P8X_ERR_ARG, "p8x_mul_mat_noalloc: x dtype %d", x_dtype);
    if (N < 1 || ldx < (size_t)t->K || ldy < (size_t)t->rows) return set_error(P8X_ERR_ARG, "p8x_mul_mat_noalloc: N %d ldx %zu ldy %zu", N, ldx, ldy);
    if (((uintptr_t)x & 15) || (ldx % 8)) return set_error(P8X_ERR_ARG, "p8x_mul_mat_noalloc: x must be 16-byte aligned with ldx %% 8 == 0");
    size_t xb, pb;
    mm_workspace(t, N, &xb, &pb);
    const size_t xb_al = (xb + 255) & ~(size_t)255;
    if (xb_al + pb > (size_t)P8X_NOALLOC_SCRATCH_BYTES)
        return set_error(P8X_ERR_UNSUPPORTED, "p8x_mul_mat_noalloc: %d tokens of a %d x %d tensor need %zu workspace bytes, above the %d-byte scratch",
                         N, t->rows, t->K, xb_al + pb, P8X_NOALLOC_SCRATCH_BYTES);
    uint8_t *base = static_cast<uint8_t *>(scratch_ptr(t->device));
    if (!base) {   // the tensor was prepared on a device whose scratch is not resolved yet (first call there)
        int rc = scratch_resolve(t->device);
        if (rc) return rc;
        base = static_cast<uint8_t *>(scratch_ptr(t->device));
    }
    // x' first, the output planes after it on a 256-byte boundary; every byte read is written earlier in the call
    return launch_mul_mat_ws(t, x, x_dtype, N, ldx, y, ldy, reinterpret_cast<_Float16 *>(base), reinterpret_cast<float *>(base + xb_al),
                             (hipStream_t)stream);
}
