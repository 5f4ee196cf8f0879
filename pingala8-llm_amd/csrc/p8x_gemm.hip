// p8x_gemm.hip -- prompt-processing GEMM: Y [N][rows] = X [N][K] W^T for a Pingala-8 tensor W.
//
// The 256-point Hadamard rotation of every weight block moves onto the activations:
//   W[prm[r], 256b + c] = (FWHT(v[r, 256b + :] S[b][r]) / 16)[c] ic[256b + c]   (+ clamp delta)
// so  Y[n, prm[r]] = sum_b S[b][r] sum_i v[r, 256b + i] x'[n, 256b + i] + delta terms, with
//   x' = FWHT(x ic) / 16 per 256-block (the GEMV's activation prep, CPU.patch:559-571, kept in fp16 here).
// Pass 1 (k_mm_act) writes x' as fp16 [N][K]. Pass 2 (k_mm) gives each wave two 32-row tiles of a 256-row
// workgroup tile: per 256-block it decodes the tiles in chunk order (rotated loads, p8x_lane.h) through a
// 4 KB fp16 LDS copy of the coset table straight into MFMA operands (v S, one rounding), and multiplies them
// with the block's x' (staged by direct-to-LDS loads) by v_mfma_f32_32x32x16_f16 with fp32 accumulation.
// Tokens are the MFMA rows and weight rows its columns, so each lane's outputs run along 32 consecutive sorted
// rows (coalesced stores). Sorted-row planes (one per K split) are then summed in a fixed order, un-permuted
// and given the sparse clamp delta (CPU.patch:1193) on the original activations by k_mm_finish; a tensor
// with identity rows and one K range writes y directly and only adds the delta.
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

constexpr int kMmTok = 128;      // tokens per workgroup tile (4 MFMA row tiles of 32)

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
    const uint32_t *a2;     // [2][256] coset table words (A[f] + h c), h-major
    int N, rows, K, nb, ng;
    int tiles_m, tiles_n, nsplit, kper, direct;
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

template <int C, int NWMAX>
__device__ __forceinline__ half8v decode_pair(const AnySlice<NWMAX> &ls, const uint32_t *tab, uint32_t bankbytes, int s) {
    const half2v s2 = {__builtin_bit_cast(_Float16, (uint16_t)ls.s), __builtin_bit_cast(_Float16, (uint16_t)ls.s)};
    const uint32_t hq = coset_bytes(ls.H, bankbytes, s >> 1);
    uint32_t w0[3], w1[3];
    lookup_chunk<C>(ls, tab, 2 * s, hq, w0);
    lookup_chunk<C>(ls, tab, 2 * s + 1, hq, w1);
    half2v a, b, c, d;
    weights_chunk<C>(w0, s2, a, b);
    weights_chunk<C>(w1, s2, c, d);
    half8v o;
    o[0] = a.x; o[1] = a.y; o[2] = b.x; o[3] = b.y; o[4] = c.x; o[5] = c.y; o[6] = d.x; o[7] = d.y;
    return o;
}

// classes decoded by an instantiation: the tensor's class set (class 0 decodes as zeros in all of them)
constexpr int kMmCmC3 = 1 << 3, kMmCmAll = 0xFE;
constexpr int kMmMain = 3;   // the class with a branch-free path in every instantiation (the 2-bit bulk)
__host__ __device__ constexpr int mm_nwmax(int cm) { return cm == kMmCmC3 ? 8 : 24; }
// Waves per workgroup (each: 64 weight rows x 128 tokens, 128 accumulator registers): the class-3 kernel fits in 256
// registers per wave and runs two waves per SIMD (one's decode overlaps the other's MFMAs) in 8-wave workgroups of
// 512 rows that share the x' tile and the table; the every-class kernel needs more and runs one wave per SIMD.
__host__ __device__ constexpr int mm_waves(int cm) { return cm == kMmCmC3 ? 8 : 4; }

template <int CM, int NWMAX>
__device__ __forceinline__ half8v decode_any(const AnySlice<NWMAX> &ls, int c, const uint32_t *tab, uint32_t bankbytes, int s) {
    switch (c) {
        case 1: if constexpr ((CM >> 1) & 1) return decode_pair<1>(ls, tab, bankbytes, s); break;
        case 2: if constexpr ((CM >> 2) & 1) return decode_pair<2>(ls, tab, bankbytes, s); break;
        case 3: if constexpr ((CM >> 3) & 1) return decode_pair<3>(ls, tab, bankbytes, s); break;
        case 4: if constexpr ((CM >> 4) & 1) return decode_pair<4>(ls, tab, bankbytes, s); break;
        case 5: if constexpr ((CM >> 5) & 1) return decode_pair<5>(ls, tab, bankbytes, s); break;
        case 6: if constexpr ((CM >> 6) & 1) return decode_pair<6>(ls, tab, bankbytes, s); break;
        case 7: if constexpr ((CM >> 7) & 1) return decode_pair<7>(ls, tab, bankbytes, s); break;
        default: break;
    }
    return half8v{};
}

// x' half-block tile in LDS: half sh of block b holds, per token, columns 128 kh + 64 sh + 8 c8 + (0..7) as
// chunk c = 8 kh + c8 at position c ^ (t & 15) of the token's 256-byte row, so the 16-byte operand reads of
// 16 consecutive tokens cover all 64 banks once.
constexpr int kMmXsHalfs = kMmTok * 128;

// Stage half sh of block b: with IPW = 128 / (4 NWAVES) instructions per wave, instruction i of wave w fills token
// rows 4 (IPW w + i) + (0..3); lane l lands at the instruction's LDS base + 16 l (direct-to-LDS), i.e. row + (l >> 4),
// position l & 15.
template <int NWAVES>
__device__ __forceinline__ void mm_stage(const MmJob &J, _Float16 *xb, int tok0, int b, int sh, int w, int lane) {
    constexpr int IPW = kMmTok / (4 * NWAVES);   // instructions per wave
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
        const int row = 4 * (IPW * w + i), t = row + (lane >> 4);
        const int ts = min(tok0 + t, J.N - 1);   // rows past N repeat the last token (never written out)
        const int c = (lane & 15) ^ (t & 15);
        const _Float16 *src = J.xr + (size_t)ts * J.K + 256 * b + 128 * (c >> 3) + 64 * sh + 8 * (c & 7);
        __builtin_amdgcn_global_load_lds(src, xb + row * 128, 16, 0, 0);
    }
}

// issue the raw payload loads of the wave's two tiles at block b
template <int CM, int NWMAX>
__device__ __forceinline__ void mm_issue(const MmJob &J, AnyRaw<NWMAX> (&raw)[2], int (&cl)[2], const int (&g)[2], int b, int j, int kh) {
#pragma unroll
    for (int tj = 0; tj < 2; ++tj) {
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
template <int CM, int NWMAX>
__device__ __forceinline__ void mm_prepare(AnySlice<NWMAX> (&ls)[2], const int (&cl)[2], const AnyRaw<NWMAX> (&raw)[2]) {
#pragma unroll
    for (int tj = 0; tj < 2; ++tj) {
        if constexpr (CM == kMmCmC3) ls[tj].template from_raw<3>(raw[tj]);   // zero raw words, S = 0: zero weights
        else prepare_any<CM>(ls[tj], cl[tj], raw[tj]);
    }
}

// The 8 MFMA steps of one half-block (steps s = 8 sh .. 8 sh + 7) from x' buffer xb.
template <int CM, int NWMAX>
__device__ __forceinline__ void mm_half(const _Float16 *__restrict__ xb, const AnySlice<NWMAX> (&ls)[2], const int (&cl)[2], const uint32_t *tab,
                                        uint32_t bankbytes, int sh, int j, int kh, float16v (&acc)[4][2]) {
    auto read_a = [&](int s8, half8v (&A)[4]) {
#pragma unroll
        for (int ti = 0; ti < 4; ++ti)
            A[ti] = *reinterpret_cast<const half8v *>(xb + (32 * ti + j) * 128 + 8 * ((8 * kh + s8) ^ (j & 15)));
    };
    if (CM == kMmCmC3 || (cl[0] == kMmMain && cl[1] == kMmMain)) {
        // software-pipelined by one step: x' operands and table words of step s + 1 are read before the 8 MFMAs of
        // step s, which then wait only for the fp16 conversion of their B operands
        const half2v s2[2] = {{__builtin_bit_cast(_Float16, (uint16_t)ls[0].s), __builtin_bit_cast(_Float16, (uint16_t)ls[0].s)},
                              {__builtin_bit_cast(_Float16, (uint16_t)ls[1].s), __builtin_bit_cast(_Float16, (uint16_t)ls[1].s)}};
        auto lookups = [&](int s, uint32_t (&W)[2][2][3]) {
#pragma unroll
            for (int tj = 0; tj < 2; ++tj) {
                const uint32_t hq = coset_bytes(ls[tj].H, bankbytes, s >> 1);
                lookup_chunk<kMmMain>(ls[tj], tab, 2 * s, hq, W[tj][0]);
                lookup_chunk<kMmMain>(ls[tj], tab, 2 * s + 1, hq, W[tj][1]);
            }
        };
        half8v A[4];
        uint32_t W[2][2][3];
        read_a(0, A);
        lookups(8 * sh, W);
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8) {
            half8v An[4];
            uint32_t Wn[2][2][3];
            if (s8 < 7) { read_a(s8 + 1, An); lookups(8 * sh + s8 + 1, Wn); }
            half8v B[2];
#pragma unroll
            for (int tj = 0; tj < 2; ++tj) {
                half2v a, b, c, d;
                weights_chunk<kMmMain>(W[tj][0], s2[tj], a, b);
                weights_chunk<kMmMain>(W[tj][1], s2[tj], c, d);
                B[tj][0] = a.x; B[tj][1] = a.y; B[tj][2] = b.x; B[tj][3] = b.y;
                B[tj][4] = c.x; B[tj][5] = c.y; B[tj][6] = d.x; B[tj][7] = d.y;
            }
#pragma unroll
            for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                for (int tj = 0; tj < 2; ++tj) acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[ti], B[tj], acc[ti][tj], 0, 0, 0);
            if (s8 < 7) {
#pragma unroll
                for (int ti = 0; ti < 4; ++ti) A[ti] = An[ti];
#pragma unroll
                for (int tj = 0; tj < 2; ++tj)
#pragma unroll
                    for (int u = 0; u < 2; ++u)
#pragma unroll
                        for (int q = 0; q < 3; ++q) W[tj][u][q] = Wn[tj][u][q];
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8) {
            half8v A[4], B[2];
            read_a(s8, A);
#pragma unroll
            for (int tj = 0; tj < 2; ++tj) B[tj] = decode_any<CM>(ls[tj], cl[tj], tab, bankbytes, 8 * sh + s8);
#pragma unroll
            for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                for (int tj = 0; tj < 2; ++tj) acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[ti], B[tj], acc[ti][tj], 0, 0, 0);
        }
    }
}

// One workgroup per CU of mm_waves(CM) waves (each: 64 weight rows x 128 tokens, 128 accumulator registers). K
// advances by half-blocks; the x' of the next half-block and the next block's payload are in flight while the current
// half-block is multiplied.
template <int CM>
__global__ __launch_bounds__(64 * mm_waves(CM)) __attribute__((amdgpu_waves_per_eu(mm_waves(CM) / 4, mm_waves(CM) / 4)))
void k_mm(MmJob J) {
    constexpr int NWMAX = mm_nwmax(CM), NWAVES = mm_waves(CM), kMmThreads = 64 * NWAVES, kMmRows = 64 * NWAVES;
    __shared__ uint32_t tab[kTabWords];   // first: LDS address 0, replicated coset table (bytes offset by 128)
    __shared__ __attribute__((aligned(16))) _Float16 xs0[kMmXsHalfs];   // half 0 of a block
    __shared__ __attribute__((aligned(16))) _Float16 xs1[kMmXsHalfs];   // half 1
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31, kh = lane >> 5;
    const uint32_t bankbytes = (uint32_t)(j << 2) * 0x01010101u;
    // Workgroups are dealt to the 8 XCDs round-robin (XCD = blockIdx % 8). Linear tile order is x'-slice-major
    // (slice = token tile x K split, then row tile), and each XCD takes one contiguous run of it, so the
    // workgroups that read one x' slice share an L2.
    const int per = (J.tiles_m * J.tiles_n * J.nsplit + kXcds - 1) / kXcds;
    const int lin = (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
    if (lin >= J.tiles_m * J.tiles_n * J.nsplit) return;
    const int tm = lin % J.tiles_m, slice = lin / J.tiles_m;
    const int ks = slice % J.nsplit, tn = slice / J.nsplit;
    {
        uint4 *t4 = reinterpret_cast<uint4 *>(tab);
        for (int i = tid; i < kTabWords / 4; i += kMmThreads) {
            const int f = i >> 4, h = (i >> 3) & 1;
            const uint32_t v = J.a2[h * 256 + f] ^ 0x80808080u;
            t4[i] = make_uint4(v, v, v, v);
        }
    }
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
    AnySlice<NWMAX> ls[2];
    AnyRaw<NWMAX> raw[2];
    int cl[2], ncl[2];
    mm_stage<NWAVES>(J, xs0, tok0, b0, 0, w, lane);
    mm_issue<CM>(J, raw, cl, g, b0, j, kh);
    __builtin_amdgcn_s_waitcnt(0);
    mm_prepare<CM>(ls, cl, raw);
    __syncthreads();   // table and the first half-block's x' are in LDS
    // The two x' buffers are separate LDS objects named statically (half 0 always in xs0, half 1 in xs1), so
    // the compiler can tell the operand reads from the in-flight direct-to-LDS writes and does not wait for them.
    for (int b = b0; b < b1; ++b) {
        mm_stage<NWAVES>(J, xs1, tok0, b, 1, w, lane);
        if (b + 1 < b1) mm_issue<CM>(J, raw, ncl, g, b + 1, j, kh);
        mm_half<CM>(xs0, ls, cl, tab, bankbytes, 0, j, kh, acc);
        __builtin_amdgcn_s_waitcnt(0);   // half 1 of b landed (and the next block's payload)
        __syncthreads();
        if (b + 1 < b1) mm_stage<NWAVES>(J, xs0, tok0, b + 1, 0, w, lane);
        mm_half<CM>(xs1, ls, cl, tab, bankbytes, 1, j, kh, acc);
        __builtin_amdgcn_s_waitcnt(0);   // half 0 of b + 1 landed
        if (b + 1 < b1) {
            cl[0] = ncl[0]; cl[1] = ncl[1];
            mm_prepare<CM>(ls, cl, raw);
        }
        __syncthreads();
    }
    // acc[ti][tj] lane l, reg q: token 32 ti + 8 (q >> 2) + 4 kh + (q & 3), sorted row 32 g[tj] + j: 32 lanes
    // store 32 consecutive rows of one token
    float *dst = J.direct ? J.y : J.ws + (size_t)ks * J.N * J.rows;
    const size_t ld = J.direct ? (size_t)J.ldy : (size_t)J.rows;
#pragma unroll
    for (int tj = 0; tj < 2; ++tj) {
        if (g[tj] >= J.ng) continue;
        const int r = 32 * g[tj] + j;
#pragma unroll
        for (int ti = 0; ti < 4; ++ti)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int tok = tok0 + 32 * ti + 8 * (q >> 2) + 4 * kh + (q & 3);
                if (tok < J.N) dst[(size_t)tok * ld + r] = acc[ti][tj][q];
            }
    }
}

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
    int tiles_m, tiles_n, nsplit, kper;
};

// One workgroup per CU. Estimated time = rounds of workgroups x blocks per workgroup x the time of one block of a
// workgroup tile (a relative model: 256 x 128 for the every-class kernel, 512 x 128 at two waves per SIMD for the
// class-3 one) + the sorted-plane traffic of k_mm_finish (written once, read once, ~5 TB/s) when planes are used (K
// split, or rows to un-permute).
static bool mm_only_c3(const p8x_tensor *t) {
    for (int c = 1; c < 8; ++c) if (c != 3 && t->class_tiles[c]) return false;
    return true;
}

static MmPlan mm_plan(const p8x_tensor *t, int N) {
    MmPlan p;
    const bool c3 = mm_only_c3(t);
    const int rows_tile = 64 * mm_waves(c3 ? kMmCmC3 : kMmCmAll);
    const double block_us = c3 ? 4.9 : 3.4;   // one K block of one workgroup tile
    p.tiles_m = (t->rows + rows_tile - 1) / rows_tile;
    p.tiles_n = (N + kMmTok - 1) / kMmTok;
    const long base = (long)p.tiles_m * p.tiles_n, slots = num_cus();
    const double plane_us = 2.0 * 4.0 * N * t->rows / 5e6;
    // a split's planes stay within what the no-allocation entry point holds next to x', so that it runs the same
    // plan (and returns the same bits) as p8x_mul_mat wherever it runs at all
    const size_t xb = ((size_t)N * t->K * sizeof(_Float16) + 255) & ~(size_t)255;
    const size_t cap = xb < (size_t)P8X_NOALLOC_SCRATCH_BYTES ? (size_t)P8X_NOALLOC_SCRATCH_BYTES - xb : 0;
    double best = -1.0;
    p.nsplit = 1; p.kper = t->nb;
    for (int ns = 1; ns <= std::min(t->nb, 16); ++ns) {
        const int kper = (t->nb + ns - 1) / ns, nsr = (t->nb + kper - 1) / kper;
        if (nsr > 1 && (size_t)nsr * N * t->rows * 4 > cap) continue;
        const double cost = (double)((base * nsr + slots - 1) / slots) * kper * block_us + ((nsr > 1 || !t->prm_identity) ? nsr * plane_us : 0.0);
        if (best < 0 || cost < best) { best = cost; p.nsplit = nsr; p.kper = kper; }
    }
    return p;
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
    const int grid = ((p.tiles_m * p.tiles_n * p.nsplit + kXcds - 1) / kXcds) * kXcds;
    if (mm_only_c3(t)) hipLaunchKernelGGL(k_mm<kMmCmC3>, dim3(grid), dim3(64 * mm_waves(kMmCmC3)), 0, st, J);
    else hipLaunchKernelGGL(k_mm<kMmCmAll>, dim3(grid), dim3(64 * mm_waves(kMmCmAll)), 0, st, J);
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
