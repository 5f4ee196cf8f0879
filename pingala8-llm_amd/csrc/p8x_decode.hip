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
// Each wave walks tiles with the next tile's payload already in flight (loads into registers), so
// the decode of one tile overlaps the memory latency of the next.
#include <hip/hip_runtime.h>

#include "p8x_internal.h"
#include "p8x_lane.h"

namespace p8x {

constexpr int kDecWaves = 4;
constexpr int kDecThreads = 64 * kDecWaves;
constexpr int kStgRowWords = 132;   // dequant staging row: 512 bytes + 16 bytes of padding
// raw words held per lane: the largest class of the instantiation's class set
__host__ __device__ constexpr int dec_nw(int cm) { return cm == (1 << 3) ? 8 : 24; }

// The tiles walked are the window of row groups g0 .. g0 + gn - 1 and blocks b0 .. b0 + bn - 1 (nt = gn bn). Rotated
// outputs are relative to the window (row 32 (g - g0) + j, column 256 (b - b0) + ...); original-domain outputs keep
// the rows row0 .. row0 + nrows - 1 (original indices) at out row ro - row0 and skip the others.
struct DecodeArgs {
    const uint32_t *M; const uint16_t *S; const uint32_t *D; const uint32_t *a2; const int16_t *prm;
    const uint16_t *prmd;   // prm with bit 15 set on rows that carry clamp-delta entries
    const float *ic; const int *cp; const uint16_t *cc; const float *cv;
    void *out; size_t ld;
    int rows, K, nb, ng;
    int g0, gn, b0, bn, row0, nrows;
    size_t nt;
};

// exact ints of a decoded lane-slice of class C -> v[128] (chunk-major, element e), as float times sc
// (FP = true) or as ints (FP = false, written through the float array's bits)
template <int C, bool FP, int NW>
__device__ __forceinline__ void lane_values(const AnySlice<NW> &ls, const uint32_t *tab, uint32_t bankbytes, float sc, float (&v)[128]) {
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

// the same values from the compact 2 KB table (word (f << 1) | h): the dequantizer keeps its LDS for staging
template <int C, int NW>
__device__ __forceinline__ void lane_values_compact(const AnySlice<NW> &ls, const uint32_t *tab2, float sc, float (&v)[128]) {
    constexpr int NST = nstage_of(C), SH1 = sh1_of(C), SH2 = sh2_of(C);
#pragma unroll
    for (int t = 0; t < 32; ++t) {
        const uint32_t h = __builtin_amdgcn_ubfe(ls.H, t, 1);
        const uint32_t w0 = tab2[(ls.template field<C, 0>(t) << 1) | h];
        uint32_t w1 = 0, w2 = 0;
        if constexpr (NST > 1) w1 = tab2[(ls.template field<C, 1>(t) << 1) | h];
        if constexpr (NST > 2) w2 = tab2[(ls.template field<C, 2>(t) << 1) | h];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            int x = sext8(w0, e) * (1 << SH1);
            if constexpr (NST > 1) x += sext8(w1, e) * (1 << SH2);
            if constexpr (NST > 2) x += sext8(w2, e);
            v[4 * t + e] = (float)x * sc;
        }
    }
}

template <int CM, int NW>
__device__ __forceinline__ void lane_values_compact_any(int c, const AnySlice<NW> &ls, const uint32_t *tab2, float sc, float (&v)[128]) {
    switch (c) {
        case 1: if constexpr ((CM >> 1) & 1) { lane_values_compact<1>(ls, tab2, sc, v); break; } [[fallthrough]];
        case 2: if constexpr ((CM >> 2) & 1) { lane_values_compact<2>(ls, tab2, sc, v); break; } [[fallthrough]];
        case 3: if constexpr ((CM >> 3) & 1) { lane_values_compact<3>(ls, tab2, sc, v); break; } [[fallthrough]];
        case 4: if constexpr ((CM >> 4) & 1) { lane_values_compact<4>(ls, tab2, sc, v); break; } [[fallthrough]];
        case 5: if constexpr ((CM >> 5) & 1) { lane_values_compact<5>(ls, tab2, sc, v); break; } [[fallthrough]];
        case 6: if constexpr ((CM >> 6) & 1) { lane_values_compact<6>(ls, tab2, sc, v); break; } [[fallthrough]];
        case 7: if constexpr ((CM >> 7) & 1) { lane_values_compact<7>(ls, tab2, sc, v); break; } [[fallthrough]];
        default:
#pragma unroll
            for (int i = 0; i < 128; ++i) v[i] = 0.f;
            break;
    }
}

template <bool FP, int CM, int NW>
__device__ __forceinline__ void lane_values_any(int c, const AnySlice<NW> &ls, const uint32_t *tab, uint32_t bankbytes, float sc, float (&v)[128]) {
    switch (c) {
        case 1: if constexpr ((CM >> 1) & 1) { lane_values<1, FP>(ls, tab, bankbytes, sc, v); break; } [[fallthrough]];
        case 2: if constexpr ((CM >> 2) & 1) { lane_values<2, FP>(ls, tab, bankbytes, sc, v); break; } [[fallthrough]];
        case 3: if constexpr ((CM >> 3) & 1) { lane_values<3, FP>(ls, tab, bankbytes, sc, v); break; } [[fallthrough]];
        case 4: if constexpr ((CM >> 4) & 1) { lane_values<4, FP>(ls, tab, bankbytes, sc, v); break; } [[fallthrough]];
        case 5: if constexpr ((CM >> 5) & 1) { lane_values<5, FP>(ls, tab, bankbytes, sc, v); break; } [[fallthrough]];
        case 6: if constexpr ((CM >> 6) & 1) { lane_values<6, FP>(ls, tab, bankbytes, sc, v); break; } [[fallthrough]];
        case 7: if constexpr ((CM >> 7) & 1) { lane_values<7, FP>(ls, tab, bankbytes, sc, v); break; } [[fallthrough]];
        default:
#pragma unroll
            for (int i = 0; i < 128; ++i) v[i] = 0.f;   // class 0: zero weights (0.0f and int 0 share bits)
            break;
    }
}

// Tiles are visited in block-major order (tile index b * ng + g), so a workgroup's contiguous range shares
// few 256-column blocks; the waves of a workgroup interleave over it. While a tile is processed, the next
// tile's payload words, scale, un-permuted row and delta bounds are already loading, and every step issues
// that prefetch (the last tile repeats), so the wait counts stay exact: on gfx9 stores share the load counter,
// and a wait placed after a tile's stores would otherwise also wait for their completion.
template <int NW>
struct TileNext {
    AnyRaw<NW> raw;
    int c, ro, e0, e1;
};

__device__ __forceinline__ void tile_of(const DecodeArgs &a, size_t q, int &g, int &b) {
    b = a.b0 + (int)(q / a.gn);
    g = a.g0 + (int)(q % a.gn);
}

template <int CM, typename Body>
__device__ __forceinline__ void walk_tiles(const DecodeArgs &a, size_t first, size_t last, size_t stride, int hs, int j, bool want_rows, Body body) {
    if (first >= last) return;
    constexpr int NW = dec_nw(CM);
    TileNext<NW> nx;
    auto issue = [&](size_t q) {
        int g, b;
        tile_of(a, q, g, b);
        const uint32_t mt = a.M[(size_t)g * a.nb + b];
        nx.c = (int)(mt >> 29);
        load_any<CM>(nx.raw, nx.c, a.D + (mt & 0x1FFFFFFFu) + hs * nw_of(nx.c) * 32, j, a.S + (size_t)b * a.rows + 32 * g);
        // the flagged row only: its delta range is read when the tile is decoded, and only for flagged rows, so
        // no load here waits on another (a dependent load would wait for the payload issued before it)
        if (want_rows) nx.ro = a.prmd[32 * g + j];
    };
    issue(first);
    for (size_t q = first; q < last; q += stride) {
        AnySlice<NW> ls;
        prepare_any<CM>(ls, nx.c, nx.raw);   // consumes this tile's words
        const int c = nx.c, ro = nx.ro & 0x7FFF;
        int e0 = 0, e1 = 0;
        if (want_rows && (nx.ro & 0x8000)) { e0 = a.cp[ro]; e1 = a.cp[ro + 1]; }
        issue(q + stride < last ? q + stride : q);   // the next tile's words load during this tile
        int g, b;
        tile_of(a, q, g, b);
        body(g, b, c, ls, ro, e0, e1);
    }
}

// a workgroup's contiguous range of the block-major tile order
__device__ __forceinline__ void wg_range(const DecodeArgs &a, size_t &first, size_t &last) {
    const size_t per = (a.nt + gridDim.x - 1) / gridDim.x;
    first = (size_t)blockIdx.x * per;
    last = first + per < a.nt ? first + per : a.nt;
}

// DT: P8X_I16 (exact ints) or P8X_F32 (int * S), sorted rows, rotated domain
template <int DT, int CM>
__global__ __launch_bounds__(kDecThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_decode_rotated(const DecodeArgs a) {
    constexpr int NW = dec_nw(CM);
    __shared__ __align__(16) uint32_t tab[kTabWords];
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), hs = lane >> 5, j = lane & 31;
    const uint32_t bankbytes = (uint32_t)(j << 2) * 0x01010101u;
    build_coset_table<kDecThreads>(tab, a.a2, tid);
    __syncthreads();
    size_t first, last;
    wg_range(a, first, last);
    walk_tiles<CM>(a, first + w, last, kDecWaves, hs, j, false, [&](int g, int b, int c, const AnySlice<NW> &ls, int, int, int) {
        float v[128];
        lane_values_any<DT == P8X_F32, CM>(c, ls, tab, bankbytes, half_to_float(ls.s), v);
        const size_t o = (size_t)(32 * (g - a.g0) + j) * a.ld + 256 * (b - a.b0) + 128 * hs;
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

// original-domain weights, DT = P8X_F32 / P8X_F16 / P8X_BF16. The tile's outputs are staged in the wave's
// LDS rows (row stride 528 bytes: 16 bytes of padding spread the rows over the banks, and every chunk is an
// immediate offset from one per-lane base) and stored two whole row segments per instruction, so every store
// covers full cache lines of two output rows instead of 16 bytes of 64 rows.
template <int DT, int CM>
__global__ __launch_bounds__(kDecThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_dequant(const DecodeArgs a) {
    constexpr int NW = dec_nw(CM);
    __shared__ uint32_t tab2[512];                         // (f << 1) | h: A[f] + h c
    __shared__ __align__(16) float icw[kDecWaves][256];    // per wave: ic of the block it is on
    __shared__ __align__(16) uint32_t stg[kDecWaves][32 * kStgRowWords];   // per wave: 32 rows x 512 (+16) bytes
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), hs = lane >> 5, j = lane & 31;
    for (int i = tid; i < 512; i += kDecThreads) tab2[i] = a.a2[(i & 1) * 256 + (i >> 1)];
    __syncthreads();
    size_t first, last;
    wg_range(a, first, last);
    int icb = -1;
    uint32_t *sw = stg[w];
    walk_tiles<CM>(a, first + w, last, kDecWaves, hs, j, true, [&](int g, int b, int c, const AnySlice<NW> &ls, int ro, int e0, int e1) {
        if (b != icb) {   // a new block for this wave: its ic into the wave's LDS row (wave-local)
            const float4 c4 = reinterpret_cast<const float4 *>(a.ic + 256 * b)[lane];
            reinterpret_cast<float4 *>(icw[w])[lane] = c4;
            icb = b;
        }
        float v[128];
        lane_values_compact_any<CM>(c, ls, tab2, half_to_float(ls.s), v);
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
        const float *icl = icw[w] + 128 * hs;
#pragma unroll
        for (int i = 0; i < 128; i += 4) {
            const float4 c4 = *reinterpret_cast<const float4 *>(icl + i);
            v[i] = (v[i] * 0.0625f) * c4.x; v[i + 1] = (v[i + 1] * 0.0625f) * c4.y;
            v[i + 2] = (v[i + 2] * 0.0625f) * c4.z; v[i + 3] = (v[i + 3] * 0.0625f) * c4.w;
        }
        for (int e = e0; e < e1; ++e) {   // clamp delta (original row, column)
            const int col = (int)a.cc[e] - 256 * b - 128 * hs;
            if (col >= 0 && col < 128) {
                const float dv = a.cv[e];
#pragma unroll
                for (int i = 0; i < 128; ++i) v[i] = i == col ? v[i] + dv : v[i];
            }
        }
        // staging: row j of the wave's buffer = the tile's row j (512 bytes: the whole fp16 row, or one f32 half)
        auto put = [&](int chunk, uint4 val) { *reinterpret_cast<uint4 *>(sw + j * kStgRowWords + 4 * chunk) = val; };
        auto store_rows = [&](int col0) {   // 16 instructions, each two rows x 512 bytes; col0 in output elements
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the wave's staging writes are done
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = 2 * i + (lane >> 5), ch = lane & 31;
                const uint4 val = *reinterpret_cast<const uint4 *>(sw + row * kStgRowWords + 4 * ch);
                const int orow = __shfl(ro, row) - a.row0;   // output row; rows outside the range are skipped
                if ((unsigned)orow < (unsigned)a.nrows) {
                    if constexpr (DT == P8X_F32) *reinterpret_cast<uint4 *>((float *)a.out + (size_t)orow * a.ld + col0 + 4 * ch) = val;
                    else *reinterpret_cast<uint4 *>((uint16_t *)a.out + (size_t)orow * a.ld + col0 + 8 * ch) = val;
                }
                if ((i & 3) == 3) __builtin_amdgcn_sched_barrier(0);   // 4 stores at a time: bounds the live registers
            }
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // reads done before the buffer is written again
        };
        if constexpr (DT == P8X_F32) {
#pragma unroll
            for (int r = 0; r < 2; ++r) {   // one half-slice per round: 128 floats = 32 chunks per lane
                if (hs == r)
#pragma unroll
                    for (int t = 0; t < 32; ++t)
                        put(t, make_uint4(__builtin_bit_cast(uint32_t, v[4 * t]), __builtin_bit_cast(uint32_t, v[4 * t + 1]),
                                          __builtin_bit_cast(uint32_t, v[4 * t + 2]), __builtin_bit_cast(uint32_t, v[4 * t + 3])));
                store_rows(256 * b + 128 * r);
            }
        } else {
#pragma unroll
            for (int t = 0; t < 16; ++t) {   // 128 halfs = 16 chunks per lane, at chunk 16 hs + t of the row
                uint32_t wv[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    uint16_t h0, h1;
                    if constexpr (DT == P8X_F16) {
                        h0 = __builtin_bit_cast(uint16_t, (_Float16)v[8 * t + 2 * q]);       // v_cvt_f16_f32, RNE
                        h1 = __builtin_bit_cast(uint16_t, (_Float16)v[8 * t + 2 * q + 1]);
                    } else {
                        h0 = __builtin_bit_cast(uint16_t, (__bf16)v[8 * t + 2 * q]);         // v_cvt_pk_bf16_f32, RNE
                        h1 = __builtin_bit_cast(uint16_t, (__bf16)v[8 * t + 2 * q + 1]);
                    }
                    wv[q] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                }
                put(16 * hs + t, make_uint4(wv[0], wv[1], wv[2], wv[3]));
            }
            store_rows(256 * b);
        }
    });
}

// ------------------------------------------------------------------------------------------------ dequantize, classes 0-3
// The same outputs as k_dequant for tensors whose tiles are of classes 0-3 (one codebook stage, |A[f] + h c| <= 128),
// computed with integer butterflies wherever the reference's f32 arithmetic is exact:
//   * v S is exact in f32 (|v| <= 128, S an fp16 with 11 significant bits), and so is every sum of up to 64 of them
//     (64 * 128 * 2047 < 2^24): stages h = 1 .. 32 of the reference never round, and equal the integer transform
//     times S. Stages 1-2 act inside a 4-column chunk and come from a table (FWHT4 of each codeword, int16 x 4);
//     stages 4-32 are packed int16 butterflies (|sums| <= 64 * 128).
//   * stage 64 adds two exact values and rounds once: RN(I_a S +- I_b S) = RN((I_a +- I_b) S), so it is the integer
//     butterfly (|I| <= 16384) followed by the one f32 multiply by S;
//   * stage 128, * 0.0625 * ic (0.0625 folded into ic: scaling by a power of two is exact) and the clamp delta are
//     the reference's f32 operations on the reference's operands; f16 / bf16 are the RNE conversions of that f32.
// Lane (j, p) of a wave holds row j of the tile, columns 64 p .. 64 p + 63 of both half-slices: stages 4-32 stay in
// the lane, stage 64 pairs lane j with lane j + 32 (v_permlane32_swap on the packed ints), stage 128 pairs the lane's
// two half-slices. Each lane then writes 128 contiguous bytes (f16) per half-slice of its output row.
constexpr int kLoWaves = 4;
constexpr int kLoThreads = 64 * kLoWaves;
constexpr int kLoBandWords = 36;   // staging row: 128 bytes + 16 bytes of padding (rows spread over the banks)
typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ s16x2 as_s16x2(uint32_t v) { return __builtin_bit_cast(s16x2, v); }
__device__ __forceinline__ uint32_t as_u32(s16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// table entry (f << 1) | h: the first two butterfly stages of the codeword bytes A[f] + h c, as int16 x 4
__device__ __forceinline__ uint2 fwht4_entry(uint32_t w) {
    const int b0 = sext8(w, 0), b1 = sext8(w, 1), b2 = sext8(w, 2), b3 = sext8(w, 3);
    const int s0 = b0 + b1, s1 = b0 - b1, s2 = b2 + b3, s3 = b2 - b3;
    const int y0 = s0 + s2, y1 = s1 + s3, y2 = s0 - s2, y3 = s1 - s3;
    return make_uint2((uint32_t)(uint16_t)y0 | ((uint32_t)(uint16_t)y1 << 16), (uint32_t)(uint16_t)y2 | ((uint32_t)(uint16_t)y3 << 16));
}

// Payload words of lane-slice (hs, j) of a class-C tile (p: the half-slice's words of the wave's LDS copy, device
// layout), read so that after the bit rotation of lo_decode the lane's fields start at chunk 16 p: the stored field
// k is chunk k, so the bitstring is rotated right by d = 16 p fields (whole words here, the rest in lo_decode).
template <int C>
__device__ __forceinline__ void lo_read(uint32_t (&w)[8], const uint32_t *p, int j, int d) {
    constexpr int W1 = w1_of(C), NW = nw_of(C);
    if constexpr (W1 == 8) {
        const int wr = d >> 2;
#pragma unroll
        for (int m = 0; m < 8; ++m) w[m] = p[dev_word((m + wr) & 7, j, NW)];
    } else {
        constexpr int W = W1 - 1;
        const int wr = (d * W) >> 5;
        w[0] = p[dev_word(0, j, NW)];
#pragma unroll
        for (int m = 0; m < W; ++m) w[1 + m] = p[dev_word(1 + (m + wr) % W, j, NW)];
#pragma unroll
        for (int m = W + 1; m < 8; ++m) w[m] = 0u;
    }
}

// chunks 16 p .. 16 p + 15 of the lane-slice -> stage-2 ints, packed P[2 i] = (y0, y1), P[2 i + 1] = (y2, y3)
template <int C>
__device__ __forceinline__ void lo_decode(const uint32_t (&w)[8], int d, int p16, const uint2 *tab4, uint32_t (&P)[32]) {
    constexpr int W1 = w1_of(C);
    uint32_t r[8], z;
    if constexpr (W1 == 8) {
        const int br = 8 * (d & 3);
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = __builtin_amdgcn_alignbit(w[(i + 1) & 7], w[i], br);
        z = labels_from_bytes(r);
    } else {
        constexpr int W = W1 - 1;
        const int br = (d * W) & 31;
        r[0] = __builtin_amdgcn_alignbit(w[0], w[0], d);
#pragma unroll
        for (int i = 0; i < W; ++i) r[1 + i] = __builtin_amdgcn_alignbit(w[1 + (i + 1) % W], w[1 + i], br);
        z = r[0];
    }
    // coset bits: the trellis runs over chunks 0 .. 31 of the lane-slice; bit i here is chunk 16 p + i
    const uint32_t zt = __builtin_amdgcn_alignbit(z, z, (32 - p16) & 31);
    const uint32_t ht = trellis_coset_bits(zt);
    const uint32_t H = __builtin_amdgcn_alignbit(ht, ht, p16);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        uint32_t f;
        if constexpr (W1 == 8) {
            f = __builtin_amdgcn_ubfe(r[i >> 2], 8 * (i & 3), 8);
        } else {
            constexpr int W = W1 - 1;
            uint32_t rf[W];
#pragma unroll
            for (int q = 0; q < W; ++q) rf[q] = r[1 + q];
            f = field_of<W>(rf, i) | (__builtin_amdgcn_ubfe(r[0], i, 1) << W);
        }
        const uint2 e = tab4[(f << 1) | __builtin_amdgcn_ubfe(H, i, 1)];
        P[2 * i] = e.x;
        P[2 * i + 1] = e.y;
        if ((i & 3) == 3) __builtin_amdgcn_sched_barrier(0);   // 4 lookups at a time
    }
}

template <int CM>
__device__ __forceinline__ void lo_decode_any(int c, const uint32_t (&w)[8], int d, int p16, const uint2 *tab4, uint32_t (&P)[32]) {
    switch (c) {
        case 1: if constexpr ((CM >> 1) & 1) { lo_decode<1>(w, d, p16, tab4, P); break; } [[fallthrough]];
        case 2: if constexpr ((CM >> 2) & 1) { lo_decode<2>(w, d, p16, tab4, P); break; } [[fallthrough]];
        case 3: if constexpr ((CM >> 3) & 1) { lo_decode<3>(w, d, p16, tab4, P); break; } [[fallthrough]];
        default:
#pragma unroll
            for (int i = 0; i < 32; ++i) P[i] = 0u;   // class 0: zero weights
            break;
    }
}

template <int CM>
__device__ __forceinline__ void lo_read_any(int c, uint32_t (&w)[8], const uint32_t *p, int j, int d) {
    switch (c) {
        case 1: if constexpr ((CM >> 1) & 1) { lo_read<1>(w, p, j, d); break; } [[fallthrough]];
        case 2: if constexpr ((CM >> 2) & 1) { lo_read<2>(w, p, j, d); break; } [[fallthrough]];
        case 3: if constexpr ((CM >> 3) & 1) { lo_read<3>(w, p, j, d); break; } [[fallthrough]];
        default:
#pragma unroll
            for (int i = 0; i < 8; ++i) w[i] = 0u;
            break;
    }
}

// butterflies h = 4, 8, 16, 32 of the lane's 64 values (exact int16)
__device__ __forceinline__ void lo_stages(uint32_t (&P)[32]) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int st = 1 << m;
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (!(i & st))
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const s16x2 a = as_s16x2(P[2 * i + k]), b = as_s16x2(P[2 * (i + st) + k]);
                    P[2 * i + k] = as_u32(a + b);
                    P[2 * (i + st) + k] = as_u32(a - b);
                }
    }
#pragma unroll
    for (int k = 0; k < 32; ++k) __asm__ volatile("; stages %0" : "+v"(P[k]));   // materialized before the exchange
}

// butterfly h = 64 across lanes j and j + 32: the lane with p = 0 keeps x0 + x1, the one with p = 1 keeps x0 - x1
__device__ __forceinline__ void lo_stage64(uint32_t (&P)[32], s16x2 sg) {
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const auto pr = __builtin_amdgcn_permlane32_swap(P[k], P[k], false, false);   // [0]: x0, [1]: x1 (both lanes)
        P[k] = as_u32(as_s16x2(pr[0]) + as_s16x2(pr[1]) * sg);
        __asm__ volatile("; stage64 %0" : "+v"(P[k]));   // combined here: keeps at most a few exchanged pairs live
    }
}

struct LoNext {   // the next tile's class (its payload is in the wave's LDS copy)
    int c;
};
constexpr int kLoTileWords = 512;   // a tile of classes 0-3 (nw <= 8): at most 2 KB

template <int DT, int CM>
__global__ __launch_bounds__(kLoThreads) __attribute__((amdgpu_waves_per_eu(4, 4))) void k_dequant_lo(const DecodeArgs a) {
    static_assert(DT == P8X_F16 || DT == P8X_BF16, "16-bit outputs (f32 goes through k_dequant)");
    __shared__ uint2 tab4[512];
    __shared__ __align__(16) float icw[kLoWaves][256];
    __shared__ __align__(16) uint32_t stg[kLoWaves][32 * kLoBandWords];   // one 32-row x 128-byte band per wave
    __shared__ __align__(16) uint32_t pay[kLoWaves][kLoTileWords];         // the next tile's payload, per wave
    const int tid = threadIdx.x, lane_in = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    for (int i = tid; i < 512; i += kLoThreads) tab4[i] = fwht4_entry(a.a2[(i & 1) * 256 + (i >> 1)]);
    __syncthreads();
    size_t first, last;
    wg_range(a, first, last);
    first += w;
    if (first >= last) return;
    LoNext nx;
    // The next tile's payload is copied into the wave's LDS buffer (direct-to-LDS loads, no registers held) before
    // this tile's output stores, and its tile word comes through the scalar cache: stores count in vmcnt like loads,
    // so data requested after them could only be waited for together with them. A tile's row scale and row are
    // loaded at the start of its own iteration and first used after its decode.
    auto issue = [&](size_t q, int lane) {
        int g, b;
        tile_of(a, q, g, b);
        g = __builtin_amdgcn_readfirstlane(g);
        b = __builtin_amdgcn_readfirstlane(b);
        const uint32_t mt = as_const(a.M)[(size_t)g * a.nb + b];
        nx.c = (int)(mt >> 29);
        const int chunks = 16 * nw_of(nx.c);   // 16-byte pieces of the tile (both half-slices)
        if (chunks) {
            const uint32_t *base = a.D + (mt & 0x1FFFFFFFu);
#pragma unroll
            for (int i = 0; i < kLoTileWords / 256; ++i)   // lanes past the tile repeat its last piece
                __builtin_amdgcn_global_load_lds(base + 4 * min(64 * i + lane, chunks - 1), pay[w] + 256 * i, 16, 0, 0);
        }
    };
    int icb = -1;
    issue(first, lane_in);
    for (size_t q = first; q < last; q += kLoWaves) {
        // lane-derived values formed per tile: held across the loop they would be spilled, and a spill reload waits
        // for every memory operation in flight (this tile's stores included)
        int lane = lane_in;
        __asm__ volatile("" : "+v"(lane));
        const int j = lane & 31, p = lane >> 5, p16 = 16 * p;
        const int d = p16;
        const s16x2 sg = {(short)(p ? -1 : 1), (short)(p ? -1 : 1)};
        const int c = nx.c;
        uint32_t w0[8], w1[8];
        lo_read_any<CM>(c, w0, pay[w], j, d);
        lo_read_any<CM>(c, w1, pay[w] + nw_of(c) * 32, j, d);
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // read before the next tile's copy overwrites it
        int g, b;
        tile_of(a, q, g, b);
        g = __builtin_amdgcn_readfirstlane(g);
        b = __builtin_amdgcn_readfirstlane(b);
        const uint16_t s16 = a.S[(size_t)b * a.rows + 32 * g + j];
        const int rof = a.prmd[32 * g + j], ro = rof & 0x7FFF;
        if (q + kLoWaves < last) issue(q + kLoWaves, lane);
        // one half-slice at a time through its integer stages (only its 32 packed registers are being built)
        uint32_t P0[32], P1[32];
        lo_decode_any<CM>(c, w0, d, p16, tab4, P0);
        lo_stages(P0);
        lo_stage64(P0, sg);
        __asm__ volatile("" ::: "memory");
        lo_decode_any<CM>(c, w1, d, p16, tab4, P1);
        lo_stages(P1);
        lo_stage64(P1, sg);
        __asm__ volatile("" ::: "memory");
        const float S = half_to_float(s16);
        if (b != icb) {   // this block's ic / 16 into the wave's row (wave-local)
            const float4 c4 = reinterpret_cast<const float4 *>(a.ic + 256 * b)[lane];
            reinterpret_cast<float4 *>(icw[w])[lane] = make_float4(c4.x * 0.0625f, c4.y * 0.0625f, c4.z * 0.0625f, c4.w * 0.0625f);
            icb = b;
        }
        int e0 = 0, e1 = 0;
        if (rof & 0x8000) { e0 = a.cp[ro]; e1 = a.cp[ro + 1]; }
        const bool deltas = __builtin_amdgcn_ballot_w64(e0 < e1) != 0;   // wave-uniform
        const float *icl = icw[w] + 64 * p;
        // the packed 16-bit outputs: OUT[h][g] holds values 8 g .. 8 g + 7 of half-slice h (columns 64 p + ..)
        uint32_t OUT[2][8][4];
#pragma unroll
        for (int k4 = 0; k4 < 32; k4 += 4) {
            float o[2][8];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const int k = k4 + kk;
                const s16x2 x = as_s16x2(P0[k]), y = as_s16x2(P1[k]);
                const float x0 = (float)x.x * S, x1 = (float)x.y * S, y0 = (float)y.x * S, y1 = (float)y.y * S;
                const float2 c0 = *reinterpret_cast<const float2 *>(icl + 2 * k);
                const float2 c1 = *reinterpret_cast<const float2 *>(icl + 128 + 2 * k);
                o[0][2 * kk] = (x0 + y0) * c0.x;
                o[0][2 * kk + 1] = (x1 + y1) * c0.y;
                o[1][2 * kk] = (x0 - y0) * c1.x;
                o[1][2 * kk + 1] = (x1 - y1) * c1.y;
            }
            if (deltas) {   // clamp delta (original row, column), in entry order
                for (int e = e0; e < e1; ++e) {
                    const int col = (int)a.cc[e] - 256 * b;
                    const float dv = a.cv[e];
#pragma unroll
                    for (int h = 0; h < 2; ++h)
#pragma unroll
                        for (int i = 0; i < 8; ++i)
                            if (col == 128 * h + 64 * p + 2 * k4 + i) o[h][i] += dv;
                }
            }
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int q2 = 0; q2 < 4; ++q2) {
                    if constexpr (DT == P8X_F16) {   // v_cvt_pk_f16_f32: both RNE
                        const f16x2 hv = {(_Float16)o[h][2 * q2], (_Float16)o[h][2 * q2 + 1]};
                        OUT[h][k4 >> 2][q2] = __builtin_bit_cast(uint32_t, hv);
                    } else {                          // v_cvt_pk_bf16_f32: both RNE
                        const bf16x2 hv = {(__bf16)o[h][2 * q2], (__bf16)o[h][2 * q2 + 1]};
                        OUT[h][k4 >> 2][q2] = __builtin_bit_cast(uint32_t, hv);
                    }
                    __asm__ volatile("; out %0" : "+v"(OUT[h][k4 >> 2][q2]));
                }
            __builtin_amdgcn_sched_barrier(0);   // one group at a time: its packed ints are consumed as its outputs appear
        }
        // Out through the wave's LDS band, one (half-slice, quarter) band of the tile at a time: the lanes that own
        // it write their 128 bytes, then each store instruction covers 8 rows x 128 bytes (whole lines).
        uint32_t *sw = stg[w];
        int orows[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) orows[i] = (__shfl(rof, 8 * i + (lane >> 3)) & 0x7FFF) - a.row0;   // row of piece 64 i + lane
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int qq = 0; qq < 2; ++qq) {
                if (p == qq)
#pragma unroll
                    for (int gg = 0; gg < 8; ++gg)
                        *reinterpret_cast<uint4 *>(sw + j * kLoBandWords + 4 * gg) = make_uint4(OUT[h][gg][0], OUT[h][gg][1], OUT[h][gg][2], OUT[h][gg][3]);
                __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the band is written
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = 8 * i + (lane >> 3), piece = lane & 7;
                    const uint4 val = *reinterpret_cast<const uint4 *>(sw + row * kLoBandWords + 4 * piece);
                    if ((unsigned)orows[i] < (unsigned)a.nrows)
                        *reinterpret_cast<uint4 *>((uint16_t *)a.out + (size_t)orows[i] * a.ld + 256 * b + 128 * h + 64 * qq + 8 * piece) = val;
                }
                __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // read before the next band overwrites it
            }
    }
}

static DecodeArgs decode_args(const p8x_tensor *t, void *out, size_t ld) {
    DecodeArgs a{};
    a.M = t->M; a.S = t->S; a.D = t->D; a.a2 = t->a2; a.prm = t->prm; a.prmd = t->prmd;
    a.ic = t->ic; a.cp = t->cp; a.cc = t->cc; a.cv = t->cv;
    a.out = out; a.ld = ld;
    a.rows = t->rows; a.K = t->K; a.nb = t->nb; a.ng = t->ng; a.nt = t->nt;
    a.g0 = 0; a.gn = t->ng; a.b0 = 0; a.bn = t->nb; a.row0 = 0; a.nrows = t->rows;
    return a;
}

// two 4-wave workgroups per CU (the 64 KB table each), persistent
static int decode_grid(const DecodeArgs &a) {
    const size_t wgs = (a.nt + kDecWaves - 1) / kDecWaves;
    return (int)std::min<size_t>(wgs, (size_t)num_cus() * 2);
}

static bool only_class3(const p8x_tensor *t) {
    for (int c = 1; c < 8; ++c) if (c != 3 && t->class_tiles[c]) return false;
    return true;
}

// every tile of class 0-3: the integer-butterfly dequantizer
static bool classes_upto3(const p8x_tensor *t) {
    for (int c = 4; c < 8; ++c) if (t->class_tiles[c]) return false;
    return true;
}

template <int CM>
static void launch_deq_lo(int dtype, const DecodeArgs &a, int grid, hipStream_t st) {
    if (dtype == P8X_F16) hipLaunchKernelGGL((k_dequant_lo<P8X_F16, CM>), dim3(grid), dim3(kLoThreads), 0, st, a);
    else hipLaunchKernelGGL((k_dequant_lo<P8X_BF16, CM>), dim3(grid), dim3(kLoThreads), 0, st, a);
}

template <int CM>
static void launch_rot(const p8x_tensor *t, int dtype, const DecodeArgs &a, hipStream_t st) {
    if (dtype == P8X_I16) hipLaunchKernelGGL((k_decode_rotated<P8X_I16, CM>), dim3(decode_grid(a)), dim3(kDecThreads), 0, st, a);
    else hipLaunchKernelGGL((k_decode_rotated<P8X_F32, CM>), dim3(decode_grid(a)), dim3(kDecThreads), 0, st, a);
}

template <int CM>
static void launch_deq(const p8x_tensor *t, int dtype, const DecodeArgs &a, hipStream_t st) {
    if (dtype == P8X_F32) hipLaunchKernelGGL((k_dequant<P8X_F32, CM>), dim3(decode_grid(a)), dim3(kDecThreads), 0, st, a);
    else if (dtype == P8X_F16) hipLaunchKernelGGL((k_dequant<P8X_F16, CM>), dim3(decode_grid(a)), dim3(kDecThreads), 0, st, a);
    else hipLaunchKernelGGL((k_dequant<P8X_BF16, CM>), dim3(decode_grid(a)), dim3(kDecThreads), 0, st, a);
}

int launch_decode_rotated(const p8x_tensor *t, int dtype, int g0, int gn, int b0, int bn, void *out, size_t ld, hipStream_t st) {
    if (ld % 4) return set_error(P8X_ERR_ARG, "decode: ld %zu must be a multiple of 4", ld);
    DecodeArgs a = decode_args(t, out, ld);
    a.g0 = g0; a.gn = gn; a.b0 = b0; a.bn = bn; a.nt = (size_t)gn * bn;
    if (only_class3(t)) launch_rot<(1 << 3)>(t, dtype, a, st);
    else launch_rot<0xFE>(t, dtype, a, st);
    return hip_check(hipGetLastError(), "k_decode_rotated launch");
}

int launch_dequant(const p8x_tensor *t, int dtype, int row0, int nrows, void *out, size_t ld, hipStream_t st) {
    if (ld % 4) return set_error(P8X_ERR_ARG, "dequantize: ld %zu must be a multiple of 4", ld);
    DecodeArgs a = decode_args(t, out, ld);
    a.row0 = row0; a.nrows = nrows;
    if (row0 != 0 || nrows != t->rows) {   // the row groups holding those original rows (their sorted rows' groups)
        int lo = t->ng, hi = -1;
        for (int ro = row0; ro < row0 + nrows; ++ro) {
            const int g = t->pinv_host[ro] / 32;
            lo = std::min(lo, g);
            hi = std::max(hi, g);
        }
        a.g0 = lo; a.gn = hi - lo + 1; a.nt = (size_t)a.gn * a.bn;
    }
    if (classes_upto3(t) && dtype != P8X_F32) {
        const int grid = (int)std::min<size_t>((a.nt + kLoWaves - 1) / kLoWaves, (size_t)num_cus() * 4);
        if (only_class3(t)) launch_deq_lo<(1 << 3)>(dtype, a, grid, st);
        else launch_deq_lo<(1 << 1) | (1 << 2) | (1 << 3)>(dtype, a, grid, st);
    } else if (only_class3(t)) {
        launch_deq<(1 << 3)>(t, dtype, a, st);
    } else {
        launch_deq<0xFE>(t, dtype, a, st);
    }
    return hip_check(hipGetLastError(), "k_dequant launch");
}

}  // namespace p8x
