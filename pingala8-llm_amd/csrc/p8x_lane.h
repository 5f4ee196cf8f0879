// p8x_lane.h -- gfx950 lane-slice decoder shared by every kernel.
//
// One wave64 owns one tile (g, b): lane L decodes half-slice hs = L >> 5 of sorted row 32g + (L & 31).
// A lane-slice is NW(c) payload words holding 32 fields per stage. In the file, step k of lane j encodes chunk
// t = (j + k) & 31 (CPU.patch:155-158); p8x_prepare rotates every lane's fields once (k_relayout_payload) so that
// in device memory field t of every region IS chunk t, for every lane, and places the words in 16-byte groups
// (dev_word, p8x_format.h). Every loader here reads that layout as stored: all field indexing is compile-time and
// the activation chunk of a step is the same for all 32 lanes of a half-wave.
//
// Coset table in LDS: entry (f, h) = A[f] + h * c (bytewise, CPU.patch:221/:255), replicated across the
// 32 LDS banks: byte address (f << 8) | (h << 7) | (bank << 2) with bank = lane & 31, so the 32 lanes of a
// half-wave never conflict. One v_perm_b32 builds that address from the 8-bit field and a per-lane byte
// holding (h << 7) | (bank << 2).
//
// Trellis (CPU.patch:159-160, :277-283): labels z_t in chunk order -> u_t = z_t ^ u_{t-1} ^ u_{t-3},
// h_t = u_{t-2}; computed in closed form on the 32-bit label word.
#pragma once
#include <hip/hip_runtime.h>

#include "p8x_format.h"

namespace p8x {

constexpr int kTabWords = 256 * 64;   // 64 KB coset table
// gfx950 has 8 XCDs, each with its own L2; workgroups of a launch go to them round robin by index
constexpr int kXcds = 8;
constexpr int kTabBytes = kTabWords * 4;

// Fill the replicated table from a2 = [h][256] words (h-major), all threads of the block: every load first, then the
// stores (one memory round trip for the whole table). The two halves are separate so that a kernel can issue other
// loads between them.
template <int NT>
struct CosetTableFill {
    static_assert((kTabWords / 4) % NT == 0, "table build: threads must divide the table's 16-byte entries");
    static constexpr int PER = kTabWords / 4 / NT;
    uint32_t v[PER];
    __device__ __forceinline__ void load(const uint32_t *__restrict__ a2, int tid) {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = tid + k * NT;
            v[k] = ((const __attribute__((address_space(1))) uint32_t *)a2)[((i >> 3) & 1) * 256 + (i >> 4)];
        }
    }
    __device__ __forceinline__ void store(uint32_t *tab, int tid) const {
        uint4 *t4 = reinterpret_cast<uint4 *>(tab);
#pragma unroll
        for (int k = 0; k < PER; ++k) t4[tid + k * NT] = make_uint4(v[k], v[k], v[k], v[k]);
    }
};

template <int NT>
__device__ __forceinline__ void build_coset_table(uint32_t *tab, const uint32_t *__restrict__ a2, int tid) {
    CosetTableFill<NT> f;
    f.load(a2, tid);
    f.store(tab, tid);
}

// global address-space views: pointers read out of descriptors are generic; these make loads global_load
// with an SGPR base and a 32-bit lane offset instead of FLAT loads with 64-bit per-lane addresses
template <typename T>
using gptr = __attribute__((address_space(1))) T *;
template <typename T>
__device__ __forceinline__ gptr<const T> as_global(const T *p) { return (gptr<const T>)p; }
template <typename T>
__device__ __forceinline__ gptr<T> as_global_rw(T *p) { return (gptr<T>)p; }
// constant address-space view (read-only for the kernel's lifetime): uniform loads become scalar s_load,
// which wait on their own counter instead of behind the in-flight vector loads
// raw buffer resources (stride 0, byte records); word 3 is the gfx9-family default for untyped access
constexpr int kBufFlags = 0x00020000;
constexpr int kBufNT = 2;   // cache policy: non-temporal (streamed once)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, kBufFlags);
}

template <typename T>
using kptr = __attribute__((address_space(4))) T *;
template <typename T>
__device__ __forceinline__ kptr<const T> as_const(const T *p) { return (kptr<const T>)p; }

__device__ __forceinline__ uint32_t lds_word(const uint32_t *tab, uint32_t byte_addr) {
    return *reinterpret_cast<const uint32_t *>(reinterpret_cast<const char *>(tab) + byte_addr);
}

// Ties loaded values to this point of the program: nothing computed from them moves above it, so the wait for
// their loads sits here and the loads issued for later tiles stay in flight (left alone, the scheduler hoists
// the next tile's label arithmetic and waits for that tile's loads too early).
__device__ __forceinline__ void pin(uint32_t &v) { __asm__ volatile("; pin %0" : "+v"(v)); }
__device__ __forceinline__ void pin(float &v) { __asm__ volatile("; pin %0" : "+v"(v)); }
template <int N>
__device__ __forceinline__ void pin(uint32_t (&w)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) __asm__ volatile("; pin %0" : "+v"(w[i]));
}

// closed form of the 8-state trellis over one 32-chunk label word (chunk order in, chunk order out)
__device__ __forceinline__ uint32_t trellis_coset_bits(uint32_t z) {
    uint32_t u = z;
    u ^= (u << 1) ^ (u << 3);
    u ^= (u << 2) ^ (u << 6);
    u ^= (u << 4) ^ (u << 12);
    u ^= (u << 8) ^ (u << 24);
    u ^= u << 16;
    return u << 2;
}

template <int W, int N>
__device__ __forceinline__ uint32_t field_of(const uint32_t (&R)[N], int t) {
    const int pos = W * t, wi = pos >> 5, bb = pos & 31;
    if (bb + W <= 32) return __builtin_amdgcn_ubfe(R[wi], bb, W);
    return __builtin_amdgcn_alignbit(R[(wi + 1) % N], R[wi], bb) & ((1u << W) - 1u);
}

// chunk-order labels of a W1 = 8 stage-1 region: bit t = bit 7 of byte t
__device__ __forceinline__ uint32_t labels_from_bytes(const uint32_t (&R)[8]) {
    uint32_t n[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t lo = __builtin_amdgcn_udot4(R[2 * q] & 0x80808080u, 0x08040201u, 0u, false);
        n[q] = __builtin_amdgcn_udot4(R[2 * q + 1] & 0x80808080u, 0x80402010u, lo, false);   // bits 7..14
    }
    return (n[0] >> 7) | (n[1] << 1) | (n[2] << 9) | (n[3] << 17);
}

// per-lane address bytes for chunks 4q .. 4q+3: byte e = (h_{4q+e} << 7) | (bank << 2). The nibble is first
// placed at bits 7..10 so that one 24-bit multiply by 1 + 2^7 + 2^14 + 2^21 moves bit i to bit 8i + 7.
__device__ __forceinline__ uint32_t coset_bytes(uint32_t H, uint32_t bankbytes, int q) {
    const uint32_t nib7 = (4 * q >= 7 ? H >> (4 * q - 7) : H << (7 - 4 * q)) & 0x780u;
    return (__umul24(nib7, 0x00204081u) & 0x80808080u) | bankbytes;
}

// Raw payload words of one lane-slice of class C (one 32-bit load per word), plus the lane's fp16 row scale.
// Kept separate from the decode so a wave can hold the next tile's words in flight while it decodes the current one.
template <int C>
struct RawSlice {
    static constexpr int W1 = w1_of(C), W2 = w2_of(C), W3 = w3_of(C), NW = nw_of(C);
    uint32_t w[NW];
    uint32_t s;   // fp16 row scale, zero-extended by its load

    template <int W, int WB, int O>
    static __device__ __forceinline__ void region_offsets(uint32_t hsoff, int j, uint32_t (&vo)[NW]) {
#pragma unroll
        for (int m = 0; m < W; ++m) vo[O + m] = 4u * (hsoff + (uint32_t)dev_word(WB + m, j, NW));
    }

    // Byte offsets, within a tile's payload, of the lane's NW words in load order. They depend only on the
    // lane (j, and hsoff = hs * NW * 32 for its half-slice), so a wave computes them once.
    static __device__ __forceinline__ void lane_offsets(uint32_t hsoff, int j, uint32_t (&vo)[NW]) {
        if constexpr (W1 == 8) {
            region_offsets<8, 0, 0>(hsoff, j, vo);
        } else {
            vo[0] = 4u * (hsoff + (uint32_t)dev_word(0, j, NW));
            region_offsets<W1 - 1, 1, 1>(hsoff, j, vo);
        }
        if constexpr (W2 > 0) region_offsets<W2, W1, W1>(hsoff, j, vo);
        if constexpr (W3 > 0) region_offsets<W3, W1 + W2, W1 + W2>(hsoff, j, vo);
    }

    // Buffer-resource loads: the tile's payload byte offset and its scale-row byte offset ride in the uniform
    // soffset; the lane parts (vo, vs = 2 j) are fixed. A resource with no records reads zeros without
    // touching memory, which is how a prefetch past the end of a run is issued unconditionally.
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rd, uint32_t toff, const uint32_t (&vo)[NW],
                                         __amdgpu_buffer_rsrc_t rs, uint32_t soff, uint32_t vs) {
#pragma unroll
        for (int m = 0; m < NW; ++m) w[m] = __builtin_amdgcn_raw_buffer_load_b32(rd, vo[m], toff, kBufNT);
        s = __builtin_amdgcn_raw_buffer_load_b16(rs, vs, soff, kBufNT);
    }
};

template <int W, int O, int NWT>
__device__ __forceinline__ void copy_region(const uint32_t (&w)[NWT], uint32_t (&R)[W]) {
#pragma unroll
    for (int i = 0; i < W; ++i) R[i] = w[O + i];
}

// Decoded state of one lane-slice of class C.
template <int C>
struct LaneSlice {
    static constexpr int W1 = w1_of(C), W2 = w2_of(C), W3 = w3_of(C), NW = nw_of(C);
    static constexpr int NR1 = W1 == 8 ? 8 : (W1 > 0 ? W1 - 1 : 1);
    static constexpr int NR2 = W2 ? W2 : 1, NR3 = W3 ? W3 : 1;
    uint32_t r0;           // W1 < 8: label word, chunk order
    uint32_t r1[NR1];
    uint32_t r2[NR2];
    uint32_t r3[NR3];
    uint32_t H;            // coset bits, chunk order
    uint32_t bankbytes;

    // same state from words already in registers
    __device__ __forceinline__ void from_raw(const RawSlice<C> &raw) {
        if constexpr (W1 == 8) {
            copy_region<8, 0>(raw.w, r1);
        } else {
            r0 = raw.w[0];
            copy_region<W1 - 1, 1>(raw.w, r1);
        }
        if constexpr (W2 > 0) copy_region<W2, W1>(raw.w, r2);
        if constexpr (W3 > 0) copy_region<W3, W1 + W2>(raw.w, r3);
    }

    __device__ __forceinline__ void prepare(uint32_t bb) {
        uint32_t z;
        if constexpr (W1 == 8) z = labels_from_bytes(r1);
        else z = r0;
        H = trellis_coset_bits(z);
        bankbytes = bb;
    }

    // address bytes of chunks 4q .. 4q+3 (computed once per group, passed to addr)
    __device__ __forceinline__ uint32_t group_bytes(int q) const { return coset_bytes(H, bankbytes, q); }

    // LDS byte address of stage S (0..2) at chunk t, hq = group_bytes(t >> 2)
    template <int S>
    __device__ __forceinline__ uint32_t addr(int t, uint32_t hq) const {
        const int e = t & 3;
        if constexpr (S == 0) {
            if constexpr (W1 == 8) return __builtin_amdgcn_perm(r1[t >> 2], hq, 0x0c0c0000u | ((4u + e) << 8) | e);
            else {
                const uint32_t f = field_of<W1 - 1>(r1, t) | (__builtin_amdgcn_ubfe(r0, t, 1) << (W1 - 1));
                return __builtin_amdgcn_perm(f, hq, 0x0c0c0400u | e);
            }
        } else if constexpr (S == 1) {
            if constexpr (W2 == 8) return __builtin_amdgcn_perm(r2[t >> 2], hq, 0x0c0c0000u | ((4u + e) << 8) | e);
            else return __builtin_amdgcn_perm(field_of<W2>(r2, t), hq, 0x0c0c0400u | e);
        } else {
            return __builtin_amdgcn_perm(r3[t >> 2], hq, 0x0c0c0000u | ((4u + e) << 8) | e);
        }
    }
};

// ------------------------------------------------------------------------------------------------ 16-byte loads
// The same lane-slice loaded in 16-byte groups: a wave loads group q of its half-slice as one contiguous
// 16-byte-per-lane access (512 bytes per 32 lanes, whole cache lines per instruction). Field k of a region is
// chunk k (the device payload is in chunk order), so the activation chunk of step k is the same for all lanes.
template <int W, int OFF, int NW>
__device__ __forceinline__ uint32_t field_at(const uint32_t (&w)[NW], int k) {
    const int pos = W * k, wi = OFF + (pos >> 5), bb = pos & 31;
    if (bb + W <= 32) return __builtin_amdgcn_ubfe(w[wi], bb, W);
    return __builtin_amdgcn_alignbit(w[wi + 1], w[wi], bb) & ((1u << W) - 1u);
}

template <int C>
struct QuadSlice {
    static constexpr int W1 = w1_of(C), W2 = w2_of(C), W3 = w3_of(C), NW = nw_of(C);
    static constexpr int NQ = NW / 4, NP = (NW % 4) / 2;   // 16-byte groups and a trailing word pair per lane
    static constexpr int O1 = W1 == 8 ? 0 : 1, O2 = W1, O3 = W1 + W2;   // first word of each stage's fields
    uint32_t w[NW];
    uint32_t s;   // fp16 row scale, zero-extended by its load

    // lane byte offsets in the device layout (dev_word): of its first 16-byte group, and of its trailing pair
    static __device__ __forceinline__ uint32_t quad_offset(int hs, int j) { return (uint32_t)(hs * NW * 128 + 16 * j); }
    static __device__ __forceinline__ uint32_t pair_offset(int hs, int j) { return (uint32_t)(hs * NW * 128 + 512 * NQ + 8 * j); }

    // vo = quad_offset: group q sits 512 q bytes further; vp = pair_offset (classes with NW % 4 == 2)
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rd, uint32_t toff, uint32_t vo, uint32_t vp,
                                         __amdgpu_buffer_rsrc_t rs, uint32_t soff, uint32_t vs) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(rd, vo + 512u * q, toff, kBufNT);
            w[4 * q] = v[0];
            w[4 * q + 1] = v[1];
            w[4 * q + 2] = v[2];
            w[4 * q + 3] = v[3];
        }
        if constexpr (NP) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(rd, vp, toff, kBufNT);
            w[4 * NQ] = v[0];
            w[4 * NQ + 1] = v[1];
        }
        s = __builtin_amdgcn_raw_buffer_load_b16(rs, vs, soff, kBufNT);
    }

    // coset bits, chunk order
    __device__ __forceinline__ uint32_t coset_bits() const {
        uint32_t z;
        if constexpr (W1 == 8) {
            uint32_t r[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) r[i] = w[i];
            z = labels_from_bytes(r);
        } else {
            z = w[0];
        }
        return trellis_coset_bits(z);
    }

    // LDS byte address of stage S at chunk k, hq = coset_bytes(H, bankbytes, k >> 2)
    template <int S>
    __device__ __forceinline__ uint32_t addr(int k, uint32_t hq) const {
        const int e = k & 3;
        if constexpr (S == 0) {
            if constexpr (W1 == 8) return __builtin_amdgcn_perm(w[k >> 2], hq, 0x0c0c0000u | ((4u + e) << 8) | e);
            else {
                const uint32_t f = field_at<W1 - 1, O1>(w, k) | (__builtin_amdgcn_ubfe(w[0], k, 1) << (W1 - 1));
                return __builtin_amdgcn_perm(f, hq, 0x0c0c0400u | e);
            }
        } else if constexpr (S == 1) {
            if constexpr (W2 == 8) return __builtin_amdgcn_perm(w[O2 + (k >> 2)], hq, 0x0c0c0000u | ((4u + e) << 8) | e);
            else return __builtin_amdgcn_perm(field_at<W2, O2>(w, k), hq, 0x0c0c0400u | e);
        } else {
            return __builtin_amdgcn_perm(w[O3 + (k >> 2)], hq, 0x0c0c0000u | ((4u + e) << 8) | e);
        }
    }
};

// ------------------------------------------------------------------------------------------------ any class
// Raw payload words of one lane-slice (any class up to NWMAX words), plus the lane's fp16 row scale: issued ahead
// of use, then decoded into an AnySlice (labels, trellis).
template <int NWMAX>
struct AnyRaw {
    uint32_t w[NWMAX];
    uint32_t s;   // fp16 row scale, zero-extended by its load

    template <int W, int WB, int NW>
    __device__ __forceinline__ void region(const uint32_t *__restrict__ p, int j) {
#pragma unroll
        for (int m = 0; m < W; ++m) w[WB + m] = __builtin_nontemporal_load(p + dev_word(WB + m, j, NW));
    }
    // p = the tile's half-slice base (tile payload + hs * NW * 32 words)
    template <int C>
    __device__ __forceinline__ void load(const uint32_t *__restrict__ p, int j, const uint16_t *__restrict__ srow) {
        constexpr int W1 = w1_of(C), W2 = w2_of(C), W3 = w3_of(C), NW = nw_of(C);
        if constexpr (W1 == 8) region<8, 0, NW>(p, j);
        else {
            w[0] = __builtin_nontemporal_load(p + dev_word(0, j, NW));
            region<W1 - 1, 1, NW>(p, j);
        }
        if constexpr (W2 > 0) region<W2, W1, NW>(p, j);
        if constexpr (W3 > 0) region<W3, W1 + W2, NW>(p, j);
        s = srow[j];
    }
};

// Lane-slice words of any class up to NWMAX words (chunk order), plus the coset bits in chunk order. Region
// layout as stored: [label word if W1 < 8] stage-1 fields, stage 2, stage 3.
template <int NWMAX>
struct AnySlice {
    uint32_t r[NWMAX];
    uint32_t H;
    uint32_t s;   // fp16 row scale, zero-extended by its load

    template <int W, int WB>
    __device__ __forceinline__ void copy(const AnyRaw<NWMAX> &raw) {
#pragma unroll
        for (int i = 0; i < W; ++i) r[WB + i] = raw.w[WB + i];
    }
    template <int C>
    __device__ __forceinline__ void from_raw(const AnyRaw<NWMAX> &raw) {
        constexpr int W1 = w1_of(C), W2 = w2_of(C), W3 = w3_of(C);
        uint32_t z;
        if constexpr (W1 == 8) {
            copy<8, 0>(raw);
            uint32_t R[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) R[i] = r[i];
            z = labels_from_bytes(R);
        } else {
            r[0] = raw.w[0];
            z = r[0];
            copy<W1 - 1, 1>(raw);
        }
        if constexpr (W2 > 0) copy<W2, W1>(raw);
        if constexpr (W3 > 0) copy<W3, W1 + W2>(raw);
        H = trellis_coset_bits(z);
        s = raw.s;
    }

    // stage-S field of chunk t (W1 < 8: the label bit on top of the W1 - 1 stored bits)
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
                else f = __builtin_amdgcn_alignbit(r[1 + (wi % W)], r[wi], bb) & ((1u << W) - 1u);
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

    // LDS byte address of stage S at chunk t in the replicated table (p8x_lane.h layout: (f << 8) | (h << 7) |
    // (bank << 2)); hq = coset_bytes(H, bankbytes, t >> 2) holds the (h << 7) | (bank << 2) byte of each chunk
    template <int C, int S>
    __device__ __forceinline__ uint32_t addr(int t, uint32_t hq) const {
        constexpr int W1 = w1_of(C), W2 = w2_of(C);
        const int e = t & 3;
        if constexpr (S == 0) {
            if constexpr (W1 == 8) return __builtin_amdgcn_perm(r[t >> 2], hq, 0x0c0c0000u | ((4u + e) << 8) | e);
            else {
                constexpr int W = W1 - 1;
                const int pos = W * t, wi = 1 + (pos >> 5), bb = pos & 31;
                uint32_t f;
                if (bb + W <= 32) f = __builtin_amdgcn_ubfe(r[wi], bb, W);
                else f = __builtin_amdgcn_alignbit(r[1 + (wi % W)], r[wi], bb) & ((1u << W) - 1u);
                f |= __builtin_amdgcn_ubfe(r[0], t, 1) << W;
                return __builtin_amdgcn_perm(f, hq, 0x0c0c0400u | e);
            }
        } else if constexpr (S == 1) {
            if constexpr (W2 == 8) return __builtin_amdgcn_perm(r[W1 + (t >> 2)], hq, 0x0c0c0000u | ((4u + e) << 8) | e);
            else {
                const int pos = W2 * t, wi = pos >> 5, bb = pos & 31;
                uint32_t f;
                if (bb + W2 <= 32) f = __builtin_amdgcn_ubfe(r[W1 + wi], bb, W2);
                else f = __builtin_amdgcn_alignbit(r[W1 + (wi + 1) % W2], r[W1 + wi], bb) & ((1u << W2) - 1u);
                return __builtin_amdgcn_perm(f, hq, 0x0c0c0400u | e);
            }
        } else {
            return __builtin_amdgcn_perm(r[W1 + W2 + (t >> 2)], hq, 0x0c0c0000u | ((4u + e) << 8) | e);
        }
    }
};

// class dispatch over the classes of mask CM (uniform per wave: the tile's class)
template <int CM, int NWMAX>
__device__ __forceinline__ void load_any(AnyRaw<NWMAX> &raw, int c, const uint32_t *p, int j, const uint16_t *srow) {
    switch (c) {
        case 1: if constexpr ((CM >> 1) & 1) raw.template load<1>(p, j, srow); break;
        case 2: if constexpr ((CM >> 2) & 1) raw.template load<2>(p, j, srow); break;
        case 3: if constexpr ((CM >> 3) & 1) raw.template load<3>(p, j, srow); break;
        case 4: if constexpr ((CM >> 4) & 1) raw.template load<4>(p, j, srow); break;
        case 5: if constexpr ((CM >> 5) & 1) raw.template load<5>(p, j, srow); break;
        case 6: if constexpr ((CM >> 6) & 1) raw.template load<6>(p, j, srow); break;
        case 7: if constexpr ((CM >> 7) & 1) raw.template load<7>(p, j, srow); break;
        default: break;
    }
}

template <int CM, int NWMAX>
__device__ __forceinline__ void prepare_any(AnySlice<NWMAX> &ls, int c, const AnyRaw<NWMAX> &raw) {
    switch (c) {
        case 1: if constexpr ((CM >> 1) & 1) ls.template from_raw<1>(raw); break;
        case 2: if constexpr ((CM >> 2) & 1) ls.template from_raw<2>(raw); break;
        case 3: if constexpr ((CM >> 3) & 1) ls.template from_raw<3>(raw); break;
        case 4: if constexpr ((CM >> 4) & 1) ls.template from_raw<4>(raw); break;
        case 5: if constexpr ((CM >> 5) & 1) ls.template from_raw<5>(raw); break;
        case 6: if constexpr ((CM >> 6) & 1) ls.template from_raw<6>(raw); break;
        case 7: if constexpr ((CM >> 7) & 1) ls.template from_raw<7>(raw); break;
        default: break;
    }
}

__device__ __forceinline__ int sext8(uint32_t w, int e) { return (int)(int8_t)(w >> (8 * e)); }

}  // namespace p8x
