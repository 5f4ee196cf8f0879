// p8x_format.h -- Pingala-8 native tensor format constants, shared by host and device code.
//
// Tile = 32 sorted rows x 256 columns; two 128-column half-slices per tile; one lane (row) of a
// half-slice holds NW(c) payload words = 32 fields per stage (stage widths W1/W2/W3 by class c).
// Class tables and shifts: CPU.patch:188-195 (patches/llama_cpu_vs_7ac59a6.patch).
// Slot layout: CPU.patch:8-51 and :3817-3824.
#pragma once
#include <stddef.h>
#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define P8X_HD __host__ __device__ __forceinline__
#else
#define P8X_HD inline
#endif

namespace p8x {

constexpr uint32_t kMagic0 = 0x4E525656u;   // trailer word 0
constexpr uint32_t kMagic1 = 0x31354952u;   // trailer word 1
constexpr uint32_t kNS = 108u;              // 8-state trellis, u_t = z_t ^ u_{t-1} ^ u_{t-3}, h_t = u_{t-2}
constexpr uint32_t kTRL = 2u;               // stage-1 index kept whole for W1 = 8
constexpr size_t kHeaderBytes = 2064;       // A | B | c, NS, TRL, word 515

P8X_HD constexpr int w1_of(int c) { return c == 0 ? 0 : c == 1 ? 4 : c == 2 ? 6 : 8; }
P8X_HD constexpr int w2_of(int c) { return c == 4 ? 2 : c == 5 ? 4 : c >= 6 ? 8 : 0; }
P8X_HD constexpr int w3_of(int c) { return c == 7 ? 8 : 0; }
P8X_HD constexpr int sh1_of(int c) { return c == 4 ? 2 : c == 5 ? 3 : c == 6 ? 2 : c == 7 ? 4 : 0; }
P8X_HD constexpr int sh2_of(int c) { return c == 7 ? 2 : 0; }
P8X_HD constexpr int nw_of(int c) { return w1_of(c) + w2_of(c) + w3_of(c); }
P8X_HD constexpr int nstage_of(int c) { return c == 0 ? 0 : c <= 3 ? 1 : c <= 6 ? 2 : 3; }

P8X_HD constexpr size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }

// Payload word i of lane j inside a half-slice of a class with NW words per lane.
// In the file (and the reference's memory), word pairs of the 32 lanes interleave: [i >> 1][j][i & 1]
// (CPU.patch:292-297). p8x_prepare re-lays each tile's payload on the device so that a lane's words come in 16-byte
// groups: the first NW & ~3 words as [i >> 2][j][i & 3] (512 contiguous bytes per group of the 32 lanes), the last two
// of NW = 6 and 10 as in the file after them ([j][i & 1]). Every kernel reads this device layout; one buffer load of
// 16 bytes per lane then fetches a lane's four consecutive words.
P8X_HD constexpr int file_word(int i, int j) { return ((i >> 1) << 6) + 2 * j + (i & 1); }
P8X_HD constexpr int dev_word(int i, int j, int nw) {
    return i < (nw & ~3) ? ((i >> 2) << 7) + 4 * j + (i & 3) : ((nw & ~3) << 5) + 2 * j + (i & 1);
}
P8X_HD constexpr size_t offset_S(size_t nt) { return kHeaderBytes + 4 * nt; }
P8X_HD constexpr size_t offset_D(size_t nt) { return align16(kHeaderBytes + 68 * nt); }

// fp16 bits -> f32 (exact; on the GPU the v_cvt_f32_f16 instruction, also exact for subnormals)
P8X_HD float half_to_float(uint16_t h) {
#if defined(__HIP_DEVICE_COMPILE__)
    return (float)__builtin_bit_cast(_Float16, h);
#endif
    const uint32_t sign = (uint32_t)(h >> 15) << 31, ex = (h >> 10) & 31u, man = h & 1023u;
    uint32_t bits;
    if (ex == 0) {
        float f = (float)man * (1.0f / 16777216.0f);
        bits = __builtin_bit_cast(uint32_t, f) | sign;
    } else if (ex == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    return __builtin_bit_cast(float, bits);
}

// f32 -> fp16 bits, round to nearest even
P8X_HD uint16_t float_to_half(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    const uint32_t sign = (u >> 16) & 0x8000u, fe = (u >> 23) & 255u, man = u & 0x7fffffu;
    const int e = (int)fe - 112;
    if (fe == 255) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        const uint32_t m = man | 0x800000u;
        const int sh = 14 - e;
        uint32_t q = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = man >> 13, he = (uint32_t)e;
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) {
        q++;
        if (q == 0x400u) { q = 0; he++; if (he >= 31) return (uint16_t)(sign | 0x7c00u); }
    }
    return (uint16_t)(sign | (he << 10) | q);
}

// f32 -> bf16 bits, round to nearest even (NaN kept quiet)
P8X_HD uint16_t float_to_bf16(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

P8X_HD float bf16_to_float(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// bytewise int8x4 add without carries between bytes (the CPU core's coset add, CPU.patch:221)
P8X_HD uint32_t add_bytes(uint32_t a, uint32_t b) {
    return ((a & 0x7f7f7f7fu) + (b & 0x7f7f7f7fu)) ^ ((a ^ b) & 0x80808080u);
}

}  // namespace p8x
