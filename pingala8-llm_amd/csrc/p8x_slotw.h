// p8x_slotw.h -- host-side helpers shared by the slot producers (random timing slots and the encoders).
// Slot layout: header A|B|c|NS|TRL|0, tile words M, fp16 scales S[b][r], 16-aligned payload D, then the side
// regions placed top-down from the slot end (delta, c16, prm, pinv, signs, trailer) (CPU.patch:8-51, :3817-3824).
#pragma once
#include <cstring>
#include <vector>

#include "p8x_format.h"

namespace p8x {
namespace slotw {

struct Rng {   // splitmix64
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniform() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }
};

inline size_t need_bytes(size_t kbytes, size_t rows, size_t K, size_t nd) {
    return align16(kbytes) + align16(8 * nd) + align16(2 * K) + 2 * align16(2 * rows) + 256 + 32 + 64;
}

struct Side {
    std::vector<uint16_t> c16;
    std::vector<int16_t> prm;   // sorted row -> original row
    std::vector<int8_t> sg;
    std::vector<uint16_t> drow, dcol;
    std::vector<float> dval;
};

// Lays out header + M + S, zero-fills the gaps and writes the side regions; the payload (payload_words words)
// must already be in `buf` from offset_D. Returns the slot size.
inline size_t write_slot(uint8_t *buf, int rows, int K, const uint32_t *A, uint32_t cs, const std::vector<uint32_t> &M,
                         const std::vector<uint16_t> &S, size_t payload_words, const Side &sd) {
    const size_t nt = M.size(), nd = sd.drow.size();
    const size_t kbytes = offset_D(nt) + 4 * payload_words;
    const size_t n = need_bytes(kbytes, rows, K, nd);
    uint32_t *w = reinterpret_cast<uint32_t *>(buf);
    memcpy(w, A, 1024);
    memcpy(w + 256, A, 1024);
    w[512] = cs; w[513] = kNS; w[514] = kTRL; w[515] = 0;
    memcpy(buf + kHeaderBytes, M.data(), 4 * nt);
    memcpy(buf + offset_S(nt), S.data(), 2 * S.size());
    memset(buf + kHeaderBytes + 68 * nt, 0, offset_D(nt) - (kHeaderBytes + 68 * nt));
    memset(buf + kbytes, 0, n - kbytes);
    const size_t t = n - 32, sgo = t - 256;
    const size_t q = (sgo - 2 * (size_t)rows) & ~(size_t)15, p = (q - 2 * (size_t)rows) & ~(size_t)15;
    const size_t c = (p - 2 * (size_t)K) & ~(size_t)15, e = (c - 8 * nd) & ~(size_t)15;
    if (nd) {
        memcpy(buf + e, sd.drow.data(), 2 * nd);
        memcpy(buf + e + 2 * nd, sd.dcol.data(), 2 * nd);
        memcpy(buf + e + 4 * nd, sd.dval.data(), 4 * nd);
    }
    memcpy(buf + c, sd.c16.data(), 2 * (size_t)K);
    memcpy(buf + p, sd.prm.data(), 2 * (size_t)rows);
    std::vector<int16_t> pinv(rows);
    for (int r = 0; r < rows; ++r) pinv[sd.prm[r]] = (int16_t)r;
    memcpy(buf + q, pinv.data(), 2 * (size_t)rows);
    memcpy(buf + sgo, sd.sg.data(), 256);
    const uint32_t tr[8] = {kMagic0, kMagic1, (uint32_t)kbytes, (uint32_t)nd, (uint32_t)rows, (uint32_t)K, kNS, 1u};
    memcpy(buf + t, tr, 32);
    return n;
}

// 256-point Walsh-Hadamard transform scaled by 1/16 (an involution), in double
inline void fwht256_d(double *v) {
    for (int h = 1; h < 256; h <<= 1)
        for (int i = 0; i < 256; ++i)
            if (!(i & h)) { const double a = v[i], b = v[i + h]; v[i] = a + b; v[i + h] = a - b; }
    for (int i = 0; i < 256; ++i) v[i] *= 0.0625;
}

// the same in f32 with the dequantizer's butterfly order (CPU.patch:533-537)
inline void fwht256_f(float *v) {
    for (int h = 1; h < 256; h <<= 1)
        for (int i = 0; i < 256; ++i)
            if (!(i & h)) { const float a = v[i], b = v[i + h]; v[i] = a + b; v[i + h] = a - b; }
    for (int i = 0; i < 256; ++i) v[i] *= 0.0625f;
}

// Hadamard signs (+-1) drawn from a seed
inline std::vector<int8_t> seeded_signs(uint64_t seed) {
    std::vector<int8_t> sg(256);
    Rng r(seed);
    for (int i = 0; i < 256; ++i) sg[i] = (r.next() & 1) ? 1 : -1;
    return sg;
}

}  // namespace slotw
}  // namespace p8x
