// p8x_synth.cpp -- host-side producers of tensor slots (not on the hot path).
//
// p8x_synth_random: random valid codes, the reference's timing arm (CPU.patch:4391-4458).
// The encoders of real weights (p8x_encode_tensor and its class-3 special case p8x_quantize_tensor) are in
// p8x_encode.cpp.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/p8x.h"
#include "p8x_codebook.h"
#include "p8x_format.h"
#include "p8x_slotw.h"

using namespace p8x;

using namespace p8x::slotw;

extern "C" {

size_t p8x_slot_bytes(int rows, int K, const size_t class_tiles[8], int nd) {
    size_t words = 0, nt = 0;
    for (int c = 0; c < 8; ++c) { words += class_tiles[c] * 64 * (size_t)nw_of(c); nt += class_tiles[c]; }
    return need_bytes(offset_D(nt) + 4 * words, (size_t)rows, (size_t)K, (size_t)nd);
}

int p8x_synth_random(uint64_t seed, int rows, int K, const double *class_p, int codebook, int nd, int permute_rows,
                     void *out, size_t cap, size_t *n_out) {
    if (rows <= 0 || K <= 0 || rows % 32 || K % 256 || rows >= 32768 || nd < 0 || !class_p || !n_out) return P8X_ERR_ARG;
    const int ng = rows / 32, nb = K / 256;
    const size_t nt = (size_t)ng * nb;
    if ((size_t)nd > (size_t)rows * K) return P8X_ERR_ARG;
    Rng rng(seed);
    double cum[8], tot = 0;
    for (int c = 0; c < 8; ++c) { tot += class_p[c] > 0 ? class_p[c] : 0; cum[c] = tot; }
    if (tot <= 0) return P8X_ERR_ARG;
    std::vector<uint32_t> M(nt);
    size_t words = 0, hist[8] = {0};
    for (size_t i = 0; i < nt; ++i) {
        const double u = rng.uniform() * tot;
        int c = 0;
        while (c < 7 && u >= cum[c]) ++c;
        M[i] = (uint32_t)words | ((uint32_t)c << 29);
        words += (size_t)64 * nw_of(c);
        hist[c]++;
    }
    if (words >= (1u << 29)) return P8X_ERR_ARG;
    const size_t need = p8x_slot_bytes(rows, K, hist, nd);
    *n_out = need;
    if (!out || cap < need) return P8X_ERR_ARG;
    uint8_t *buf = (uint8_t *)out;
    uint32_t A[256], cs;
    if (codebook == 0) { memcpy(A, kShippedA, sizeof A); cs = kShippedC; }
    else {
        for (int f = 0; f < 256; ++f) {
            A[f] = 0;
            for (int e = 0; e < 4; ++e) A[f] |= (uint32_t)(uint8_t)(int8_t)((int)(rng.next() % 129) - 64) << (8 * e);
        }
        cs = 0;
        for (int e = 0; e < 4; ++e) cs |= (uint32_t)(uint8_t)(int8_t)((int)(rng.next() % 33) - 16) << (8 * e);
    }
    std::vector<uint16_t> S((size_t)nb * rows);
    for (int b = 0; b < nb; ++b)
        for (int r = 0; r < rows; ++r) {
            const uint32_t c = M[(size_t)(r / 32) * nb + b] >> 29;
            S[(size_t)b * rows + r] = c ? float_to_half((float)(2e-4 + rng.uniform() * 1e-4)) : 0;
        }
    uint32_t *D = reinterpret_cast<uint32_t *>(buf + offset_D(nt));
    {   // payload: independent streams per thread chunk keep generation fast and deterministic
        const size_t nthr = std::min<size_t>(8, std::max<size_t>(1, words / (1 << 22)));
        std::vector<std::thread> th;
        for (size_t tI = 0; tI < nthr; ++tI)
            th.emplace_back([&, tI] {
                Rng r2(seed ^ (0xA5A5A5A5ull * (tI + 1)));
                const size_t lo = words * tI / nthr, hi = words * (tI + 1) / nthr;
                for (size_t i = lo; i < hi; i += 2) {
                    const uint64_t v = r2.next();
                    D[i] = (uint32_t)v;
                    if (i + 1 < hi) D[i + 1] = (uint32_t)(v >> 32);
                }
            });
        for (auto &x : th) x.join();
    }
    Side sd;
    sd.c16.resize(K);
    for (int k = 0; k < K; ++k) sd.c16[k] = float_to_half((float)(0.5 + 1.5 * rng.uniform()));
    sd.prm.resize(rows);
    for (int r = 0; r < rows; ++r) sd.prm[r] = (int16_t)r;
    if (permute_rows)
        for (int r = rows - 1; r > 0; --r) std::swap(sd.prm[r], sd.prm[rng.next() % (uint64_t)(r + 1)]);
    sd.sg.resize(256);
    for (int i = 0; i < 256; ++i) sd.sg[i] = (rng.next() & 1) ? 1 : -1;
    if (nd) {
        std::vector<uint64_t> pos;
        while ((int)pos.size() < nd) {
            const uint64_t p = rng.next() % ((uint64_t)rows * K);
            if (std::find(pos.begin(), pos.end(), p) == pos.end()) pos.push_back(p);
        }
        std::sort(pos.begin(), pos.end());
        for (uint64_t p : pos) {
            sd.drow.push_back((uint16_t)(p / K));
            sd.dcol.push_back((uint16_t)(p % K));
            sd.dval.push_back((float)((rng.uniform() - 0.5) * 0.1));
        }
    }
    write_slot(buf, rows, K, A, cs, M, S, words, sd);
    return P8X_OK;
}

}  // extern "C"
