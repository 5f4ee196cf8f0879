// p8x_synth.cpp -- host-side producers of tensor slots (not on the hot path).
//
// p8x_synth_random: random valid codes, the reference's timing arm (CPU.patch:4391-4458).
// p8x_quantize_tensor: class-3 plain-MSE encoder = the identity-Hessian special case of the reference
// encoder (research/detail/r59_sourcecoding.py:39-98, research/detail/r48k.py:213-239):
//   rotated target T = FWHT256(W * c * sg) / 16 per 256-block (the inverse of the decoder's transform),
//   S = fp16(1.05 * rms(T) / 23.557), X = T / S in codebook units; per 4-vector the best entry of each
//   half of the codebook (index MSB b = 0/1) for coset h = 0/1; an 8-state Viterbi per 128-column
//   half-slice (start state 0, free end) with edge (s, b) -> ((s << 1) | (b ^ par(s & 5))) & 7, h = par(s & 2);
//   clamp delta = clamp(W_dec, +-wmax) - W_dec for |W_dec| > wmax = fp16(1.001 max|W|) (r51_delta.py:14).
// Payload packing follows the kernel byte layout: lane j of a half-slice stores chunk t = (j + k) & 31 as
// its k-th 8-bit field, words interleaved [i >> 1][j][i & 1] (research/detail/r51_transcode.py:28-69).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/p8x.h"
#include "p8x_codebook.h"
#include "p8x_format.h"

using namespace p8x;

namespace {

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

size_t need_bytes(size_t kbytes, size_t rows, size_t K, size_t nd) {
    return align16(kbytes) + align16(8 * nd) + align16(2 * K) + 2 * align16(2 * rows) + 256 + 32 + 64;
}

struct Side {
    std::vector<uint16_t> c16;
    std::vector<int16_t> prm;
    std::vector<int8_t> sg;
    std::vector<uint16_t> drow, dcol;
    std::vector<float> dval;
};

// lay out header + M + S + payload (already in `buf` from offset_D) and the side regions; returns slot size
size_t write_slot(uint8_t *buf, int rows, int K, const uint32_t *A, uint32_t cs, const std::vector<uint32_t> &M,
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

void fwht256_d(double *v) {
    for (int h = 1; h < 256; h <<= 1)
        for (int i = 0; i < 256; ++i)
            if (!(i & h)) { const double a = v[i], b = v[i + h]; v[i] = a + b; v[i + h] = a - b; }
    for (int i = 0; i < 256; ++i) v[i] *= 0.0625;
}

}  // namespace

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

int p8x_quantize_tensor(const float *W, int rows, int K, const uint16_t *c16, uint64_t sign_seed, void *out, size_t cap, size_t *n_out) {
    if (!W || rows <= 0 || K <= 0 || rows % 32 || K % 256 || rows >= 32768 || !n_out) return P8X_ERR_ARG;
    const int ng = rows / 32, nb = K / 256;
    const size_t nt = (size_t)ng * nb, words = nt * 512;
    Side sd;
    sd.c16.resize(K);
    for (int k = 0; k < K; ++k) sd.c16[k] = c16 ? c16[k] : (uint16_t)0x3C00;
    sd.sg.resize(256);
    {
        Rng r(sign_seed);
        for (int i = 0; i < 256; ++i) sd.sg[i] = (r.next() & 1) ? 1 : -1;
    }
    sd.prm.resize(rows);
    for (int r = 0; r < rows; ++r) sd.prm[r] = (int16_t)r;
    // codebook with coset folded: value of (f, h), as the decoder sees it (bytewise)
    float cb[2][256][4];
    for (int h = 0; h < 2; ++h)
        for (int f = 0; f < 256; ++f) {
            const uint32_t v = h ? add_bytes(kShippedA[f], kShippedC) : kShippedA[f];
            for (int e = 0; e < 4; ++e) cb[h][f][e] = (float)(int8_t)(v >> (8 * e));
        }
    std::vector<uint16_t> S((size_t)nb * rows);
    std::vector<uint8_t> idx((size_t)rows * K / 4);   // chosen 8-bit entry per (row, chunk), natural order
    std::vector<double> wdec((size_t)rows * K);
    float amax = 0.f;
    for (size_t i = 0; i < (size_t)rows * K; ++i) amax = std::max(amax, std::fabs(W[i]));
    const int nthr = std::max(1, std::min(16, (int)std::thread::hardware_concurrency()));
    std::vector<std::thread> th;
    for (int tI = 0; tI < nthr; ++tI)
        th.emplace_back([&, tI] {
            std::vector<double> T(256), rec(256);
            for (int r = tI; r < rows; r += nthr) {
                for (int b = 0; b < nb; ++b) {
                    for (int i = 0; i < 256; ++i) {
                        const int k = 256 * b + i;
                        T[i] = (double)W[(size_t)r * K + k] * (double)half_to_float(sd.c16[k]) * (double)sd.sg[i];
                    }
                    fwht256_d(T.data());
                    double ss = 0;
                    for (int i = 0; i < 256; ++i) ss += T[i] * T[i];
                    const double rms = std::sqrt(ss / 256.0);
                    const uint16_t s16 = float_to_half((float)(1.05 * rms / 23.557000147255682));
                    S[(size_t)b * rows + r] = s16;
                    const double sc = half_to_float(s16);
                    for (int hs = 0; hs < 2; ++hs) {
                        // per chunk: best entry and cost for (h, msb)
                        double cost[32][2][2];
                        uint8_t best[32][2][2];
                        for (int t = 0; t < 32; ++t) {
                            double x[4];
                            for (int e = 0; e < 4; ++e) x[e] = sc > 0 ? T[128 * hs + 4 * t + e] / sc : 0.0;
                            for (int h = 0; h < 2; ++h)
                                for (int m = 0; m < 2; ++m) {
                                    double bc = 1e300; int bf = 128 * m;
                                    for (int f = 128 * m; f < 128 * m + 128; ++f) {
                                        double dd = 0;
                                        for (int e = 0; e < 4; ++e) { const double q = x[e] - cb[h][f][e]; dd += q * q; }
                                        if (dd < bc) { bc = dd; bf = f; }
                                    }
                                    cost[t][h][m] = bc; best[t][h][m] = (uint8_t)bf;
                                }
                        }
                        // Viterbi over 8 states (bit 0 = u_{t-1}, bit 1 = u_{t-2}, bit 2 = u_{t-3})
                        double pmv[8];
                        uint8_t bp[32][8];   // predecessor state << 1 | msb
                        for (int s = 0; s < 8; ++s) pmv[s] = s == 0 ? 0.0 : 1e300;
                        for (int t = 0; t < 32; ++t) {
                            double nm[8];
                            for (int s = 0; s < 8; ++s) nm[s] = 1e300;
                            for (int s = 0; s < 8; ++s) {
                                if (pmv[s] >= 1e300) continue;
                                const int h = (s >> 1) & 1, par = (s ^ (s >> 2)) & 1;
                                for (int m = 0; m < 2; ++m) {
                                    const int u = m ^ par, s2 = ((s << 1) | u) & 7;
                                    const double c2 = pmv[s] + cost[t][h][m];
                                    if (c2 < nm[s2]) { nm[s2] = c2; bp[t][s2] = (uint8_t)((s << 1) | m); }
                                }
                            }
                            for (int s = 0; s < 8; ++s) pmv[s] = nm[s];
                        }
                        int s = 0;
                        for (int s2 = 1; s2 < 8; ++s2) if (pmv[s2] < pmv[s]) s = s2;
                        for (int t = 31; t >= 0; --t) {
                            const int prev = bp[t][s] >> 1, m = bp[t][s] & 1, h = (prev >> 1) & 1;
                            const uint8_t f = best[t][h][m];
                            idx[((size_t)r * K + 256 * b + 128 * hs) / 4 + t] = f;
                            for (int e = 0; e < 4; ++e) rec[128 * hs + 4 * t + e] = (double)cb[h][f][e] * sc;
                            s = prev;
                        }
                    }
                    fwht256_d(rec.data());   // decoded weight in fp64 (for the clamp delta)
                    for (int i = 0; i < 256; ++i) {
                        const int k = 256 * b + i;
                        wdec[(size_t)r * K + k] = rec[i] * (double)sd.sg[i] / (double)half_to_float(sd.c16[k]);
                    }
                }
            }
        });
    for (auto &x : th) x.join();
    const double wmax = half_to_float(float_to_half(amax * 1.001f));
    for (int r = 0; r < rows; ++r)
        for (int k = 0; k < K; ++k) {
            const double v = wdec[(size_t)r * K + k];
            if (std::fabs(v) > wmax) {
                sd.drow.push_back((uint16_t)r); sd.dcol.push_back((uint16_t)k);
                sd.dval.push_back((float)(std::max(-wmax, std::min(wmax, v)) - v));
            }
        }
    if (sd.drow.size() > 65535) return P8X_ERR_UNSUPPORTED;
    const size_t need = need_bytes(offset_D(nt) + 4 * words, (size_t)rows, (size_t)K, sd.drow.size());
    *n_out = need;
    if (!out || cap < need) return P8X_ERR_ARG;
    uint8_t *buf = (uint8_t *)out;
    std::vector<uint32_t> M(nt);
    for (size_t i = 0; i < nt; ++i) M[i] = (uint32_t)(i * 512) | (3u << 29);
    uint32_t *D = reinterpret_cast<uint32_t *>(buf + offset_D(nt));
    for (int g = 0; g < ng; ++g)
        for (int b = 0; b < nb; ++b) {
            uint32_t *tile = D + ((size_t)g * nb + b) * 512;
            for (int hs = 0; hs < 2; ++hs)
                for (int j = 0; j < 32; ++j) {
                    const uint8_t *ch = &idx[((size_t)(32 * g + j) * K + 256 * b + 128 * hs) / 4];
                    uint32_t lw[8] = {0};
                    for (int k = 0; k < 32; ++k) lw[k >> 2] |= (uint32_t)ch[(j + k) & 31] << (8 * (k & 3));
                    for (int i = 0; i < 8; ++i) tile[hs * 256 + (i >> 1) * 64 + 2 * j + (i & 1)] = lw[i];
                }
        }
    write_slot(buf, rows, K, kShippedA, kShippedC, M, S, words, sd);
    return P8X_OK;
}

}  // extern "C"
