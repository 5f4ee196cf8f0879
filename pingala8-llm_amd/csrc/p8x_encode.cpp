// p8x_encode.cpp -- host encoder of Pingala-8 slots: every class 0..7, LDLQ (Hessian-weighted) error feedback,
// rate allocation of classes over tiles. Restates the reference's tensor encoder (research/detail/r48k.py):
//   k_tensor (:213-239): rotated target Y = FWHT256(W * c * sg) / 16 per 256-block; rotated input second moment
//     Hp = R diag(1/c) H diag(1/c) R^T, damped by damp * mean(diag Hp); U = upper Cholesky factor of Hp^-1;
//     rows sorted by ascending mean log block energy; classes by alloc(); S = fp16(alpha * rms_block / G[class]).
//   alloc (:121-141): Lagrangian bisection on lambda, then greedy upgrades by distortion gain per bit within the budget;
//     tile-blocks that hold the n largest |W| are held at class >= 6.
//   encode (:104-118): 128-column slices in order; error feedback W[:, i1:] -= E @ U[i0:i1, i1:] after each slice.
//   vit_k (:57-95): per-survivor Viterbi over the 8-state coset trellis of a 128-column slice (start state 0, free
//     end), per 4-column step metric |(x/S - off(h) - cw) A4|^2 with A4 = inverse of U's 4x4 diagonal block, and the
//     survivor's error e = (x - S cw) A4 fed back into its own remaining targets: X[j+4:] -= e U[j:j+4, j+4:].
//   best_cw (:33-55): per stage-1 half (stored MSB 0/1): classes 1-3 nearest entry; classes 4-6 the 4 nearest stage-1
//     entries, each with its nearest stage-2 entry; class 7 additionally the 4 nearest stage-2 entries per stage-1
//     candidate, each with its nearest stage-3 entry.
//   zero_ldlq (:97-102): class 0 (no code) passes its whole error on.
// Ties go to the lower index (the first state, the first candidate); floating-point operations are done one at a time
// in a fixed order, so the encoder's choices are a deterministic function of its inputs.
// The coset offset is applied as the reference does (h * MC(class) * c subtracted from the target); the decoder adds c
// to each stage's entry bytewise, which is the same value whenever no A[f] + c leaves the int8 range; codebooks where
// it does are refused.
// The clamp delta (research/detail/r51_delta.py:14) is taken against the decoder's own f32 result: for every weight with
// |W_dec| > wmax = fp16(1.001 max|W|), d = clamp(W_dec, +-wmax) - W_dec in f32.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/p8x.h"
#include "p8x_codebook.h"
#include "p8x_format.h"
#include "p8x_internal.h"
#include "p8x_slotw.h"

using namespace p8x;
using namespace p8x::slotw;

namespace {

// class gains G and allocation distortions D of the shipped codebook (research/work/r48k3/tables_vrc.json)
constexpr double kGain[8] = {1.0, 24.599957646417835, 23.557000147255682, 23.557000147255682,
                             90.2330424977153, 172.81491504645197, 79.23598791183412, 255.21758494891367};
constexpr double kDist[8] = {1.0, 0.32507115602493286, 0.17149877548217773, 0.08859153091907501,
                             0.05250249058008194, 0.046983502805233, 0.00782012939453125, 0.0006935640121810138};
// index bits per weight of each class (NW / 4)
constexpr double kRate[8] = {0.0, 1.0, 1.5, 2.0, 2.5, 3.0, 4.0, 6.0};

int default_threads() {
    const unsigned h = std::thread::hardware_concurrency();
    return (int)std::max(1u, std::min(16u, h ? h : 1u));
}

// runs f(i) for i in [0, n) on nthr threads, items handed out one at a time
template <class F>
void parallel_for(int n, int nthr, F f) {
    nthr = std::max(1, std::min(nthr, n));
    if (nthr == 1) { for (int i = 0; i < n; ++i) f(i); return; }
    std::atomic<int> next{0};
    std::vector<std::thread> th;
    for (int t = 0; t < nthr; ++t)
        th.emplace_back([&] { for (int i; (i = next.fetch_add(1)) < n;) f(i); });
    for (auto &x : th) x.join();
}

int mc_of(int c) { return (1 << sh1_of(c)) + (w2_of(c) ? (1 << sh2_of(c)) : 0) + (w3_of(c) ? 1 : 0); }

// inverse of the upper-triangular 4x4 block U[j0..j0+3][j0..j0+3] (row stride ld): back substitution, fixed order
void tri_inv4(const double *U, size_t ld, double out[16]) {
    for (int i = 0; i < 16; ++i) out[i] = 0.0;
    for (int i = 0; i < 4; ++i) {
        out[4 * i + i] = 1.0 / U[i * ld + i];
        for (int j = i + 1; j < 4; ++j) {
            double s = 0.0;
            for (int k = i; k < j; ++k) s = s + out[4 * i + k] * U[k * ld + j];
            out[4 * i + j] = -s / U[j * ld + j];
        }
    }
}

// y (1x4) @ M (4x4, row-major), fixed order
inline void vecmat4(const double y[4], const double *M, double out[4]) {
    for (int e = 0; e < 4; ++e) out[e] = ((y[0] * M[e] + y[1] * M[4 + e]) + y[2] * M[8 + e]) + y[3] * M[12 + e];
}

inline double dist4(const double a[4], const double *t, double sc) {
    const double q0 = a[0] - sc * t[0], q1 = a[1] - sc * t[1], q2 = a[2] - sc * t[2], q3 = a[3] - sc * t[3];
    return ((q0 * q0 + q1 * q1) + q2 * q2) + q3 * q3;
}

// best codeword of one half for one target: cost, stage indices and codeword in int units (without coset offset)
struct Pick {
    double cost;
    uint8_t f[3];
    double cw[4];
};

struct TopK {   // the 4 smallest (d, index), ascending; equal d keep insertion order
    double d[4];
    int i[4];
    int n = 0;
    void push(double dd, int ii) {
        int p = n < 4 ? n : 4;
        if (p == 4 && !(dd < d[3])) return;
        while (p > 0 && dd < d[p - 1]) {
            if (p < 4) { d[p] = d[p - 1]; i[p] = i[p - 1]; }
            --p;
        }
        if (p < 4) { d[p] = dd; i[p] = ii; }
        if (n < 4) ++n;
    }
};

struct Codebook {
    double A[256][4];   // entries in int units
    double c[4];        // coset vector
};

// xa: the target in metric space; TA: the step's metric-space entries (A @ A4), scaled per stage by 2^shift.
void best_cw(const double xa[4], const double (*TA)[4], const Codebook &cb, int cls, int half, Pick &out) {
    const int W1 = w1_of(cls), W2 = w2_of(cls), W3 = w3_of(cls);
    const double s1 = (double)(1 << sh1_of(cls)), s2 = (double)(1 << sh2_of(cls));
    const int K1h = 1 << (W1 - 1), f0 = half * K1h;
    if (!W2) {
        double bc = 0.0; int bf = f0;
        for (int f = f0; f < f0 + K1h; ++f) {
            const double d = dist4(xa, TA[f], s1);
            if (f == f0 || d < bc) { bc = d; bf = f; }
        }
        out.cost = bc; out.f[0] = (uint8_t)bf; out.f[1] = out.f[2] = 0;
        for (int e = 0; e < 4; ++e) out.cw[e] = cb.A[bf][e] * s1;
        return;
    }
    TopK t1;
    for (int f = f0; f < f0 + K1h; ++f) t1.push(dist4(xa, TA[f], s1), f);
    const int K2 = 1 << W2;
    double best = 0.0; int b1 = -1, b2 = 0, b3 = 0;
    for (int a = 0; a < t1.n; ++a) {
        const int i1 = t1.i[a];
        double r1[4];
        for (int e = 0; e < 4; ++e) r1[e] = xa[e] - s1 * TA[i1][e];
        if (!W3) {
            double bc = 0.0; int bg = 0;
            for (int g = 0; g < K2; ++g) {
                const double d = dist4(r1, TA[g], s2);
                if (g == 0 || d < bc) { bc = d; bg = g; }
            }
            if (b1 < 0 || bc < best) { best = bc; b1 = i1; b2 = bg; }
        } else {
            TopK t2;
            for (int g = 0; g < K2; ++g) t2.push(dist4(r1, TA[g], s2), g);
            const int K3 = 1 << W3;
            for (int a2 = 0; a2 < t2.n; ++a2) {
                const int i2 = t2.i[a2];
                double r2[4];
                for (int e = 0; e < 4; ++e) r2[e] = r1[e] - s2 * TA[i2][e];
                double bc = 0.0; int bq = 0;
                for (int q = 0; q < K3; ++q) {
                    const double d = dist4(r2, TA[q], 1.0);
                    if (q == 0 || d < bc) { bc = d; bq = q; }
                }
                if (b1 < 0 || bc < best) { best = bc; b1 = i1; b2 = i2; b3 = bq; }
            }
        }
    }
    out.cost = best; out.f[0] = (uint8_t)b1; out.f[1] = (uint8_t)b2; out.f[2] = (uint8_t)b3;
    for (int e = 0; e < 4; ++e) {
        double v = cb.A[b1][e] * s1 + cb.A[b2][e] * s2;
        if (W3) v = v + cb.A[b3][e];
        out.cw[e] = v;
    }
}

// Per-slice metric tables: A4[t] (4x4) and TA[t][f] = A[f] @ A4[t] for the 32 steps of a 128-column slice.
struct SliceTabs {
    double A4[32][16];
    double TA[32][256][4];
};

void make_slice_tabs(const double *U, size_t K, int i0, const Codebook &cb, SliceTabs &st) {
    for (int t = 0; t < 32; ++t) {
        const size_t j = (size_t)i0 + 4 * t;
        if (U) tri_inv4(U + j * K + j, K, st.A4[t]);
        else for (int q = 0; q < 16; ++q) st.A4[t][q] = (q % 5 == 0) ? 1.0 : 0.0;
        for (int f = 0; f < 256; ++f) vecmat4(cb.A[f], st.A4[t], st.TA[t][f]);
    }
}

// One 128-column slice of one row. x: the row's current targets (128, real units), updated in place only through
// the survivor copies; S: the block scale; U: the full factor (nullptr = identity), i0: slice start.
// Outputs: idx (32 x 3), cwint (128 decoder ints), E (128 scaled errors).
struct SliceOut {
    uint8_t idx[32][3];
    int cwint[128];
    double E[128];
};

void zero_slice(const double *x, const double *U, size_t K, int i0, const SliceTabs &st, SliceOut &o) {
    double X[128];
    memcpy(X, x, sizeof X);
    memset(o.idx, 0, sizeof o.idx);
    for (int i = 0; i < 128; ++i) o.cwint[i] = 0;
    for (int t = 0; t < 32; ++t) {
        const int j = 4 * t;
        double e[4];
        vecmat4(X + j, st.A4[t], e);
        for (int q = 0; q < 4; ++q) o.E[j + q] = e[q];
        if (U && j + 4 < 128)
            for (int c = j + 4; c < 128; ++c) {
                const double *Ur = U + ((size_t)i0 + j) * K + i0 + c;
                X[c] = X[c] - (((e[0] * Ur[0] + e[1] * Ur[K]) + e[2] * Ur[2 * K]) + e[3] * Ur[3 * K]);
            }
    }
}

void vit_slice(const double *x, double S, int cls, const Codebook &cb, const double *U, size_t K, int i0,
               const SliceTabs &st, SliceOut &o) {
    constexpr int NS = 8;
    constexpr double INF = __builtin_huge_val();
    static thread_local double Xs[2][NS][128];
    double PM[NS];
    uint8_t SRC[32][NS], ID[32][NS][3];
    double XN[32][NS][4], CW[32][NS][4];
    const int mc = mc_of(cls);
    double off[2][4];
    for (int e = 0; e < 4; ++e) { off[0][e] = 0.0; off[1][e] = (double)mc * cb.c[e]; }
    int cur = 0;
    for (int s = 0; s < NS; ++s) { memcpy(Xs[cur][s], x, sizeof(double) * 128); PM[s] = s ? INF : 0.0; }
    for (int t = 0; t < 32; ++t) {
        const int j = 4 * t;
        const double *Am = st.A4[t];
        const double (*TA)[4] = st.TA[t];
        Pick pk[NS][2];
        bool live[NS];
        Pick cache[2][2];
        bool have[2] = {false, false};
        for (int s = 0; s < NS; ++s) {
            live[s] = PM[s] < INF;
            if (!live[s]) continue;
            const int h = (s >> 1) & 1;
            if (!U && have[h]) { pk[s][0] = cache[h][0]; pk[s][1] = cache[h][1]; continue; }
            double y[4], xa[4];
            for (int e = 0; e < 4; ++e) y[e] = Xs[cur][s][j + e] / S - off[h][e];
            vecmat4(y, Am, xa);
            for (int b = 0; b < 2; ++b) {
                best_cw(xa, TA, cb, cls, b, pk[s][b]);
                for (int e = 0; e < 4; ++e) pk[s][b].cw[e] = pk[s][b].cw[e] + off[h][e];
            }
            if (!U) { cache[h][0] = pk[s][0]; cache[h][1] = pk[s][1]; have[h] = true; }
        }
        double nPM[NS];
        const int nxt = cur ^ 1;
        for (int d = 0; d < NS; ++d) {
            // the two sources of d: s = d >> 1 and s | 4, with u = d & 1 = b ^ par(s & 5)
            int src = -1, bsel = 0;
            double best = INF;
            for (int hi = 0; hi < 2; ++hi) {
                const int s = (d >> 1) | (hi << 2);
                if (!live[s]) continue;
                const int b = (d & 1) ^ ((s ^ (s >> 2)) & 1);
                const double c = PM[s] + pk[s][b].cost;
                if (src < 0 || c < best) { best = c; src = s; bsel = b; }
            }
            nPM[d] = src < 0 ? INF : best;
            if (src < 0) continue;
            const Pick &p = pk[src][bsel];
            SRC[t][d] = (uint8_t)src;
            ID[t][d][0] = p.f[0]; ID[t][d][1] = p.f[1]; ID[t][d][2] = p.f[2];
            for (int e = 0; e < 4; ++e) { XN[t][d][e] = Xs[cur][src][j + e]; CW[t][d][e] = p.cw[e]; }
            if (t + 1 < 32) {
                double r[4], ev[4];
                for (int e = 0; e < 4; ++e) r[e] = Xs[cur][src][j + e] - p.cw[e] * S;
                vecmat4(r, Am, ev);
                double *dst = Xs[nxt][d];
                const double *sx = Xs[cur][src];
                if (U) {
                    const double *U0 = U + ((size_t)i0 + j) * K + i0;
                    for (int c = j + 4; c < 128; ++c)
                        dst[c] = sx[c] - (((ev[0] * U0[c] + ev[1] * U0[K + c]) + ev[2] * U0[2 * K + c]) + ev[3] * U0[3 * K + c]);
                } else {
                    for (int c = j + 4; c < 128; ++c) dst[c] = sx[c];
                }
            }
        }
        memcpy(PM, nPM, sizeof PM);
        cur = nxt;
    }
    int s = 0;
    for (int q = 1; q < NS; ++q) if (PM[q] < PM[s]) s = q;
    for (int t = 31; t >= 0; --t) {
        const int j = 4 * t;
        double r[4], ev[4];
        for (int e = 0; e < 4; ++e) {
            const double qv = CW[t][s][e] * S;
            r[e] = XN[t][s][e] - qv;
            o.cwint[j + e] = (int)CW[t][s][e];
        }
        vecmat4(r, st.A4[t], ev);
        for (int e = 0; e < 4; ++e) o.E[j + e] = ev[e];
        o.idx[t][0] = ID[t][s][0]; o.idx[t][1] = ID[t][s][1]; o.idx[t][2] = ID[t][s][2];
        s = SRC[t][s];
    }
}

// ---------------------------------------------------------------- dense factorization (rotated-domain factor U)
// In-place lower Cholesky factor of the n x n row-major SPD matrix A (lower triangle read and written).
bool chol_lower(double *A, int n, int nthr) {
    const int NB = 64;
    for (int k0 = 0; k0 < n; k0 += NB) {
        const int k1 = std::min(n, k0 + NB);
        for (int j = k0; j < k1; ++j) {   // diagonal block, left-looking within the block
            double d = A[(size_t)j * n + j];
            for (int m = k0; m < j; ++m) d -= A[(size_t)j * n + m] * A[(size_t)j * n + m];
            if (!(d > 0.0) || !std::isfinite(d)) return false;
            d = std::sqrt(d);
            A[(size_t)j * n + j] = d;
            for (int i = j + 1; i < k1; ++i) {
                double s = A[(size_t)i * n + j];
                for (int m = k0; m < j; ++m) s -= A[(size_t)i * n + m] * A[(size_t)j * n + m];
                A[(size_t)i * n + j] = s / d;
            }
        }
        const int rest = n - k1;
        if (rest <= 0) break;
        parallel_for(rest, nthr, [&](int ii) {   // panel rows: L21 = A21 L11^-T
            double *Ai = A + (size_t)(k1 + ii) * n;
            for (int j = k0; j < k1; ++j) {
                double s = Ai[j];
                const double *Aj = A + (size_t)j * n;
                for (int m = k0; m < j; ++m) s -= Ai[m] * Aj[m];
                Ai[j] = s / Aj[j];
            }
        });
        parallel_for(rest, nthr, [&](int ii) {   // trailing update A22 -= L21 L21^T (lower part)
            const int i = k1 + ii;
            double *Ai = A + (size_t)i * n;
            int j = k1;
            for (; j + 3 <= i; j += 4) {
                const double *B0 = A + (size_t)j * n, *B1 = B0 + n, *B2 = B1 + n, *B3 = B2 + n;
                double a0 = 0, a1 = 0, a2 = 0, a3 = 0;
                for (int m = k0; m < k1; ++m) {
                    const double v = Ai[m];
                    a0 += v * B0[m]; a1 += v * B1[m]; a2 += v * B2[m]; a3 += v * B3[m];
                }
                Ai[j] -= a0; Ai[j + 1] -= a1; Ai[j + 2] -= a2; Ai[j + 3] -= a3;
            }
            for (; j <= i; ++j) {
                const double *Bj = A + (size_t)j * n;
                double a = 0;
                for (int m = k0; m < k1; ++m) a += Ai[m] * Bj[m];
                Ai[j] -= a;
            }
        });
    }
    return true;
}

// Inverse of the lower-triangular L (row-major n x n) into Li (lower), columns in groups of 8.
void tri_inv_lower(const double *L, double *Li, int n, int nthr) {
    const int G = 8, ng = (n + G - 1) / G;
    parallel_for(ng, nthr, [&](int gi) {
        const int j0 = gi * G, j1 = std::min(n, j0 + G), w = j1 - j0;
        std::vector<double> X((size_t)n * G, 0.0);   // X[i][q] = Li[i][j0 + q]
        for (int i = j0; i < n; ++i) {
            const double *Lr = L + (size_t)i * n;
            double acc[G] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int m = j0; m < i; ++m) {
                const double v = Lr[m];
                const double *xm = &X[(size_t)m * G];
                for (int q = 0; q < G; ++q) acc[q] += v * xm[q];
            }
            for (int q = 0; q < w; ++q) {
                const int j = j0 + q;
                double v;
                if (i < j) v = 0.0;
                else if (i == j) v = 1.0 / Lr[i];
                else v = -acc[q] / Lr[i];
                X[(size_t)i * G + q] = v;
            }
        }
        for (int i = 0; i < n; ++i)
            for (int q = 0; q < w; ++q) Li[(size_t)i * n + j0 + q] = i >= j0 ? X[(size_t)i * G + q] : 0.0;
    });
}

int factor(const float *H, const uint16_t *c16, const int8_t *sg, int K, double damp, double *U, int nthr) {
    const int nb = K / 256;
    std::vector<double> cf(K);
    for (int k = 0; k < K; ++k) {
        cf[k] = c16 ? (double)half_to_float(c16[k]) : 1.0;
        if (!(cf[k] != 0.0) || !std::isfinite(cf[k])) return set_error(P8X_ERR_ARG, "p8x_encode: column scale %d is zero or not finite", k);
    }
    // T = (R Hc)^T computed row by row: row i of Hc rotated, stored as column i; then each row of T rotated again.
    std::vector<double> T((size_t)K * K);
    parallel_for(K, nthr, [&](int i) {
        double v[256];
        for (int b = 0; b < nb; ++b) {
            for (int q = 0; q < 256; ++q) {
                const int k = 256 * b + q;
                v[q] = (double)H[(size_t)i * K + k] / cf[i] / cf[k] * (double)sg[q];
            }
            fwht256_d(v);
            for (int q = 0; q < 256; ++q) T[(size_t)(256 * b + q) * K + i] = v[q];
        }
    });
    parallel_for(K, nthr, [&](int i) {
        double *row = &T[(size_t)i * K];
        for (int b = 0; b < nb; ++b) {
            for (int q = 0; q < 256; ++q) row[256 * b + q] *= (double)sg[q];
            fwht256_d(row + 256 * b);
        }
    });
    double md = 0.0;
    for (int i = 0; i < K; ++i) md += T[(size_t)i * K + i];
    md /= K;
    for (int i = 0; i < K; ++i) T[(size_t)i * K + i] += damp * md;
    // U = P inv(chol(P Hq P)) P (P = index reversal): U upper with U^T U = Hq^-1
    std::vector<double> Hr((size_t)K * K);
    parallel_for(K, nthr, [&](int i) {
        for (int j = 0; j <= i; ++j) Hr[(size_t)i * K + j] = T[(size_t)(K - 1 - i) * K + (K - 1 - j)];
    });
    std::vector<double>().swap(T);
    if (!chol_lower(Hr.data(), K, nthr)) return set_error(P8X_ERR_ARG, "p8x_encode: damped rotated H is not positive definite");
    std::vector<double> Li((size_t)K * K);
    tri_inv_lower(Hr.data(), Li.data(), K, nthr);
    parallel_for(K, nthr, [&](int i) {
        for (int j = 0; j < K; ++j) U[(size_t)i * K + j] = j >= i ? Li[(size_t)(K - 1 - i) * K + (K - 1 - j)] : 0.0;
    });
    return P8X_OK;
}

// ---------------------------------------------------------------- class allocation (research/detail/r48k.py:121-141)
void alloc(const double *E, int nt, double budget, const double *dist, const uint8_t *floor_, uint8_t *cls) {
    std::vector<double> Dm((size_t)nt * 8);
    double Rm[8];
    for (int k = 0; k < 8; ++k) Rm[k] = 256.0 * kRate[k];
    for (int i = 0; i < nt; ++i)
        for (int k = 0; k < 8; ++k)
            Dm[(size_t)i * 8 + k] = (floor_ && floor_[i] && k < 6) ? 1e300 : E[i] * dist[k];
    std::vector<uint8_t> c(nt);
    auto pick = [&](double lam) {
        double R = 0.0;
        for (int i = 0; i < nt; ++i) {
            int bk = 0; double bv = 0.0;
            for (int k = 0; k < 8; ++k) {
                const double v = Dm[(size_t)i * 8 + k] + lam * Rm[k];
                if (k == 0 || v < bv) { bv = v; bk = k; }
            }
            c[i] = (uint8_t)bk;
            R += Rm[bk];
        }
        return R;
    };
    double lo = 1e-12, hi = 1e6;
    for (int it = 0; it < 80; ++it) {
        const double mid = std::sqrt(lo * hi);
        if (pick(mid) > budget) lo = mid; else hi = mid;
    }
    double R = pick(hi);
    for (int it = 0; it < 400; ++it) {
        const double slack = budget - R;
        double best = 0.0; int ai = -1, ak = 0;
        for (int k = 1; k < 8; ++k) {
            double g = 0.0; int gi = 0; bool any = false;
            for (int i = 0; i < nt; ++i) {
                double gain = 0.0;
                const double dR = Rm[k] - Rm[c[i]];
                if (c[i] < k && dR <= slack && dR > 0) gain = (Dm[(size_t)i * 8 + c[i]] - Dm[(size_t)i * 8 + k]) / dR;
                if (!any || gain > g) { g = gain; gi = i; any = true; }
            }
            if (g > best) { best = g; ai = gi; ak = k; }
        }
        if (ai < 0) break;
        R += Rm[ak] - Rm[c[ai]];
        c[ai] = (uint8_t)ak;
    }
    memcpy(cls, c.data(), (size_t)nt);
}

// double -> fp16 bits, round to nearest even (the f32 candidate and its neighbours, compared in double)
uint16_t double_to_half(double x) {
    const uint16_t h = float_to_half((float)x);
    if ((h & 0x7c00u) == 0x7c00u) return h;
    uint16_t best = h;
    double bd = std::fabs((double)half_to_float(h) - x);
    for (int d = -1; d <= 1; d += 2) {
        const uint16_t m = h & 0x7fffu;
        if ((d < 0 && m == 0) || (d > 0 && m >= 0x7bffu)) continue;
        const uint16_t c = (uint16_t)((h & 0x8000u) | (uint16_t)(m + d));
        const double cd = std::fabs((double)half_to_float(c) - x);
        if (cd < bd || (cd == bd && !(c & 1u))) { bd = cd; best = c; }
    }
    return best;
}

void put_bits(uint32_t *lw, int wb, int W, int k, uint32_t v) {
    const int pos = W * k, wi = wb + (pos >> 5), bb = pos & 31;
    const uint64_t x = (uint64_t)(v & ((1u << W) - 1u)) << bb;
    lw[wi] |= (uint32_t)x;
    if (bb + W > 32) lw[wi + 1] |= (uint32_t)(x >> 32);
}

}  // namespace

extern "C" {

void p8x_encode_defaults(p8x_encode_params *p) {
    if (!p) return;
    memset(p, 0, sizeof *p);
    p->damp = 0.1;
    p->bits_per_weight = 2.0;
    p->n_salient = 4;
    p->alpha = 1.05;
}

void p8x_encode_free(void *slot) { free(slot); }

int p8x_encode_factor(const float *H, const uint16_t *c16, const int8_t *signs, uint64_t sign_seed, int K, double damp,
                      int threads, double *U) {
    if (!H || !U || K <= 0 || K % 256 || !(damp >= 0.0))
        return set_error(P8X_ERR_ARG, "p8x_encode_factor: need H, U, K %% 256 == 0 (K %d), damp >= 0", K);
    std::vector<int8_t> sg = signs ? std::vector<int8_t>(signs, signs + 256) : seeded_signs(sign_seed);
    for (int i = 0; i < 256; ++i) if (sg[i] != 1 && sg[i] != -1) return set_error(P8X_ERR_ARG, "p8x_encode_factor: sign %d is not +-1", i);
    return factor(H, c16, sg.data(), K, damp, U, threads > 0 ? threads : default_threads());
}

int p8x_encode_alloc(const double *E, int n_tiles, double budget_bits, const double *dist, const uint8_t *floor_,
                     uint8_t *classes) {
    if (!E || !classes || n_tiles <= 0 || !(budget_bits >= 0.0)) return set_error(P8X_ERR_ARG, "p8x_encode_alloc: bad arguments");
    alloc(E, n_tiles, budget_bits / 32.0, dist ? dist : kDist, floor_, classes);
    return P8X_OK;
}

int p8x_encode_tensor(const float *W, int rows, int K, const p8x_encode_params *pp, void **out, size_t *n_out) {
    if (!W || !out || !n_out || rows <= 0 || K <= 0 || rows % 32 || K % 256 || rows >= 32768 || K > 65536)
        return set_error(P8X_ERR_ARG, "p8x_encode: shape %d x %d (need rows %% 32 == 0, rows < 32768, K %% 256 == 0, K <= 65536)", rows, K);
    *out = nullptr; *n_out = 0;
    p8x_encode_params p;
    if (pp) p = *pp; else p8x_encode_defaults(&p);
    if (!(p.alpha > 0.0) || !(p.damp >= 0.0) || p.n_salient < 0) return set_error(P8X_ERR_ARG, "p8x_encode: need alpha > 0, damp >= 0, n_salient >= 0");
    const int nthr = p.threads > 0 ? p.threads : default_threads();
    const int ng = rows / 32, nb = K / 256, nsl = K / 128;
    const size_t nt = (size_t)ng * nb;
    const double *gain = p.gain ? p.gain : kGain;
    const double *dist = p.dist ? p.dist : kDist;
    for (int k = 1; k < 8; ++k) if (!(gain[k] > 0.0) || !std::isfinite(gain[k])) return set_error(P8X_ERR_ARG, "p8x_encode: gain of class %d", k);

    // codebook (the encoder applies the coset offset unwrapped: refuse codebooks where A + c wraps)
    const uint32_t *Aw = p.A ? p.A : kShippedA;
    const uint32_t cs = p.A ? p.cs : kShippedC;
    Codebook cb;
    for (int e = 0; e < 4; ++e) cb.c[e] = (double)(int8_t)(cs >> (8 * e));
    for (int f = 0; f < 256; ++f)
        for (int e = 0; e < 4; ++e) {
            const int a = (int8_t)(Aw[f] >> (8 * e));
            cb.A[f][e] = (double)a;
            if (a + (int)cb.c[e] > 127 || a + (int)cb.c[e] < -128)
                return set_error(P8X_ERR_UNSUPPORTED, "p8x_encode: codebook entry %d + coset leaves int8", f);
        }

    Side sd;
    sd.c16.resize(K);
    std::vector<double> cf(K);
    for (int k = 0; k < K; ++k) {
        sd.c16[k] = p.c16 ? p.c16[k] : (uint16_t)0x3C00;
        cf[k] = (double)half_to_float(sd.c16[k]);
        if (!(cf[k] != 0.0) || !std::isfinite(cf[k])) return set_error(P8X_ERR_ARG, "p8x_encode: column scale %d is zero or not finite", k);
    }
    sd.sg = p.signs ? std::vector<int8_t>(p.signs, p.signs + 256) : seeded_signs(p.sign_seed);
    for (int i = 0; i < 256; ++i) if (sd.sg[i] != 1 && sd.sg[i] != -1) return set_error(P8X_ERR_ARG, "p8x_encode: sign %d is not +-1", i);

    // input second moment -> rotated-domain factor
    std::vector<double> Uown;
    const double *U = p.U;
    if (!U && p.H) {
        Uown.resize((size_t)K * K);
        const int rc = factor(p.H, sd.c16.data(), sd.sg.data(), K, p.damp, Uown.data(), nthr);
        if (rc != P8X_OK) return rc;
        U = Uown.data();
    }
    if (U) for (int i = 0; i < K; ++i) if (!(U[(size_t)i * K + i] > 0.0)) return set_error(P8X_ERR_ARG, "p8x_encode: U[%d][%d] is not positive", i, i);

    // rotated targets and block energies
    std::vector<double> Y((size_t)rows * K), Ebk((size_t)rows * nb);
    float amax = 0.f;
    for (size_t i = 0; i < (size_t)rows * K; ++i) {
        if (!std::isfinite(W[i])) return set_error(P8X_ERR_ARG, "p8x_encode: W[%zu] is not finite", i);
        amax = std::max(amax, std::fabs(W[i]));
    }
    parallel_for(rows, nthr, [&](int r) {
        for (int b = 0; b < nb; ++b) {
            double *v = &Y[(size_t)r * K + 256 * b];
            for (int i = 0; i < 256; ++i) {
                const int k = 256 * b + i;
                v[i] = (double)W[(size_t)r * K + k] * cf[k] * (double)sd.sg[i];
            }
            fwht256_d(v);
            double ss = 0.0;
            for (int i = 0; i < 256; ++i) ss += v[i] * v[i];
            Ebk[(size_t)r * nb + b] = ss;
        }
    });

    // row order
    sd.prm.resize(rows);
    if (p.prm) {
        std::vector<char> seen(rows, 0);
        for (int r = 0; r < rows; ++r) {
            const int v = p.prm[r];
            if (v < 0 || v >= rows || seen[v]) return set_error(P8X_ERR_ARG, "p8x_encode: prm is not a permutation (entry %d)", r);
            seen[v] = 1; sd.prm[r] = (int16_t)v;
        }
    } else {
        std::vector<double> key(rows);
        for (int r = 0; r < rows; ++r) {
            double s = 0.0;
            for (int b = 0; b < nb; ++b) s += std::log(std::max(Ebk[(size_t)r * nb + b], 1e-30));
            key[r] = s / nb;
        }
        std::vector<int> ord(rows);
        for (int r = 0; r < rows; ++r) ord[r] = r;
        std::stable_sort(ord.begin(), ord.end(), [&](int a, int b) { return key[a] < key[b]; });
        for (int r = 0; r < rows; ++r) sd.prm[r] = (int16_t)ord[r];
    }
    std::vector<int> pinv(rows);
    for (int r = 0; r < rows; ++r) pinv[sd.prm[r]] = r;

    // classes per tile (sorted-row order)
    std::vector<uint8_t> cls(nt);
    if (p.classes) {
        for (size_t i = 0; i < nt; ++i) {
            if (p.classes[i] > 7) return set_error(P8X_ERR_ARG, "p8x_encode: class %d of tile %zu", p.classes[i], i);
            cls[i] = p.classes[i];
        }
    } else {
        if (!(p.bits_per_weight >= 0.0)) return set_error(P8X_ERR_ARG, "p8x_encode: bits_per_weight < 0");
        std::vector<double> wb(nb, 1.0);
        if (U) {
            double tot = 0.0;
            for (int b = 0; b < nb; ++b) {
                double s = 0.0;
                for (int i = 0; i < 256; ++i) {
                    const double u = U[(size_t)(256 * b + i) * K + 256 * b + i];
                    s += 1.0 / (u * u);
                }
                wb[b] = s / 256.0;
                tot += wb[b];
            }
            const double mean = tot / nb;
            for (int b = 0; b < nb; ++b) wb[b] = wb[b] / mean;
        }
        std::vector<double> Et(nt, 0.0);
        for (int g = 0; g < ng; ++g)
            for (int b = 0; b < nb; ++b) {
                double s = 0.0;
                for (int j = 0; j < 32; ++j) s += Ebk[(size_t)sd.prm[32 * g + j] * nb + b] * wb[b];
                Et[(size_t)g * nb + b] = s;
            }
        std::vector<uint8_t> fl;
        if (p.n_salient > 0) {
            fl.assign(nt, 0);
            const size_t n = (size_t)rows * K, m = std::min<size_t>((size_t)p.n_salient, n);
            std::vector<size_t> ord(n);
            for (size_t i = 0; i < n; ++i) ord[i] = i;
            std::partial_sort(ord.begin(), ord.begin() + m, ord.end(), [&](size_t a, size_t b) {
                const float x = std::fabs(W[a]), y = std::fabs(W[b]);
                return x > y || (x == y && a < b);
            });
            for (size_t q = 0; q < m; ++q) {
                const size_t r = ord[q] / K, col = ord[q] % K;
                fl[(size_t)(pinv[r] / 32) * nb + col / 256] = 1;
            }
        }
        alloc(Et.data(), (int)nt, p.bits_per_weight * rows * K / 32.0, dist, fl.empty() ? nullptr : fl.data(), cls.data());
    }
    size_t words = 0;
    std::vector<uint32_t> M(nt);
    for (size_t i = 0; i < nt; ++i) {
        M[i] = (uint32_t)words | ((uint32_t)cls[i] << 29);
        words += (size_t)64 * nw_of(cls[i]);
    }
    if (words >= (1u << 29)) return set_error(P8X_ERR_UNSUPPORTED, "p8x_encode: payload of %zu words exceeds the 29-bit tile offset", words);

    // block scales S[b][sorted row]
    std::vector<uint16_t> S((size_t)nb * rows);
    for (int r = 0; r < rows; ++r)
        for (int b = 0; b < nb; ++b) {
            const int c = cls[(size_t)(pinv[r] / 32) * nb + b];
            const double rms = std::max(std::sqrt(Ebk[(size_t)r * nb + b] / 256.0), 1e-12);
            S[(size_t)b * rows + pinv[r]] = c ? float_to_half((float)(p.alpha * rms / gain[c])) : (uint16_t)0;
        }

    // per-slice metric tables
    std::vector<SliceTabs> tabs(nsl);
    parallel_for(nsl, nthr, [&](int s) { make_slice_tabs(U, (size_t)K, 128 * s, cb, tabs[s]); });

    // rows
    const float wmax = half_to_float(double_to_half((double)amax * 1.001));
    std::vector<float> icf(K);
    for (int k = 0; k < K; ++k) icf[k] = (float)sd.sg[k & 255] / half_to_float(sd.c16[k]);
    std::vector<uint8_t> idx((size_t)rows * (K / 4) * 3);
    std::vector<std::vector<uint16_t>> dcol(rows);
    std::vector<std::vector<float>> dval(rows);
    constexpr int RB = 8;   // rows per task: one pass over U's rows serves the feedback of all of them
    parallel_for((rows + RB - 1) / RB, nthr, [&](int blk) {
        const int r0 = blk * RB, nr = std::min(RB, rows - r0);
        std::vector<double> w(Y.begin() + (size_t)r0 * K, Y.begin() + (size_t)(r0 + nr) * K);
        std::vector<int> ival((size_t)nr * K);
        std::vector<double> acc(U ? (size_t)nr * K : 0);
        std::vector<SliceOut> so(nr);
        for (int s = 0; s < nsl; ++s) {
            const int i0 = 128 * s, b = s / 2, i1 = i0 + 128;
            for (int q = 0; q < nr; ++q) {
                const int r = r0 + q, sr = pinv[r];
                const int c = cls[(size_t)(sr / 32) * nb + b];
                const double Sd = (double)half_to_float(S[(size_t)b * rows + sr]);
                double *wr = &w[(size_t)q * K];
                if (c == 0 || Sd == 0.0) zero_slice(wr + i0, U, (size_t)K, i0, tabs[s], so[q]);
                else vit_slice(wr + i0, Sd, c, cb, U, (size_t)K, i0, tabs[s], so[q]);
                memcpy(&idx[((size_t)r * (K / 4) + i0 / 4) * 3], so[q].idx, sizeof so[q].idx);
                for (int i = 0; i < 128; ++i) ival[(size_t)q * K + i0 + i] = so[q].cwint[i];
            }
            if (U && i1 < K) {   // W[:, i1:] -= E @ U[i0:i1, i1:], each sum taken over i in ascending order
                std::fill(acc.begin(), acc.end(), 0.0);
                for (int i = 0; i < 128; ++i) {
                    const double *Ur = U + (size_t)(i0 + i) * K;
                    for (int q = 0; q < nr; ++q) {
                        const double e = so[q].E[i];
                        double *a = &acc[(size_t)q * K];
                        for (int col = i1; col < K; ++col) a[col] = a[col] + e * Ur[col];
                    }
                }
                for (int q = 0; q < nr; ++q)
                    for (int col = i1; col < K; ++col) w[(size_t)q * K + col] = w[(size_t)q * K + col] - acc[(size_t)q * K + col];
            }
        }
        // the decoder's f32 result for these rows (CPU.patch:1012-1027 order) and their clamp deltas
        float v[256];
        for (int q = 0; q < nr; ++q) {
            const int r = r0 + q, sr = pinv[r];
            for (int b = 0; b < nb; ++b) {
                const float sc = half_to_float(S[(size_t)b * rows + sr]);
                for (int i = 0; i < 256; ++i) v[i] = (float)ival[(size_t)q * K + 256 * b + i] * sc;
                fwht256_f(v);
                for (int i = 0; i < 256; ++i) {
                    const float x = v[i] * icf[256 * b + i];
                    if (std::fabs(x) > wmax) {
                        const float cl = x > 0 ? wmax : -wmax;
                        dcol[r].push_back((uint16_t)(256 * b + i));
                        dval[r].push_back(cl - x);
                    }
                }
            }
        }
    });
    for (int r = 0; r < rows; ++r)
        for (size_t q = 0; q < dcol[r].size(); ++q) {
            sd.drow.push_back((uint16_t)r); sd.dcol.push_back(dcol[r][q]); sd.dval.push_back(dval[r][q]);
        }
    if (sd.drow.size() > 65535) return set_error(P8X_ERR_UNSUPPORTED, "p8x_encode: %zu clamp deltas (at most 65535)", sd.drow.size());

    const size_t need = need_bytes(offset_D(nt) + 4 * words, (size_t)rows, (size_t)K, sd.drow.size());
    uint8_t *buf = (uint8_t *)malloc(need);
    if (!buf) return set_error(P8X_ERR_NOMEM, "p8x_encode: out of host memory (%zu bytes)", need);
    uint32_t *D = reinterpret_cast<uint32_t *>(buf + offset_D(nt));
    parallel_for(ng, nthr, [&](int g) {
        for (int b = 0; b < nb; ++b) {
            const int c = cls[(size_t)g * nb + b];
            const int nw = nw_of(c);
            if (!nw) continue;
            const int W1 = w1_of(c), W2 = w2_of(c), W3 = w3_of(c);
            uint32_t *tile = D + (M[(size_t)g * nb + b] & 0x1FFFFFFFu);
            for (int hs = 0; hs < 2; ++hs)
                for (int j = 0; j < 32; ++j) {
                    const int r = sd.prm[32 * g + j];
                    const uint8_t *ch = &idx[((size_t)r * (K / 4) + (256 * b + 128 * hs) / 4) * 3];
                    uint32_t lw[24] = {0};
                    for (int k = 0; k < 32; ++k) {
                        const uint8_t *f = ch + 3 * ((j + k) & 31);
                        if (W1 == 8) put_bits(lw, 0, 8, k, f[0]);
                        else {
                            lw[0] |= (uint32_t)((f[0] >> (W1 - 1)) & 1u) << k;
                            put_bits(lw, 1, W1 - 1, k, f[0]);
                        }
                        if (W2) put_bits(lw, W1, W2, k, f[1]);
                        if (W3) put_bits(lw, W1 + W2, W3, k, f[2]);
                    }
                    for (int i = 0; i < nw; ++i) tile[(size_t)hs * nw * 32 + file_word(i, j)] = lw[i];
                }
        }
    });
    uint32_t Ahdr[256];
    memcpy(Ahdr, Aw, sizeof Ahdr);
    write_slot(buf, rows, K, Ahdr, cs, M, S, words, sd);
    *out = buf;
    *n_out = need;
    return P8X_OK;
}

// the class-3, identity-metric special case with rows in their original order
int p8x_quantize_tensor(const float *W, int rows, int K, const uint16_t *c16, uint64_t sign_seed, void *out, size_t cap,
                        size_t *n_out) {
    if (!W || rows <= 0 || K <= 0 || rows % 32 || K % 256 || rows >= 32768 || !n_out)
        return set_error(P8X_ERR_ARG, "p8x_quantize_tensor: shape %d x %d", rows, K);
    p8x_encode_params p;
    p8x_encode_defaults(&p);
    p.c16 = c16;
    p.sign_seed = sign_seed;
    std::vector<uint8_t> cls((size_t)(rows / 32) * (K / 256), 3);
    p.classes = cls.data();
    std::vector<int16_t> prm(rows);
    for (int r = 0; r < rows; ++r) prm[r] = (int16_t)r;
    p.prm = prm.data();
    void *slot = nullptr;
    size_t n = 0;
    const int rc = p8x_encode_tensor(W, rows, K, &p, &slot, &n);
    if (rc != P8X_OK) return rc;
    *n_out = n;
    if (!out || cap < n) { free(slot); return set_error(P8X_ERR_ARG, "p8x_quantize_tensor: output needs %zu bytes", n); }
    memcpy(out, slot, n);
    free(slot);
    return P8X_OK;
}

}  // extern "C"
