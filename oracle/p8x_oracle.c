/*
 * p8x_oracle.c -- scalar CPU restatement of the Pingala-8 hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see p8x_oracle.h). Written from the format description and the
 * reference CPU core; every function cites the lines of patches/llama_cpu_vs_7ac59a6.patch
 * ("CPU.patch") whose behaviour it restates. Float operations are done one at a time in the
 * reference's order so that f32 results are bit-identical; build with -ffp-contract=off.
 */
#include "p8x_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- class tables (CPU.patch:188-195) */
int orc_w1(int c) { return c == 0 ? 0 : c == 1 ? 4 : c == 2 ? 6 : 8; }
int orc_w2(int c) { return c == 4 ? 2 : c == 5 ? 4 : c >= 6 ? 8 : 0; }
int orc_w3(int c) { return c == 7 ? 8 : 0; }
int orc_sh1(int c) { static const int t[8] = {0, 0, 0, 0, 2, 3, 2, 4}; return t[c & 7]; }
int orc_sh2(int c) { return c == 7 ? 2 : 0; }
int orc_nw(int c) { return orc_w1(c) + orc_w2(c) + orc_w3(c); }
int orc_nstage(int c) { return c == 0 ? 0 : c <= 3 ? 1 : c <= 6 ? 2 : 3; }
int orc_mc(int c) { return (1 << orc_sh1(c)) + (orc_w2(c) ? (1 << orc_sh2(c)) : 0) + (orc_w3(c) ? 1 : 0); }

/* ---------------------------------------------------------------- IEEE half <-> float (CPU.patch:197-219) */
float orc_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31, ex = (h >> 10) & 31u, man = h & 1023u, bits;
    float f;
    if (ex == 0) {                       /* zero / subnormal: man * 2^-24, exact in f32 */
        f = (float)man * (1.0f / 16777216.0f);
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (ex == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f2h(float f) {              /* round to nearest even */
    uint32_t u; memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u, fe = (u >> 23) & 255u, man = u & 0x7fffffu;
    int e = (int)fe - 112;               /* half exponent */
    if (fe == 255) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        int sh = 14 - e;
        uint32_t q = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = man >> 13, rem = man & 0x1fffu, he = (uint32_t)e;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) {
        q++;
        if (q == 0x400u) { q = 0; he++; if (he >= 31) return (uint16_t)(sign | 0x7c00u); }
    }
    return (uint16_t)(sign | (he << 10) | q);
}

/* ---------------------------------------------------------------- layout (CPU.patch:25-51) */
static size_t a16(size_t v) { return (v + 15) & ~(size_t)15; }

size_t orc_need(size_t kbytes, size_t rows, size_t K, size_t nd) {
    return a16(kbytes) + a16(8 * nd) + a16(2 * K) + 2 * a16(2 * rows) + 256 + 32 + 64;
}

void orc_offsets(size_t n, size_t rows, size_t K, size_t nd, size_t off[6]) {
    size_t t = n - 32, sg = t - 256;
    size_t q = (sg - 2 * rows) & ~(size_t)15;
    size_t p = (q - 2 * rows) & ~(size_t)15;
    size_t c = (p - 2 * K) & ~(size_t)15;
    size_t e = (c - 8 * nd) & ~(size_t)15;
    off[0] = e; off[1] = c; off[2] = p; off[3] = q; off[4] = sg; off[5] = t;
}

/* ---------------------------------------------------------------- open (CPU.patch:234-275, :4335-4352) */
int orc_open(orc_tensor *t, const uint8_t *base, size_t n, int rows, int K) {
    memset(t, 0, sizeof(*t));
    /* fixed regions: header 2064, Hadamard signs 256, trailer 32 (vrn_offsets, CPU.patch:37-44) */
    if (n < 2064 + 256 + 32 || rows <= 0 || K <= 0 || K % 256 || rows % 32 || rows >= 32768) return 1;
    uint32_t tr[8];
    memcpy(tr, base + n - 32, 32);
    if (tr[0] != 0x4E525656u || tr[1] != 0x31354952u || tr[4] != (uint32_t)rows || tr[5] != (uint32_t)K || tr[6] != 108u) return 1;
    t->base = base; t->n = n; t->rows = rows; t->K = K;
    t->nb = K / 256; t->ng = rows / 32; t->nsl = K / 128; t->nd = (int)tr[3];
    t->nt = (size_t)t->ng * t->nb; t->kbytes = tr[2];
    t->A = (const uint32_t *)base;
    t->cs = t->A[512];
    if (t->A[513] != 108u || t->A[514] != 2u) return 2;
    t->M = (const uint32_t *)(base + 2064);
    t->S = (const uint16_t *)(base + 2064 + 4 * t->nt);
    t->D = (const uint32_t *)(base + a16(2064 + 68 * t->nt));
    size_t off[6];
    orc_offsets(n, (size_t)rows, (size_t)K, (size_t)t->nd, off);
    if (off[0] > n || t->kbytes > off[0]) return 3;   /* off[0] > n: the top-down regions wrapped below 0 */
    size_t words = 0;
    for (size_t i = 0; i < t->nt; ++i) words += (size_t)64 * orc_nw((int)(t->M[i] >> 29));
    if (a16(2064 + 68 * t->nt) + 4 * words != t->kbytes) return 4;
    t->c16 = (const uint16_t *)(base + off[1]);
    t->prm = (const int16_t *)(base + off[2]);
    t->pinv = (const int16_t *)(base + off[3]);
    t->sg = (const int8_t *)(base + off[4]);
    t->drow = (const uint16_t *)(base + off[0]);
    t->dcol = t->drow + t->nd;
    t->dval = (const float *)(base + off[0] + 4 * (size_t)t->nd);
    t->ic = (float *)malloc(sizeof(float) * (size_t)K);
    for (int i = 0; i < K; ++i) t->ic[i] = (float)t->sg[i & 255] / orc_h2f(t->c16[i]);
    t->cp = (int *)calloc((size_t)rows + 1, sizeof(int));
    t->cc = (uint16_t *)malloc(2 * (size_t)t->nd + 2);
    t->cv = (float *)malloc(4 * (size_t)t->nd + 4);
    for (int e = 0; e < t->nd; ++e) t->cp[t->drow[e] + 1]++;
    for (int r = 0; r < rows; ++r) t->cp[r + 1] += t->cp[r];
    int *fill = (int *)malloc(sizeof(int) * (size_t)rows);
    memcpy(fill, t->cp, sizeof(int) * (size_t)rows);
    for (int e = 0; e < t->nd; ++e) {          /* entry order kept within a row (CPU.patch:263-270) */
        int q = fill[t->drow[e]]++;
        t->cc[q] = t->dcol[e];
        t->cv[q] = t->dval[e];
    }
    free(fill);
    return 0;
}

void orc_close(orc_tensor *t) {
    free(t->ic); free(t->cp); free(t->cc); free(t->cv);
    t->ic = NULL; t->cp = NULL; t->cc = NULL; t->cv = NULL;
}

/* ---------------------------------------------------------------- trellis (CPU.patch:159-160, :277-283) */
/* Multiplication by (1 + x + x^3)^-1 mod x^32 over GF(2) via repeated squaring of the multiplier:
 * u_t = z_t ^ u_{t-1} ^ u_{t-3} in closed form; the coset bit is h_t = u_{t-2}, i.e. u << 2. */
uint32_t orc_trellis_word(uint32_t z) {
    uint32_t u = z;
    u ^= (u << 1) ^ (u << 3);
    u ^= (u << 2) ^ (u << 6);
    u ^= (u << 4) ^ (u << 12);
    u ^= (u << 8) ^ (u << 24);
    u ^= u << 16;
    return u << 2;
}

/* the same map run one step at a time (the 8-state shift register of research/detail/r51_transcode.py:103-107) */
uint32_t orc_trellis_serial(uint32_t z) {
    uint32_t h = 0, st = 0;                     /* st bit i = u_{t-1-i} */
    for (int t = 0; t < 32; ++t) {
        uint32_t ht = (st >> 1) & 1u;           /* u_{t-2} */
        uint32_t ut = ((z >> t) & 1u) ^ (st & 1u) ^ ((st >> 2) & 1u);
        h |= ht << t;
        st = ((st << 1) | ut) & 7u;
    }
    return h;
}

static uint32_t rotl32(uint32_t x, int r) { r &= 31; return r ? (x << r) | (x >> (32 - r)) : x; }
static uint32_t rotr32(uint32_t x, int r) { r &= 31; return r ? (x >> r) | (x << (32 - r)) : x; }

/* ---------------------------------------------------------------- lane decode (CPU.patch:285-315, :992-1010) */
/* words of lane j, half hs of a tile payload p0 (CPU.patch:292-297); zero padded to 32 words */
static void lane_words(const uint32_t *p0, int c, int hs, int j, uint32_t w[32]) {
    int nw = orc_nw(c);
    const uint32_t *p = p0 + (size_t)hs * nw * 32 + 2 * j;
    for (int i = 0; i < 32; ++i) w[i] = 0;
    for (int i = 0; i < nw; ++i) w[i] = p[(i >> 1) * 64 + (i & 1)];
}

/* width-W field k of a little-endian bit string starting at word wb (CPU.patch:285-289) */
static uint32_t field(const uint32_t *w, int wb, int W, int k) {
    int pos = W * k, wi = wb + (pos >> 5), bb = pos & 31;
    uint64_t v = (uint64_t)w[wi] | ((uint64_t)w[wi + 1] << 32);
    return (uint32_t)(v >> bb) & ((1u << W) - 1u);
}

/* stage-1 index of step k (CPU.patch:309) */
static uint32_t stage1(const uint32_t *w, int c, int k) {
    int W1 = orc_w1(c);
    if (W1 == 8) return field(w, 0, 8, k);
    return field(w, 1, W1 - 1, k) | (((w[0] >> k) & 1u) << (W1 - 1));
}

/* coset bits in STEP order for lane j (CPU.patch:299-304) */
static uint32_t lane_coset_steps(const uint32_t *w, int c, int j) {
    uint32_t pm = 0;                             /* bit k = stage-1 label of step k */
    for (int k = 0; k < 32; ++k) pm |= ((stage1(w, c, k) >> (orc_w1(c) - 1)) & 1u) << k;
    return rotr32(orc_trellis_word(rotl32(pm, j)), j);
}

/* bytewise add of two int8x4 words without carries between bytes (CPU.patch:221) */
static uint32_t add_bytes(uint32_t a, uint32_t b) {
    uint32_t r = 0;
    for (int e = 0; e < 4; ++e) r |= (uint32_t)(uint8_t)((a >> (8 * e)) + (b >> (8 * e))) << (8 * e);
    return r;
}

void orc_decode_tile(const orc_tensor *t, int g, int b, int16_t *out) {
    uint32_t mt = t->M[(size_t)g * t->nb + b];
    int c = (int)(mt >> 29);
    if (c == 0) { memset(out, 0, 32 * 256 * sizeof(int16_t)); return; }
    const uint32_t *p0 = t->D + (mt & 0x1FFFFFFFu);
    int W1 = orc_w1(c), W2 = orc_w2(c), W3 = orc_w3(c), s1 = orc_sh1(c), s2 = orc_sh2(c);
    uint32_t w[32];
    for (int hs = 0; hs < 2; ++hs) {
        for (int j = 0; j < 32; ++j) {
            lane_words(p0, c, hs, j, w);
            uint32_t hk = lane_coset_steps(w, c, j);
            for (int k = 0; k < 32; ++k) {
                uint32_t cm = ((hk >> k) & 1u) ? t->cs : 0u;
                uint32_t a1 = add_bytes(t->A[stage1(w, c, k)], cm);
                uint32_t a2 = W2 ? add_bytes(t->A[field(w, W1, W2, k)], cm) : 0u;
                uint32_t a3 = W3 ? add_bytes(t->A[field(w, W1 + W2, W3, k)], cm) : 0u;
                int col = hs * 128 + 4 * ((j + k) & 31);
                for (int e = 0; e < 4; ++e) {
                    int v = (int)(int8_t)(a1 >> (8 * e)) * (1 << s1);
                    if (W2) v += (int)(int8_t)(a2 >> (8 * e)) * (1 << s2);
                    if (W3) v += (int)(int8_t)(a3 >> (8 * e));
                    out[j * 256 + col + e] = (int16_t)v;
                }
            }
        }
    }
}

void orc_decode_all(const orc_tensor *t, int16_t *out) {
    int16_t tile[32 * 256];
    for (int g = 0; g < t->ng; ++g)
        for (int b = 0; b < t->nb; ++b) {
            orc_decode_tile(t, g, b, tile);
            for (int j = 0; j < 32; ++j)
                memcpy(out + (size_t)(32 * g + j) * t->K + 256 * b, tile + j * 256, 256 * sizeof(int16_t));
        }
}

/* ---------------------------------------------------------------- bit-by-bit per-weight decode (CPU.patch:4020-4066) */
static uint32_t lane_bits(const uint32_t *p, int j, int wb, int pos, int W) {
    uint32_t v = 0;
    for (int q = 0; q < W; ++q) {
        int ps = pos + q, wi = wb + ps / 32;
        v |= ((p[(wi >> 1) * 64 + 2 * j + (wi & 1)] >> (ps % 32)) & 1u) << q;
    }
    return v;
}

static uint32_t lane_stage1_chunk(const uint32_t *p, int j, int c, int tchunk) {
    int W1 = orc_w1(c), k = (tchunk - j) & 31;
    if (W1 < 8) return lane_bits(p, j, 1, (W1 - 1) * k, W1 - 1) | (lane_bits(p, j, 0, k, 1) << (W1 - 1));
    return lane_bits(p, j, 0, 8 * k, 8);
}

int orc_weight_int(const orc_tensor *t, int r, int col) {
    int g = r >> 5, j = r & 31, b = col >> 8, hs = (col >> 7) & 1, tc = (col & 127) >> 2, e = col & 3;
    uint32_t mt = t->M[(size_t)g * t->nb + b];
    int c = (int)(mt >> 29);
    if (!c) return 0;
    int W1 = orc_w1(c), W2 = orc_w2(c), W3 = orc_w3(c), k = (tc - j) & 31;
    const uint32_t *p = t->D + (mt & 0x1FFFFFFFu) + (size_t)hs * orc_nw(c) * 32;
    uint32_t f1 = lane_stage1_chunk(p, j, c, tc);
    uint32_t f2 = W2 ? lane_bits(p, j, W1, W2 * k, W2) : 0, f3 = W3 ? lane_bits(p, j, W1 + W2, W3 * k, W3) : 0;
    int u[32], h = 0;
    for (int q = 0; q < tc; ++q) {              /* recursive shift register, reset per half-slice */
        int z = (int)((lane_stage1_chunk(p, j, c, q) >> (W1 - 1)) & 1u);
        u[q] = z ^ (q >= 1 ? u[q - 1] : 0) ^ (q >= 3 ? u[q - 3] : 0);
    }
    if (tc >= 2) h = u[tc - 2];
    int ce = h ? (int)(int8_t)(t->cs >> (8 * e)) : 0;
    int v = ((int)(int8_t)(t->A[f1] >> (8 * e)) + ce) * (1 << orc_sh1(c));
    if (W2) v += ((int)(int8_t)(t->A[f2] >> (8 * e)) + ce) * (1 << orc_sh2(c));
    if (W3) v += (int)(int8_t)(t->A[f3] >> (8 * e)) + ce;
    return v;
}

/* ---------------------------------------------------------------- FWHT + dequant (CPU.patch:533-537, :1012-1027) */
void orc_fwht256(float *v) {
    for (int h = 1; h < 256; h <<= 1)
        for (int i = 0; i < 256; ++i)
            if (!(i & h)) {
                float a = v[i], b = v[i + h];
                v[i] = a + b;
                v[i + h] = a - b;
            }
    for (int i = 0; i < 256; ++i) v[i] *= 0.0625f;
}

void orc_dequant_f32(const orc_tensor *t, float *W) {
    int16_t tile[32 * 256];
    float v[256];
    for (int g = 0; g < t->ng; ++g)
        for (int b = 0; b < t->nb; ++b) {
            orc_decode_tile(t, g, b, tile);
            for (int j = 0; j < 32; ++j) {
                int r = 32 * g + j, ro = t->prm[r];
                float sc = orc_h2f(t->S[(size_t)b * t->rows + r]);
                for (int i = 0; i < 256; ++i) v[i] = (float)tile[j * 256 + i] * sc;
                orc_fwht256(v);
                for (int i = 0; i < 256; ++i) v[i] *= t->ic[256 * b + i];
                for (int e = t->cp[ro]; e < t->cp[ro + 1]; ++e) {
                    int col = (int)t->cc[e] - 256 * b;
                    if (col >= 0 && col < 256) v[col] += t->cv[e];
                }
                memcpy(W + (size_t)ro * t->K + 256 * b, v, sizeof(v));
            }
        }
}

/* ---------------------------------------------------------------- activation prep (CPU.patch:559-616, :4292-4307) */
static void rotate_block(const orc_tensor *t, const float *x, int b, float v[256]) {
    for (int i = 0; i < 256; ++i) v[i] = x[256 * b + i] * t->ic[256 * b + i];
    orc_fwht256(v);
}

void orc_rotate_act(const orc_tensor *t, const float *x, float *xr) {
    for (int b = 0; b < t->nb; ++b) rotate_block(t, x, b, xr + 256 * b);
}

void orc_prep_q8_128(const orc_tensor *t, const float *x, int8_t *q, float *d, int32_t *sx) {
    float v[256];
    for (int b = 0; b < t->nb; ++b) {
        rotate_block(t, x, b, v);
        for (int hs = 0; hs < 2; ++hs) {
            const float *u = v + 128 * hs;
            float am = 0.f;
            for (int i = 0; i < 128; ++i) am = fmaxf(am, fabsf(u[i]));
            float dd = am / 127.f, id = dd > 0.f ? 1.f / dd : 0.f;
            int32_t s = 0;
            for (int i = 0; i < 128; ++i) {
                int qi = (int)nearbyintf(u[i] * id);
                q[256 * b + 128 * hs + i] = (int8_t)qi;
                s += qi;
            }
            d[2 * b + hs] = dd;
            sx[2 * b + hs] = s;
        }
    }
}

void orc_prep_x16(const orc_tensor *t, const float *x, int8_t *qh, float *dh, int32_t *sh, int8_t *ql, float *dl, int32_t *sl) {
    float v[256];
    for (int b = 0; b < t->nb; ++b) {
        rotate_block(t, x, b, v);
        for (int hs = 0; hs < 2; ++hs) {
            const float *u = v + 128 * hs;
            float am = 0.f;
            for (int i = 0; i < 128; ++i) am = fmaxf(am, fabsf(u[i]));
            float dd = am / 8191.f, id = dd > 0.f ? 1.f / dd : 0.f;
            int32_t a = 0, c = 0;
            for (int i = 0; i < 128; ++i) {
                int qq = (int)nearbyintf(u[i] * id);
                int hi = (qq + 64) >> 7, lo = qq - 128 * hi;
                qh[256 * b + 128 * hs + i] = (int8_t)hi;
                ql[256 * b + 128 * hs + i] = (int8_t)lo;
                a += hi; c += lo;
            }
            dh[2 * b + hs] = 128.f * dd; dl[2 * b + hs] = dd;
            sh[2 * b + hs] = a; sl[2 * b + hs] = c;
        }
    }
}

/* ggml block_q8_1 over x', following ggml's quantize_row_q8_1_ref (llama.cpp @7ac59a6, not vendored in the reference):
 * d = amax/127, id = 1/d, q = roundf(x * id) (ties away from zero), d stored as fp16, s = fp16(d * sum q).
 * The reference calls ggml's CUDA quantize_row_q8_1_cuda at CPU.patch:1576 and restates its rounding as rintf(x/d) in
 * its own check at CPU.patch:2283-2286; the conventions differ only at exact ties (and in s, which the VR products do
 * not read). Pinned by crafted ties in tests/test_oracle.py. */
void orc_quantize_q8_1(const orc_tensor *t, const float *x, uint8_t *blocks) {
    float *xr = (float *)malloc(sizeof(float) * (size_t)t->K);
    orc_rotate_act(t, x, xr);
    for (int ib = 0; ib < t->K / 32; ++ib) {
        const float *u = xr + 32 * ib;
        float am = 0.f;
        for (int i = 0; i < 32; ++i) am = fmaxf(am, fabsf(u[i]));
        float dd = am / 127.f, id = dd != 0.f ? 1.f / dd : 0.f;
        uint8_t *blk = blocks + 36 * (size_t)ib;
        int s = 0;
        for (int i = 0; i < 32; ++i) {
            int qi = (int)roundf(u[i] * id);
            blk[4 + i] = (uint8_t)(int8_t)qi;
            s += qi;
        }
        uint16_t hd = orc_f2h(dd), hsum = orc_f2h((float)s * dd);
        memcpy(blk, &hd, 2);
        memcpy(blk + 2, &hsum, 2);
    }
    free(xr);
}

/* ---------------------------------------------------------------- integer partials and fp64 GEMV (CPU.patch:617-668, :3951-4016) */
void orc_partials_q8_128(const orc_tensor *t, const int8_t *q, int32_t *isum) {
    int16_t tile[32 * 256];
    for (int g = 0; g < t->ng; ++g)
        for (int b = 0; b < t->nb; ++b) {
            orc_decode_tile(t, g, b, tile);
            for (int j = 0; j < 32; ++j)
                for (int hs = 0; hs < 2; ++hs) {
                    int64_t s = 0;
                    for (int i = 0; i < 128; ++i) s += (int64_t)tile[j * 256 + 128 * hs + i] * q[256 * b + 128 * hs + i];
                    isum[(size_t)(32 * g + j) * t->nsl + 2 * b + hs] = (int32_t)s;
                }
        }
}

void orc_partials_q8_1(const orc_tensor *t, const uint8_t *blocks, int32_t *isum) {
    int16_t tile[32 * 256];
    int nq = t->K / 32;
    for (int g = 0; g < t->ng; ++g)
        for (int b = 0; b < t->nb; ++b) {
            orc_decode_tile(t, g, b, tile);
            for (int j = 0; j < 32; ++j)
                for (int qb = 0; qb < 8; ++qb) {
                    const int8_t *qs = (const int8_t *)(blocks + 36 * (size_t)(8 * b + qb) + 4);
                    int64_t s = 0;
                    for (int i = 0; i < 32; ++i) s += (int64_t)tile[j * 256 + 32 * qb + i] * qs[i];
                    isum[(size_t)(32 * g + j) * nq + 8 * b + qb] = (int32_t)s;
                }
        }
}

static void add_delta_f64(const orc_tensor *t, const float *x, double *y) {
    for (int ro = 0; ro < t->rows; ++ro)
        for (int e = t->cp[ro]; e < t->cp[ro + 1]; ++e) y[ro] += (double)t->cv[e] * (double)x[t->cc[e]];
}

void orc_gemv_q8_128_f64(const orc_tensor *t, const float *x, double *y) {
    int8_t *q = (int8_t *)malloc((size_t)t->K);
    float *d = (float *)malloc(sizeof(float) * (size_t)t->nsl);
    int32_t *sx = (int32_t *)malloc(sizeof(int32_t) * (size_t)t->nsl);
    int32_t *isum = (int32_t *)malloc(sizeof(int32_t) * (size_t)t->rows * t->nsl);
    orc_prep_q8_128(t, x, q, d, sx);
    orc_partials_q8_128(t, q, isum);
    for (int r = 0; r < t->rows; ++r) {
        double acc = 0.0;
        for (int s = 0; s < t->nsl; ++s)
            acc += (double)isum[(size_t)r * t->nsl + s] * (double)d[s] * (double)orc_h2f(t->S[(size_t)(s >> 1) * t->rows + r]);
        y[t->prm[r]] = acc;
    }
    add_delta_f64(t, x, y);
    free(q); free(d); free(sx); free(isum);
}

/* fp64 GEMV on x16 activations (vrc_prep_block16 planes, CPU.patch:575-616; the planes are two virtual columns that the
 * reference sums before the clamp delta, CPU.patch:1232-1244, :1193): y[prm[r]] = sum_s S (hi_s 128 d_s + lo_s d_s)
 * + delta . x, with hi_s / lo_s the integer partials of each plane */
void orc_gemv_x16_f64(const orc_tensor *t, const float *x, double *y) {
    int8_t *qh = (int8_t *)malloc((size_t)t->K), *ql = (int8_t *)malloc((size_t)t->K);
    float *dh = (float *)malloc(sizeof(float) * (size_t)t->nsl), *dl = (float *)malloc(sizeof(float) * (size_t)t->nsl);
    int32_t *sh = (int32_t *)malloc(sizeof(int32_t) * (size_t)t->nsl), *sl = (int32_t *)malloc(sizeof(int32_t) * (size_t)t->nsl);
    int32_t *ih = (int32_t *)malloc(sizeof(int32_t) * (size_t)t->rows * t->nsl), *il = (int32_t *)malloc(sizeof(int32_t) * (size_t)t->rows * t->nsl);
    orc_prep_x16(t, x, qh, dh, sh, ql, dl, sl);
    orc_partials_q8_128(t, qh, ih);
    orc_partials_q8_128(t, ql, il);
    for (int r = 0; r < t->rows; ++r) {
        double acc = 0.0;
        for (int s = 0; s < t->nsl; ++s) {
            const double sc = (double)orc_h2f(t->S[(size_t)(s >> 1) * t->rows + r]);
            acc += ((double)ih[(size_t)r * t->nsl + s] * (double)dh[s] + (double)il[(size_t)r * t->nsl + s] * (double)dl[s]) * sc;
        }
        y[t->prm[r]] = acc;
    }
    add_delta_f64(t, x, y);
    free(qh); free(ql); free(dh); free(dl); free(sh); free(sl); free(ih); free(il);
}

/* the same fp64 GEMV for ncols activation columns x [ncols][ldx] -> y [ncols][rows], each tile decoded once;
 * per column the arithmetic (integer partials, then the half-slice sum in order) is orc_gemv_q8_128_f64's */
void orc_gemv_q8_128_f64_cols(const orc_tensor *t, const float *x, int ncols, size_t ldx, double *y) {
    int8_t *q = (int8_t *)malloc((size_t)t->K * ncols);
    float *d = (float *)malloc(sizeof(float) * (size_t)t->nsl * ncols);
    int32_t *sx = (int32_t *)malloc(sizeof(int32_t) * (size_t)t->nsl);
    int32_t *isum = (int32_t *)malloc(sizeof(int32_t) * (size_t)t->rows * t->nsl * ncols);
    int16_t tile[32 * 256];
    for (int n = 0; n < ncols; ++n) orc_prep_q8_128(t, x + (size_t)n * ldx, q + (size_t)n * t->K, d + (size_t)n * t->nsl, sx);
    for (int g = 0; g < t->ng; ++g)
        for (int b = 0; b < t->nb; ++b) {
            orc_decode_tile(t, g, b, tile);
            for (int n = 0; n < ncols; ++n)
                for (int j = 0; j < 32; ++j)
                    for (int hs = 0; hs < 2; ++hs) {
                        const int8_t *qn = q + (size_t)n * t->K + 256 * b + 128 * hs;
                        int64_t s = 0;
                        for (int i = 0; i < 128; ++i) s += (int64_t)tile[j * 256 + 128 * hs + i] * qn[i];
                        isum[((size_t)n * t->rows + 32 * g + j) * t->nsl + 2 * b + hs] = (int32_t)s;
                    }
        }
    for (int n = 0; n < ncols; ++n) {
        double *yn = y + (size_t)n * t->rows;
        for (int r = 0; r < t->rows; ++r) {
            double acc = 0.0;
            for (int s = 0; s < t->nsl; ++s)
                acc += (double)isum[((size_t)n * t->rows + r) * t->nsl + s] * (double)d[(size_t)n * t->nsl + s] *
                       (double)orc_h2f(t->S[(size_t)(s >> 1) * t->rows + r]);
            yn[t->prm[r]] = acc;
        }
        add_delta_f64(t, x + (size_t)n * ldx, yn);
    }
    free(q); free(d); free(sx); free(isum);
}

void orc_gemv_q8_1_f64(const orc_tensor *t, const float *x, double *y) {
    int nq = t->K / 32;
    uint8_t *blk = (uint8_t *)malloc(36 * (size_t)nq);
    int32_t *isum = (int32_t *)malloc(sizeof(int32_t) * (size_t)t->rows * nq);
    orc_quantize_q8_1(t, x, blk);
    orc_partials_q8_1(t, blk, isum);
    for (int r = 0; r < t->rows; ++r) {
        double acc = 0.0;
        for (int s = 0; s < nq; ++s) {
            uint16_t hd; memcpy(&hd, blk + 36 * (size_t)s, 2);
            acc += (double)isum[(size_t)r * nq + s] * (double)orc_h2f(hd) * (double)orc_h2f(t->S[(size_t)(s >> 3) * t->rows + r]);
        }
        y[t->prm[r]] = acc;
    }
    add_delta_f64(t, x, y);
    free(blk); free(isum);
}

void orc_dense_f64(const float *W, int rows, int K, const float *x, int N, double *y) {
    for (int n = 0; n < N; ++n)
        for (int r = 0; r < rows; ++r) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += (double)W[(size_t)r * K + k] * (double)x[(size_t)n * K + k];
            y[(size_t)n * rows + r] = acc;
        }
}
