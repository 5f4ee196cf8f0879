// p8x_host.cpp -- host side of the C ABI: slot validation, device metadata, argument checks.
//
// p8x_prepare restates the reference's load-time checks and derived data: trailer/header checks and
// ic = sg / c (vrc_init, CPU.patch:240-275), kbytes against the M words and the delta CSR by original row
// (vr_prepare_native, CPU.patch:4335-4390). Failures return P8X_ERR_FORMAT instead of aborting.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "p8x_internal.h"

namespace p8x {

static thread_local char g_err[512] = "";

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_check(hipError_t e, const char *what) {
    if (e == hipSuccess) return P8X_OK;
    return set_error(P8X_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int num_cus() {
    static int cus = -1;
    if (cus < 0) {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess) cus = prop.multiProcessorCount;
        else cus = 256;
    }
    return cus;
}

static int nw_tile(uint32_t m) { return nw_of((int)(m >> 29)); }

void side_offsets(size_t n, size_t rows, size_t K, size_t nd, size_t off[6]) {
    const size_t t = n - 32, sg = t - 256;
    const size_t q = (sg - 2 * rows) & ~(size_t)15;
    const size_t p = (q - 2 * rows) & ~(size_t)15;
    const size_t c = (p - 2 * K) & ~(size_t)15;
    const size_t e = (c - 8 * nd) & ~(size_t)15;
    off[0] = e; off[1] = c; off[2] = p; off[3] = q; off[4] = sg; off[5] = t;
}

// row scales [nb][rows] -> [ng][nb][32], one element per thread
__global__ void k_regroup_scales(const uint16_t *__restrict__ S, uint16_t *__restrict__ Sg, int nb, int rows, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const size_t gb = i >> 5;
    const int j = (int)(i & 31), g = (int)(gb / nb), b = (int)(gb % nb);
    Sg[i] = S[(size_t)b * rows + 32 * g + j];
}

// Field k of a region of W-bit fields starting at word o of a lane's words (bit string little-endian across words).
__device__ uint32_t lane_field(const uint32_t *w, int o, int W, int k) {
    const int pos = W * k, wi = o + (pos >> 5), bb = pos & 31;
    uint64_t v = w[wi];
    if (bb + W > 32) v |= (uint64_t)w[wi + 1] << 32;
    return (uint32_t)(v >> bb) & ((1u << W) - 1u);
}
__device__ void lane_field_put(uint32_t *w, int o, int W, int k, uint32_t f) {
    const int pos = W * k, wi = o + (pos >> 5), bb = pos & 31;
    w[wi] |= f << bb;
    if (bb + W > 32) w[wi + 1] |= f >> (32 - bb);
}
// lane j's region (32 fields of W bits at word o): stored field k encodes chunk (j + k) & 31 (CPU.patch:155-158);
// out field t = chunk t
__device__ void lane_region_to_chunks(const uint32_t *in, uint32_t *out, int o, int W, int j) {
    for (int t = 0; t < 32; ++t) lane_field_put(out, o, W, t, lane_field(in, o, W, (t - j) & 31));
}

// Tile payloads from the file layout to the device layout, one 64-thread block per tile, thread (hs, j) for the
// NW words of lane j of half-slice hs: every region's fields rotated into chunk order (field t = chunk t, so the
// chunk of a step is the same for every lane), the label word of classes with W1 < 8 likewise (bit t = chunk t),
// and the words placed in 16-byte groups (file_word -> dev_word). Every tile lies inside the payload (checked at
// prepare).
__global__ void k_relayout_payload(const uint32_t *__restrict__ src, uint32_t *__restrict__ dst, const uint32_t *__restrict__ M) {
    const uint32_t m = M[blockIdx.x];
    const int c = (int)(m >> 29), nw = nw_of(c), w1 = w1_of(c), w2 = w2_of(c), w3 = w3_of(c);
    const int hs = threadIdx.x >> 5, j = threadIdx.x & 31;
    const size_t base = (size_t)(m & 0x1FFFFFFFu) + (size_t)hs * nw * 32;
    uint32_t in[24], out[24];
    for (int i = 0; i < nw; ++i) { in[i] = src[base + file_word(i, j)]; out[i] = 0u; }
    if (w1 == 8) lane_region_to_chunks(in, out, 0, 8, j);
    else if (w1 > 0) {
        out[0] = (in[0] << j) | (j ? in[0] >> (32 - j) : 0u);   // label bit k -> bit (j + k) & 31
        lane_region_to_chunks(in, out, 1, w1 - 1, j);
    }
    if (w2) lane_region_to_chunks(in, out, w1, w2, j);
    if (w3) lane_region_to_chunks(in, out, w1 + w2, w3, j);
    for (int i = 0; i < nw; ++i) dst[base + dev_word(i, j, nw)] = out[i];
}

}  // namespace p8x

using namespace p8x;

extern "C" {

const char *p8x_version(void) { return "p8x 0.1 (gfx950)"; }

const char *p8x_error_string(int code) {
    switch (code) {
        case P8X_OK: return "ok";
        case P8X_ERR_ARG: return "invalid argument";
        case P8X_ERR_FORMAT: return "slot bytes fail the tensor contract";
        case P8X_ERR_HIP: return "HIP runtime error";
        case P8X_ERR_UNSUPPORTED: return "unsupported request";
        case P8X_ERR_NOMEM: return "out of memory";
        default: return "unknown error";
    }
}

const char *p8x_last_error(void) { return g_err; }

size_t p8x_need(size_t kbytes, int rows, int K, int nd) {
    return align16(kbytes) + align16(8 * (size_t)nd) + align16(2 * (size_t)K) + 2 * align16(2 * (size_t)rows) + 256 + 32 + 64;
}

int p8x_probe(const void *slot, size_t n, int rows, int K) {
    if (!slot || n < kHeaderBytes + 256 + 32) return 0;
    uint32_t tr[8];
    memcpy(tr, (const uint8_t *)slot + n - 32, 32);
    return tr[0] == kMagic0 && tr[1] == kMagic1 && tr[4] == (uint32_t)rows && tr[5] == (uint32_t)K && tr[6] == kNS;
}


void p8x_release(p8x_tensor *t) {
    if (!t) return;
    for (void *p : {(void *)t->owned, (void *)t->Dl, (void *)t->wy, (void *)t->wglu, (void *)t->wslot, (void *)t->djob, (void *)t->Sg, (void *)t->a2, (void *)t->ic, (void *)t->cp, (void *)t->cc, (void *)t->cv, (void *)t->wq,
                    (void *)t->wd, (void *)t->wsum, (void *)t->wq81, (void *)t->wpart, (void *)t->wcnt, (void *)t->drows, (void *)t->pinv, (void *)t->prmd, (void *)t->wx16, (void *)t->wmm})
        if (p) (void)hipFree(p);
    delete t;
}

int p8x_prepare(const void *slot, size_t n, int rows, int K, int on_device, p8x_tensor **out) {
    if (!slot || !out) return set_error(P8X_ERR_ARG, "p8x_prepare: null pointer");
    *out = nullptr;
    if (rows <= 0 || K <= 0 || K % 256 || rows % 32 || rows >= 32768)
        return set_error(P8X_ERR_ARG, "p8x_prepare: shape %d x %d (need K %% 256 == 0, rows %% 32 == 0, rows < 32768)", rows, K);
    // fixed regions: header, Hadamard signs, trailer (the variable ones are checked against the trailer below)
    if (n < kHeaderBytes + 256 + 32) return set_error(P8X_ERR_FORMAT, "p8x_prepare: slot of %zu bytes is too small", n);
    const uint8_t *src = (const uint8_t *)slot;
    auto fetch = [&](size_t off, size_t len, void *dst) -> int {
        if (off + len > n) return set_error(P8X_ERR_FORMAT, "p8x_prepare: region [%zu, %zu) beyond the slot", off, off + len);
        if (!len) return P8X_OK;
        if (on_device) return hip_check(hipMemcpy(dst, src + off, len, hipMemcpyDeviceToHost), "p8x_prepare: read slot");
        memcpy(dst, src + off, len);
        return P8X_OK;
    };
    int rc;
    uint32_t tr[8];
    if ((rc = fetch(n - 32, 32, tr))) return rc;
    if (tr[0] != kMagic0 || tr[1] != kMagic1)
        return set_error(P8X_ERR_FORMAT, "p8x_prepare: bad trailer magic %08x %08x", tr[0], tr[1]);
    if (tr[4] != (uint32_t)rows || tr[5] != (uint32_t)K || tr[6] != kNS)
        return set_error(P8X_ERR_FORMAT, "p8x_prepare: trailer rows %u K %u ns %u, expected %d %d %u", tr[4], tr[5], tr[6], rows, K, kNS);
    const int nb = K / 256, ng = rows / 32, nsl = K / 128, nd = (int)tr[3];
    const size_t nt = (size_t)ng * nb, kbytes = tr[2];
    std::vector<uint32_t> hdr(516), M(nt);
    if ((rc = fetch(0, 2064, hdr.data()))) return rc;
    if (hdr[513] != kNS || hdr[514] != kTRL)
        return set_error(P8X_ERR_FORMAT, "p8x_prepare: header NS %u TRL %u (need %u, %u)", hdr[513], hdr[514], kNS, kTRL);
    if ((rc = fetch(kHeaderBytes, 4 * nt, M.data()))) return rc;
    size_t off[6];
    if ((size_t)nd > n / 8) return set_error(P8X_ERR_FORMAT, "p8x_prepare: delta count %d too large", nd);
    side_offsets(n, (size_t)rows, (size_t)K, (size_t)nd, off);
    if (off[0] > n || kbytes > off[0]) return set_error(P8X_ERR_FORMAT, "p8x_prepare: kbytes %zu overlaps the side regions", kbytes);
    size_t words = 0, hist[8] = {0};
    for (size_t i = 0; i < nt; ++i) { words += (size_t)64 * nw_tile(M[i]); hist[M[i] >> 29]++; }
    if (offset_D(nt) + 4 * words != kbytes)
        return set_error(P8X_ERR_FORMAT, "p8x_prepare: kbytes %zu != M-implied %zu", kbytes, offset_D(nt) + 4 * words);
    for (size_t i = 0; i < nt; ++i) {   // every tile's payload must lie inside D
        const size_t o = M[i] & 0x1FFFFFFFu;
        if (o + (size_t)64 * nw_tile(M[i]) > words)
            return set_error(P8X_ERR_FORMAT, "p8x_prepare: tile %zu payload offset %zu out of range", i, o);
    }
    std::vector<uint16_t> c16(K);
    std::vector<int16_t> prm(rows);
    std::vector<int8_t> sg(256);
    std::vector<uint16_t> drow(nd), dcol(nd);
    std::vector<float> dval(nd);
    if ((rc = fetch(off[1], 2 * (size_t)K, c16.data()))) return rc;
    if ((rc = fetch(off[2], 2 * (size_t)rows, prm.data()))) return rc;
    if ((rc = fetch(off[4], 256, sg.data()))) return rc;
    if (nd) {
        if ((rc = fetch(off[0], 2 * (size_t)nd, drow.data()))) return rc;
        if ((rc = fetch(off[0] + 2 * (size_t)nd, 2 * (size_t)nd, dcol.data()))) return rc;
        if ((rc = fetch(off[0] + 4 * (size_t)nd, 4 * (size_t)nd, dval.data()))) return rc;
    }
    {   // prm must be a permutation (CPU.patch:4852-4857)
        std::vector<char> seen(rows, 0);
        for (int r = 0; r < rows; ++r) {
            if (prm[r] < 0 || prm[r] >= rows || seen[prm[r]]) return set_error(P8X_ERR_FORMAT, "p8x_prepare: prm is not a permutation (row %d)", r);
            seen[prm[r]] = 1;
        }
    }
    for (int e = 0; e < nd; ++e)
        if (drow[e] >= rows || dcol[e] >= K) return set_error(P8X_ERR_FORMAT, "p8x_prepare: delta entry %d out of range", e);
    for (int i = 0; i < 256; ++i)
        if (sg[i] != 1 && sg[i] != -1) return set_error(P8X_ERR_FORMAT, "p8x_prepare: Hadamard sign %d is %d", i, sg[i]);

    // derived host data
    // coset entries A[f] + c with the CPU core's bytewise int8 add (CPU.patch:221, :255), which wraps when |A + c|
    // exceeds 127; every kernel decodes through this table, so products equal dequantize_row's weights times x
    // for any codebook (the shipped one never wraps: A + c lies in [-76, 62])
    std::vector<uint32_t> a2(512);
    for (int f = 0; f < 256; ++f) {
        a2[f] = hdr[f];
        a2[256 + f] = add_bytes(hdr[f], hdr[512]);
    }
    // the same entries as four fp16 each (exact: |v| <= 128), entry 2 f + h, behind the words in the device copy
    // (the prompt GEMM's fp16 table replicates them)
    std::vector<uint16_t> a2h(512 * 4);
    for (int r = 0; r < 512; ++r)
        for (int e = 0; e < 4; ++e) {
            const int v = (int8_t)(a2[(r & 1) * 256 + (r >> 1)] >> (8 * e));
            const unsigned a = (unsigned)(v < 0 ? -v : v);
            const int ex = a ? 31 - __builtin_clz(a) : 0;
            a2h[4 * r + e] = a ? (uint16_t)((v < 0 ? 0x8000u : 0u) | (unsigned)(ex + 15) << 10 | ((a << (10 - ex)) & 0x3FFu)) : 0;
        }
    std::vector<float> ic(K);
    for (int k = 0; k < K; ++k) ic[k] = (float)sg[k & 255] / half_to_float(c16[k]);
    uint64_t ic_hash = 1469598103934665603ull;   // FNV-1a over the rotation's bytes (K included)
    for (int k = 0; k < K; ++k) {
        uint32_t b;
        memcpy(&b, &ic[k], 4);
        for (int i = 0; i < 4; ++i) ic_hash = (ic_hash ^ ((b >> (8 * i)) & 0xFFu)) * 1099511628211ull;
    }
    std::vector<int> cp(rows + 1, 0);
    std::vector<uint16_t> cc(nd);
    std::vector<float> cv(nd);
    for (int e = 0; e < nd; ++e) cp[drow[e] + 1]++;
    for (int r = 0; r < rows; ++r) cp[r + 1] += cp[r];
    {
        std::vector<int> fill(cp.begin(), cp.end() - 1);
        for (int e = 0; e < nd; ++e) { const int q = fill[drow[e]]++; cc[q] = dcol[e]; cv[q] = dval[e]; }
    }

    p8x_tensor *t = new p8x_tensor();
    t->rows = rows; t->K = K; t->nb = nb; t->ng = ng; t->nsl = nsl; t->nd = nd;
    t->n = n; t->nt = nt; t->kbytes = kbytes;
    t->stream_bytes = 4 * nt + 64 * nt + 4 * words;
    t->ic_hash = ic_hash;
    t->ic_host = ic;
    for (int c = 0; c < 8; ++c) t->class_tiles[c] = hist[c];
    for (int c = 1; c < 8; ++c)
        if (hist[c] == nt) {   // one class: are the tiles in order (tile i at word i * 64 nw)?
            t->lin_words = 64u * (unsigned)nw_of(c);
            for (size_t i = 0; i < nt && t->lin_words; ++i)
                if ((size_t)(M[i] & 0x1FFFFFFFu) != i * t->lin_words) t->lin_words = 0;
        }
    memcpy(t->a2_host, a2.data(), sizeof t->a2_host);
    (void)hipGetDevice(&t->device);
    if ((rc = scratch_resolve(t->device))) { delete t; return rc; }   // set-up of the no-allocation entry point
    if ((rc = act_cache_resolve(t->device))) { delete t; return rc; }   // and of the prepared-activation reuse
    auto fail = [&](int code) { p8x_release(t); return code; };
    auto alloc = [&](void **p, size_t bytes, const char *what) -> int {
        if (hipMalloc(p, bytes ? bytes : 16) != hipSuccess) return set_error(P8X_ERR_NOMEM, "p8x_prepare: hipMalloc %s (%zu B)", what, bytes);
        return P8X_OK;
    };
    if (on_device) {
        t->base = src;
    } else {
        // payload tiles on 256-byte boundaries: every tile then covers whole cache lines
        const size_t pad = (256 - offset_D(nt) % 256) % 256;
        if ((rc = alloc((void **)&t->owned, n + pad, "slot"))) return fail(rc);
        if ((rc = hip_check(hipMemcpy(t->owned + pad, src, n, hipMemcpyHostToDevice), "p8x_prepare: upload slot"))) return fail(rc);
        t->base = t->owned + pad;
    }
    t->M = (const uint32_t *)(t->base + kHeaderBytes);
    t->S = (const uint16_t *)(t->base + offset_S(nt));
    t->D = (const uint32_t *)(t->base + offset_D(nt));
    t->prm = (const int16_t *)(t->base + off[2]);
    if (words) {
        // payload to the device layout (16-byte groups per lane): in place in the library's copy (through a temporary
        // copy of the file payload), or into a payload copy of its own when the caller owns the slot
        uint32_t *dst = nullptr, *tmp = nullptr;
        const uint32_t *srcD = t->D;
        if (on_device) {
            if ((rc = alloc((void **)&t->Dl, 4 * words, "payload"))) return fail(rc);
            dst = t->Dl;
        } else {
            if ((rc = alloc((void **)&tmp, 4 * words, "payload staging"))) return fail(rc);
            if ((rc = hip_check(hipMemcpy(tmp, t->D, 4 * words, hipMemcpyDeviceToDevice), "p8x_prepare: payload staging"))) {
                (void)hipFree(tmp);
                return fail(rc);
            }
            srcD = tmp;
            dst = const_cast<uint32_t *>(t->D);
        }
        hipLaunchKernelGGL(k_relayout_payload, dim3((unsigned)nt), dim3(64), 0, 0, srcD, dst, t->M);
        rc = hip_check(hipGetLastError(), "p8x_prepare: payload layout");
        if (!rc) rc = hip_check(hipDeviceSynchronize(), "p8x_prepare: payload layout");
        if (tmp) (void)hipFree(tmp);
        if (rc) return fail(rc);
        t->D = dst;
    }
    for (int nc = 1; nc <= P8X_MAX_COLS; ++nc) {   // partial rows of the largest single-GEMV plan
        for (int act : {P8X_ACT_Q8_128, P8X_ACT_Q8_1}) {
            const GemvPlan plan = gemv_plan(t, nc, act, false);
            if (plan.nks > 1) t->wpart_floats = std::max(t->wpart_floats, (size_t)plan.nks * nc * rows);
            int kc;
            const int rn = rg_plan(t, nc, &kc);
            if (rn > 1) t->wpart_floats = std::max(t->wpart_floats, (size_t)rn * nc * rows);
            if (nc == 1) {
                const GemvPlan pp = gemv_plan(t, 1, act, true);
                if (pp.nks > 1) t->wpart_floats = std::max(t->wpart_floats, (size_t)pp.nks * rows);
            }
        }
    }
    if ((rc = alloc((void **)&t->Sg, 64 * nt, "regrouped scales"))) return fail(rc);
    hipLaunchKernelGGL(k_regroup_scales, dim3((unsigned)((32 * nt + 255) / 256)), dim3(256), 0, 0, t->S, t->Sg, nb, rows, 32 * nt);
    if ((rc = hip_check(hipGetLastError(), "p8x_prepare: regroup scales"))) return fail(rc);
    if ((rc = alloc((void **)&t->a2, 512 * 4 + 512 * 8, "tables"))) return fail(rc);
    if ((rc = alloc((void **)&t->ic, 4 * (size_t)K, "ic"))) return fail(rc);
    if ((rc = alloc((void **)&t->cp, 4 * (size_t)(rows + 1), "delta rows"))) return fail(rc);
    if ((rc = alloc((void **)&t->cc, 2 * (size_t)nd, "delta cols"))) return fail(rc);
    if ((rc = alloc((void **)&t->cv, 4 * (size_t)nd, "delta values"))) return fail(rc);
    if ((rc = alloc((void **)&t->wq, (size_t)P8X_MAX_COLS * K, "q"))) return fail(rc);
    if ((rc = alloc((void **)&t->wd, 4 * (size_t)P8X_MAX_COLS * nsl, "d"))) return fail(rc);
    if ((rc = alloc((void **)&t->wsum, 4 * (size_t)P8X_MAX_COLS * nsl, "sum"))) return fail(rc);
    if ((rc = alloc((void **)&t->wq81, (size_t)36 * P8X_MAX_COLS * (K / 32), "q8_1"))) return fail(rc);
    if ((rc = alloc((void **)&t->wpart, 4 * t->wpart_floats, "partials"))) return fail(rc);
    if ((rc = alloc((void **)&t->wy, 4 * (size_t)P8X_MAX_COLS * rows, "x16 plane rows"))) return fail(rc);
    if ((rc = alloc((void **)&t->wglu, 8 * (size_t)rows, "gate / up slots"))) return fail(rc);
    if ((rc = hip_check(hipMemset(t->wglu, 0, 8 * (size_t)rows), "p8x_prepare: gate / up slots"))) return fail(rc);
    if ((rc = alloc((void **)&t->wslot, 8 * (size_t)rows, "K-half slots"))) return fail(rc);
    if ((rc = hip_check(hipMemset(t->wslot, 0, 8 * (size_t)rows), "p8x_prepare: K-half slots"))) return fail(rc);
    if ((rc = alloc((void **)&t->wcnt, 4 * (size_t)ng, "counters"))) return fail(rc);
    {
        std::vector<int16_t> pinv(rows);
        bool ident = true;
        for (int r = 0; r < rows; ++r) { pinv[prm[r]] = (int16_t)r; ident = ident && prm[r] == r; }
        t->prm_identity = ident;
        t->pinv_host = pinv;
        if ((rc = alloc((void **)&t->pinv, 2 * (size_t)rows, "pinv"))) return fail(rc);
        if ((rc = hip_check(hipMemcpy(t->pinv, pinv.data(), 2 * (size_t)rows, hipMemcpyHostToDevice), "p8x_prepare: pinv"))) return fail(rc);
    }
    {   // sorted row -> original row with the delta flag: the single-GEMV epilogue needs one load per row
        std::vector<uint16_t> pd(rows);
        for (int r = 0; r < rows; ++r) pd[r] = (uint16_t)((uint16_t)prm[r] | (cp[prm[r] + 1] > cp[prm[r]] ? 0x8000u : 0u));
        if ((rc = alloc((void **)&t->prmd, 2 * (size_t)rows, "flagged permutation"))) return fail(rc);
        if ((rc = hip_check(hipMemcpy(t->prmd, pd.data(), 2 * (size_t)rows, hipMemcpyHostToDevice), "p8x_prepare: flagged permutation"))) return fail(rc);
    }
    std::vector<int> drows;
    for (int r = 0; r < rows; ++r) if (cp[r + 1] > cp[r]) drows.push_back(r);
    t->ndrows = (int)drows.size();
    t->dorig = drows;
    if ((rc = alloc((void **)&t->drows, 4 * std::max<size_t>(1, drows.size()), "delta row list"))) return fail(rc);
    if (!drows.empty() && (rc = hip_check(hipMemcpy(t->drows, drows.data(), 4 * drows.size(), hipMemcpyHostToDevice), "p8x_prepare: delta rows")))
        return fail(rc);
    if ((rc = hip_check(hipMemcpy(t->a2, a2.data(), 512 * 4, hipMemcpyHostToDevice), "p8x_prepare: tables")) ||
        (rc = hip_check(hipMemcpy(t->a2 + 512, a2h.data(), 512 * 8, hipMemcpyHostToDevice), "p8x_prepare: tables"))) return fail(rc);
    if ((rc = hip_check(hipMemcpy(t->ic, ic.data(), 4 * (size_t)K, hipMemcpyHostToDevice), "p8x_prepare: ic"))) return fail(rc);
    if ((rc = hip_check(hipMemcpy(t->cp, cp.data(), 4 * (size_t)(rows + 1), hipMemcpyHostToDevice), "p8x_prepare: csr"))) return fail(rc);
    if (nd) {
        if ((rc = hip_check(hipMemcpy(t->cc, cc.data(), 2 * (size_t)nd, hipMemcpyHostToDevice), "p8x_prepare: csr"))) return fail(rc);
        if ((rc = hip_check(hipMemcpy(t->cv, cv.data(), 4 * (size_t)nd, hipMemcpyHostToDevice), "p8x_prepare: csr"))) return fail(rc);
    }
    if ((rc = hip_check(hipMemset(t->wcnt, 0, 4 * (size_t)ng), "p8x_prepare: counters"))) return fail(rc);
    if ((rc = upload_job(t))) return fail(rc);
    if ((rc = hip_check(hipDeviceSynchronize(), "p8x_prepare: sync"))) return fail(rc);
    *out = t;
    return P8X_OK;
}

int p8x_tensor_info(const p8x_tensor *t, p8x_info *o) {
    if (!t || !o) return set_error(P8X_ERR_ARG, "p8x_tensor_info: null pointer");
    o->rows = t->rows; o->K = t->K; o->nd = t->nd; o->ng = t->ng; o->nb = t->nb;
    o->n = t->n; o->kbytes = t->kbytes; o->stream_bytes = t->stream_bytes;
    for (int c = 0; c < 8; ++c) o->class_tiles[c] = t->class_tiles[c];
    o->dev_base = t->base;
    return P8X_OK;
}

// ---------------------------------------------------------------------------------------------- device entry points
int p8x_dequantize(const p8x_tensor *t, int dtype, void *out, size_t ld, void *stream) {
    if (!t || !out) return set_error(P8X_ERR_ARG, "p8x_dequantize: null pointer");
    if (dtype != P8X_F32 && dtype != P8X_F16 && dtype != P8X_BF16) return set_error(P8X_ERR_ARG, "p8x_dequantize: dtype %d", dtype);
    if (ld < (size_t)t->K) return set_error(P8X_ERR_ARG, "p8x_dequantize: ld %zu < K %d", ld, t->K);
    return launch_dequant(t, dtype, 0, t->rows, out, ld, (hipStream_t)stream);
}

int p8x_dequantize_rows(const p8x_tensor *t, int dtype, int row0, int nrows, void *out, size_t ld, void *stream) {
    if (!t || !out) return set_error(P8X_ERR_ARG, "p8x_dequantize_rows: null pointer");
    if (dtype != P8X_F32 && dtype != P8X_F16 && dtype != P8X_BF16) return set_error(P8X_ERR_ARG, "p8x_dequantize_rows: dtype %d", dtype);
    if (row0 < 0 || nrows < 1 || row0 + nrows > t->rows) return set_error(P8X_ERR_ARG, "p8x_dequantize_rows: rows %d + %d of %d", row0, nrows, t->rows);
    if (ld < (size_t)t->K) return set_error(P8X_ERR_ARG, "p8x_dequantize_rows: ld %zu < K %d", ld, t->K);
    return launch_dequant(t, dtype, row0, nrows, out, ld, (hipStream_t)stream);
}

int p8x_decode_rotated(const p8x_tensor *t, int dtype, void *out, size_t ld, void *stream) {
    if (!t || !out) return set_error(P8X_ERR_ARG, "p8x_decode_rotated: null pointer");
    if (dtype != P8X_I16 && dtype != P8X_F32) return set_error(P8X_ERR_ARG, "p8x_decode_rotated: dtype %d", dtype);
    if (ld < (size_t)t->K) return set_error(P8X_ERR_ARG, "p8x_decode_rotated: ld %zu < K %d", ld, t->K);
    return launch_decode_rotated(t, dtype, 0, t->ng, 0, t->nb, out, ld, (hipStream_t)stream);
}

int p8x_decode_tiles(const p8x_tensor *t, int dtype, int g0, int ng, int b0, int nb, void *out, size_t ld, void *stream) {
    if (!t || !out) return set_error(P8X_ERR_ARG, "p8x_decode_tiles: null pointer");
    if (dtype != P8X_I16 && dtype != P8X_F32) return set_error(P8X_ERR_ARG, "p8x_decode_tiles: dtype %d", dtype);
    if (g0 < 0 || ng < 1 || g0 + ng > t->ng || b0 < 0 || nb < 1 || b0 + nb > t->nb)
        return set_error(P8X_ERR_ARG, "p8x_decode_tiles: tiles [%d, +%d) x [%d, +%d) of %d x %d", g0, ng, b0, nb, t->ng, t->nb);
    if (ld < (size_t)256 * nb) return set_error(P8X_ERR_ARG, "p8x_decode_tiles: ld %zu < %d", ld, 256 * nb);
    return launch_decode_rotated(t, dtype, g0, ng, b0, nb, out, ld, (hipStream_t)stream);
}

int p8x_quantize_q8_128(const p8x_tensor *t, const float *x, int ncols, size_t ldx, int8_t *q, float *d, int32_t *sum, void *stream) {
    if (!t || !x || !q || !d) return set_error(P8X_ERR_ARG, "p8x_quantize_q8_128: null pointer");
    if (ncols < 1 || ldx < (size_t)t->K || ldx % 4 || ((uintptr_t)x & 15))
        return set_error(P8X_ERR_ARG, "p8x_quantize_q8_128: ncols %d ldx %zu (x 16-byte aligned, ldx %% 4 == 0)", ncols, ldx);
    return launch_act_q8_128(t, x, ncols, ldx, q, d, sum, (hipStream_t)stream);
}

int p8x_quantize_x16(const p8x_tensor *t, const float *x, int ncols, size_t ldx, int8_t *qh, float *dh, int32_t *sh, int8_t *ql,
                     float *dl, int32_t *sl, void *stream) {
    if (!t || !x || !qh || !dh || !ql || !dl) return set_error(P8X_ERR_ARG, "p8x_quantize_x16: null pointer");
    if (ncols < 1 || ldx < (size_t)t->K || ldx % 4 || ((uintptr_t)x & 15))
        return set_error(P8X_ERR_ARG, "p8x_quantize_x16: ncols %d ldx %zu (x 16-byte aligned, ldx %% 4 == 0)", ncols, ldx);
    return launch_act_x16(t, x, ncols, ldx, qh, dh, sh, ql, dl, sl, t->K, (hipStream_t)stream);
}

int p8x_quantize_q8_1(const p8x_tensor *t, const float *x, int ncols, size_t ldx, void *blocks, void *stream) {
    if (!t || !x || !blocks) return set_error(P8X_ERR_ARG, "p8x_quantize_q8_1: null pointer");
    if (ncols < 1 || ldx < (size_t)t->K || ldx % 4 || ((uintptr_t)x & 15))
        return set_error(P8X_ERR_ARG, "p8x_quantize_q8_1: ncols %d ldx %zu (x 16-byte aligned, ldx %% 4 == 0)", ncols, ldx);
    return launch_act_q8_1(t, x, ncols, ldx, blocks, (hipStream_t)stream);
}

int p8x_vec_dot(const p8x_tensor *t, int act, const void *q, const float *d, int ncols, const float *x, size_t ldx,
                float *y, size_t ldy, int32_t *partials, void *stream) {
    if (!t || !q || !y) return set_error(P8X_ERR_ARG, "p8x_vec_dot: null pointer");
    if (act != P8X_ACT_Q8_128 && act != P8X_ACT_Q8_1) return set_error(P8X_ERR_ARG, "p8x_vec_dot: act %d", act);
    if (act == P8X_ACT_Q8_128 && !d) return set_error(P8X_ERR_ARG, "p8x_vec_dot: Q8_128 needs d");
    if (ncols < 1 || ncols > P8X_MAX_COLS || ldy < (size_t)t->rows) return set_error(P8X_ERR_ARG, "p8x_vec_dot: ncols %d ldy %zu", ncols, ldy);
    if (x && ldx < (size_t)t->K) return set_error(P8X_ERR_ARG, "p8x_vec_dot: ldx %zu < K %d", ldx, t->K);
    return launch_gemv(t, act, q, d, ncols, x, ldx, y, ldy, partials, (hipStream_t)stream);
}

int p8x_vec_dot_rows(const p8x_tensor *t, int act, const void *q, const float *d, int ncols, int g0, int ng, const float *x, size_t ldx,
                     float *y, size_t ldy, int32_t *partials, void *stream) {
    if (!t || !q || !y) return set_error(P8X_ERR_ARG, "p8x_vec_dot_rows: null pointer");
    if (act != P8X_ACT_Q8_128 && act != P8X_ACT_Q8_1) return set_error(P8X_ERR_ARG, "p8x_vec_dot_rows: act %d", act);
    if (act == P8X_ACT_Q8_128 && !d) return set_error(P8X_ERR_ARG, "p8x_vec_dot_rows: Q8_128 needs d");
    if (ncols < 1 || ncols > P8X_MAX_COLS || ldy < (size_t)t->rows) return set_error(P8X_ERR_ARG, "p8x_vec_dot_rows: ncols %d ldy %zu", ncols, ldy);
    if (g0 < 0 || ng < 1 || g0 + ng > t->ng) return set_error(P8X_ERR_ARG, "p8x_vec_dot_rows: row groups [%d, +%d) of %d", g0, ng, t->ng);
    if (x && ldx < (size_t)t->K) return set_error(P8X_ERR_ARG, "p8x_vec_dot_rows: ldx %zu < K %d", ldx, t->K);
    return launch_gemv_range(t, act, q, d, ncols, x, ldx, y, ldy, partials, g0, ng, (hipStream_t)stream);
}

int p8x_mul_mat_vec_act(const p8x_tensor *t, int act, const float *x, int ncols, size_t ldx, float *y, size_t ldy, void *stream) {
    if (!t || !x || !y) return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec: null pointer");
    if (ncols < 1 || ncols > P8X_MAX_COLS) return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec: ncols %d (1..%d)", ncols, P8X_MAX_COLS);
    if (ldx < (size_t)t->K || ldy < (size_t)t->rows || ldx % 4 || ((uintptr_t)x & 15))
        return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec: ldx %zu ldy %zu (x 16-byte aligned, ldx %% 4 == 0)", ldx, ldy);
    hipStream_t st = (hipStream_t)stream;
    int rc;
    if (act == P8X_ACT_Q8_128)   // one launch: every task quantizes its chunk of x itself (same arithmetic as the prep)
        return launch_gemv(t, act, nullptr, nullptr, ncols, x, ldx, y, ldy, nullptr, st);
    // x16 and, within a graph evaluation (p8x_graph_begin), block_q8_1 prepare x in a launch of their own, and a later
    // call on the same input and rotation reuses the activation the previous call prepared (CPU.patch:1171-1180);
    // outside one, block_q8_1 is quantized by the GEMV's tasks (one launch)
    bool have = false;
    if (act == P8X_ACT_Q8_1) {
        uint8_t *blk = act_reuse(t, act, x, ncols, ldx, (size_t)36 * ncols * (t->K / 32), st, &have);
        if (!blk) return launch_gemv(t, act, nullptr, nullptr, ncols, x, ldx, y, ldy, nullptr, st);
        if (!have && (rc = launch_act_q8_1(t, x, ncols, ldx, blk, st))) return rc;
        return launch_gemv(t, act, blk, nullptr, ncols, x, ldx, y, ldy, nullptr, st);
    }
    if (act == P8X_ACT_X16) {
        if (2 * ncols > P8X_MAX_COLS) return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec: x16 takes at most %d columns", P8X_MAX_COLS / 2);
        const size_t qb = ((size_t)2 * ncols * t->K + 255) & ~(size_t)255;
        uint8_t *c = act_reuse(t, act, x, ncols, ldx, qb + (size_t)8 * ncols * t->nsl, st, &have);
        if (!c) return launch_gemv_x16(t, x, ncols, ldx, y, ldy, st);
        return launch_gemv_x16_on(t, x, ncols, ldx, y, ldy, reinterpret_cast<int8_t *>(c), reinterpret_cast<float *>(c + qb), have, st);
    }
    return set_error(P8X_ERR_ARG, "p8x_mul_mat_vec: act %d", act);
}

void p8x_graph_begin(void) { act_epoch_advance(); }

int p8x_mul_mat_vec(const p8x_tensor *t, const float *x, int ncols, size_t ldx, float *y, size_t ldy, void *stream) {
    return p8x_mul_mat_vec_act(t, P8X_ACT_Q8_128, x, ncols, ldx, y, ldy, stream);
}

int p8x_mul_mat_reserve(const p8x_tensor *t, int n_max) {
    if (!t || n_max < 1) return set_error(P8X_ERR_ARG, "p8x_mul_mat_reserve: null tensor or n_max %d", n_max);
    return reserve_mul_mat(t, n_max);
}

int p8x_mul_mat(const p8x_tensor *t, const void *x, int x_dtype, int N, size_t ldx, float *y, size_t ldy, void *stream) {
    if (!t || !x || !y) return set_error(P8X_ERR_ARG, "p8x_mul_mat: null pointer");
    if (x_dtype != P8X_F32 && x_dtype != P8X_BF16) return set_error(P8X_ERR_ARG, "p8x_mul_mat: x dtype %d", x_dtype);
    if (N < 1 || ldx < (size_t)t->K || ldy < (size_t)t->rows) return set_error(P8X_ERR_ARG, "p8x_mul_mat: N %d ldx %zu ldy %zu", N, ldx, ldy);
    return launch_mul_mat(t, x, x_dtype, N, ldx, y, ldy, (hipStream_t)stream);
}

}  // extern "C"
