// p8x_loader.cpp -- native Pingala-8 model files (GGUF) to slot bytes: the host side of the reference's model
// loader for VR tensors, with status codes instead of exceptions.
//
// Restates (patches/llama_cpu_vs_7ac59a6.patch, "CPU.patch"):
//   vr_native_init (CPU.patch:4700-4800): detect vr.format, check vr.ns / vr.trl / vr.n_linear / vr.layout, find the
//     linears by their ".vr_c" side tensor, validate the side tensors' types and shapes, derive rows / K / kbytes
//     (VR3: from the file size and header word 515), pick the slot size, check vr.had_signs and the linear count;
//   vr_native_load (CPU.patch:4810-4869): assemble the in-memory slot: kernel bytes (VR3: expanded), header NS/TRL,
//     tables identical across tensors, kbytes against the M words, c16 / prm (VR3: identity) / pinv / delta / signs
//     / trailer at the top-down offsets, with the permutation, delta-index and sign checks;
//   vrn3_rows / vrn3_expand (CPU.patch:4916-4950, llama-vr3.h): the VR3 file layout.
// The GGUF container (header, key-value metadata, tensor infos, aligned data section) is read directly; ggml is
// not linked. The reference also insists on its CUDA arm's environment switches (GGML_F44 ...), which have no
// meaning here and are not checked.
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "p8x_internal.h"

namespace p8x {

// ggml tensor types used by the VR side tensors, and the six quant types the reference's loader retypes a VR
// weight into (CPU.patch:4759; bytes per 256-weight block: the slot is the smallest with rows x row size >= need)
enum { kGgmlF32 = 0, kGgmlF16 = 1, kGgmlI8 = 24, kGgmlI16 = 25 };
struct SlotType { int type; int block_bytes; };
static const SlotType kSlotTypes[] = {{16, 66}, {10, 84}, {11, 110}, {12, 144}, {13, 176}, {14, 210}};   // IQ2_XXS, Q2_K .. Q6_K

enum { kGgufU8 = 0, kGgufI8, kGgufU16, kGgufI16, kGgufU32, kGgufI32, kGgufF32, kGgufBool, kGgufStr, kGgufArr, kGgufU64, kGgufI64, kGgufF64 };

struct GgufValue {
    int type = -1;
    uint64_t u = 0;     // integer / bool values
    std::string s;      // strings
};

struct GgufTensor {
    int file = 0;
    int type = 0;
    std::vector<uint64_t> ne;
    uint64_t offset = 0;   // absolute file offset of the data
    uint64_t nbytes = 0;   // ne x element size (types with a known element size), else 0
};

static int elem_bytes(int type) {
    switch (type) {
        case kGgmlF32: return 4;
        case kGgmlF16: case kGgmlI16: return 2;
        case kGgmlI8: return 1;
        default: return 0;
    }
}

class Reader {
public:
    Reader(int fd, uint64_t size) : fd_(fd), size_(size) {}
    bool read(void *dst, uint64_t n) {
        if (n > size_ || pos_ > size_ - n) return false;
        uint8_t *d = static_cast<uint8_t *>(dst);
        uint64_t done = 0;
        while (done < n) {
            const ssize_t r = pread(fd_, d + done, (size_t)std::min<uint64_t>(n - done, 1u << 30), (off_t)(pos_ + done));
            if (r <= 0) return false;
            done += (uint64_t)r;
        }
        pos_ += n;
        return true;
    }
    template <typename T> bool get(T &v) { return read(&v, sizeof v); }
    bool str(std::string &s) {
        uint64_t n;
        if (!get(n) || n > size_ - pos_) return false;
        s.resize(n);
        return n == 0 || read(&s[0], n);
    }
    bool skip(uint64_t n) {
        if (n > size_ - pos_) return false;
        pos_ += n;
        return true;
    }
    uint64_t pos() const { return pos_; }

private:
    int fd_;
    uint64_t size_, pos_ = 0;
};

static bool scalar_bytes(int t, uint64_t *n) {
    static const int sz[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    if (t < 0 || t > 12 || t == kGgufStr || t == kGgufArr) return false;
    *n = (uint64_t)sz[t];
    return true;
}

// one GGUF key-value: scalars and strings are kept, arrays are skipped
static bool read_value(Reader &r, int type, GgufValue &v, int depth = 0) {
    v.type = type;
    if (type == kGgufStr) return r.str(v.s);
    if (type == kGgufArr) {
        uint32_t et;
        uint64_t n;
        if (depth > 2 || !r.get(et) || !r.get(n)) return false;
        if (et == kGgufStr || et == kGgufArr) {
            for (uint64_t i = 0; i < n; ++i) {
                GgufValue e;
                if (!read_value(r, (int)et, e, depth + 1)) return false;
            }
            return true;
        }
        uint64_t b;
        if (!scalar_bytes((int)et, &b) || (b && n > UINT64_MAX / b)) return false;
        return r.skip(n * b);
    }
    uint64_t b;
    if (!scalar_bytes(type, &b)) return false;
    uint64_t u = 0;
    if (!r.read(&u, b)) return false;
    v.u = u;
    return true;
}

}  // namespace p8x

using namespace p8x;

struct p8x_vr_entry {
    std::string name;            // <base>.weight
    p8x_vr_desc d;
    GgufTensor w, c, prm, didx, dval;
    bool has_prm = false, has_delta = false;
};

struct p8x_vr_file {
    std::vector<int> fds;
    std::map<std::string, GgufValue> kv;           // from the first file
    std::map<std::string, GgufTensor> tensors;     // every file
    std::vector<p8x_vr_entry> vr;
    GgufTensor signs;
    int layout = 2;
    std::mutex mu;                                 // the tables of the first tensor loaded (all must match)
    std::vector<uint8_t> hdr0;
};

namespace p8x {

static int fail(const char *fmt, const std::string &a = "", const std::string &b = "") {
    return set_error(P8X_ERR_FORMAT, fmt, a.c_str(), b.c_str());
}

// the GGUF container of one file: key-values (first file only) and tensor infos with absolute data offsets
static int parse_gguf(p8x_vr_file *F, int fi, const char *path, bool keep_kv) {
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return set_error(P8X_ERR_ARG, "p8x_vr_open: cannot open %s", path);
    F->fds.push_back(fd);
    const off_t end = lseek(fd, 0, SEEK_END);
    if (end < 0) return set_error(P8X_ERR_ARG, "p8x_vr_open: cannot size %s", path);
    Reader r(fd, (uint64_t)end);
    uint32_t magic, version;
    uint64_t nt, nkv;
    if (!r.get(magic) || magic != 0x46554747u) return set_error(P8X_ERR_FORMAT, "p8x_vr_open: %s is not a GGUF file", path);
    if (!r.get(version) || version < 2 || version > 3) return set_error(P8X_ERR_FORMAT, "p8x_vr_open: %s: GGUF version %u (2 or 3)", path, version);
    if (!r.get(nt) || !r.get(nkv) || nt > (uint64_t)end || nkv > (uint64_t)end)
        return set_error(P8X_ERR_FORMAT, "p8x_vr_open: %s: bad GGUF counts", path);
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < nkv; ++i) {
        std::string key;
        uint32_t type;
        GgufValue v;
        if (!r.str(key) || !r.get(type) || !read_value(r, (int)type, v)) return set_error(P8X_ERR_FORMAT, "p8x_vr_open: %s: bad key-value %llu", path, (unsigned long long)i);
        if (key == "general.alignment" && type == kGgufU32) alignment = v.u;
        if (keep_kv) F->kv[key] = v;
    }
    if (alignment == 0 || (alignment & (alignment - 1))) return set_error(P8X_ERR_FORMAT, "p8x_vr_open: %s: alignment %llu", path, (unsigned long long)alignment);
    std::vector<std::pair<std::string, GgufTensor>> infos;
    for (uint64_t i = 0; i < nt; ++i) {
        std::string name;
        uint32_t nd, type;
        GgufTensor t;
        t.file = fi;
        if (!r.str(name) || !r.get(nd) || nd == 0 || nd > 4) return set_error(P8X_ERR_FORMAT, "p8x_vr_open: %s: bad tensor info %llu", path, (unsigned long long)i);
        t.ne.resize(nd);
        for (uint32_t d = 0; d < nd; ++d)
            if (!r.get(t.ne[d])) return set_error(P8X_ERR_FORMAT, "p8x_vr_open: %s: bad tensor info %llu", path, (unsigned long long)i);
        if (!r.get(type) || !r.get(t.offset)) return set_error(P8X_ERR_FORMAT, "p8x_vr_open: %s: bad tensor info %llu", path, (unsigned long long)i);
        t.type = (int)type;
        infos.emplace_back(name, t);
    }
    const uint64_t data = (r.pos() + alignment - 1) / alignment * alignment;
    for (auto &it : infos) {
        GgufTensor &t = it.second;
        if (t.offset > UINT64_MAX - data) return fail("p8x_vr_open: tensor '%s' has a data offset past any file", it.first);
        t.offset += data;
        const int eb = elem_bytes(t.type);
        if (eb) {
            uint64_t n = (uint64_t)eb;
            for (uint64_t e : t.ne) {
                if (e && n > UINT64_MAX / e) return fail("p8x_vr_open: tensor '%s' is too large", it.first);
                n *= e;
            }
            t.nbytes = n;
            if (t.offset > (uint64_t)end || n > (uint64_t)end - t.offset) return fail("p8x_vr_open: tensor '%s' lies beyond the end of its file", it.first);
        }
        if (F->tensors.count(it.first)) return fail("p8x_vr_open: tensor '%s' appears twice", it.first);
        F->tensors[it.first] = t;
    }
    return P8X_OK;
}

static int read_at(const p8x_vr_file *F, const GgufTensor &t, uint64_t off, void *dst, uint64_t n) {
    uint8_t *d = static_cast<uint8_t *>(dst);
    uint64_t done = 0;
    while (done < n) {
        const ssize_t r = pread(F->fds[t.file], d + done, (size_t)std::min<uint64_t>(n - done, 1u << 30), (off_t)(t.offset + off + done));
        if (r <= 0) return set_error(P8X_ERR_FORMAT, "p8x_vr: short read");
        done += (uint64_t)r;
    }
    return P8X_OK;
}

static const GgufValue *kv_u32(const p8x_vr_file *F, const char *key) {
    const auto it = F->kv.find(key);
    return it != F->kv.end() && it->second.type == kGgufU32 ? &it->second : nullptr;
}

static bool ends_with(const std::string &s, const char *suf) {
    const size_t n = strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

static size_t kernel_bytes(size_t rows, size_t K, size_t payload_words) {   // vrn_kbytes (CPU.patch:47-50)
    return offset_D((rows / 32) * (K / 256)) + 4 * payload_words;
}

static size_t nw_of_class(uint32_t c) { return (size_t)nw_of((int)(c & 7u)); }

}  // namespace p8x

extern "C" {

size_t p8x_vr3_rows(size_t fbytes, size_t K, uint32_t w515, size_t *kbytes) {
    if ((w515 & 0xFFFFFFF8u) != P8X_VR3_TAG || (w515 & 7u) == 0 || K == 0 || K % 256 || fbytes < kHeaderBytes) return 0;
    const size_t tw = 64 * nw_of_class(w515), per = 64 + 4 * tw, nb = K / 256;
    if ((fbytes - kHeaderBytes) % per) return 0;
    const size_t nt = (fbytes - kHeaderBytes) / per;
    if (nt == 0 || nt % nb || nt * tw >= ((size_t)1 << 29)) return 0;
    const size_t rows = 32 * (nt / nb);
    if (rows >= 32768) return 0;
    if (kbytes) *kbytes = kernel_bytes(rows, K, nt * tw);
    return rows;
}

int p8x_vr3_expand(const void *file_bytes, size_t fbytes, size_t rows, size_t K, void *dst, size_t cap) {
    if (!file_bytes || !dst || fbytes < kHeaderBytes) return set_error(P8X_ERR_ARG, "p8x_vr3_expand: bad arguments");
    const uint8_t *f = static_cast<const uint8_t *>(file_bytes);
    uint8_t *d = static_cast<uint8_t *>(dst);
    uint32_t w515;
    memcpy(&w515, f + 2060, 4);
    size_t kb = 0;
    if (p8x_vr3_rows(fbytes, K, w515, &kb) != rows || rows == 0) return set_error(P8X_ERR_FORMAT, "p8x_vr3_expand: not a VR3 tensor of %zu rows", rows);
    if (cap < kb) return set_error(P8X_ERR_ARG, "p8x_vr3_expand: %zu bytes needed, %zu given", kb, cap);
    // header without word 515 (the value a layout-2 file carries is 0), arithmetic M words (tile i at i x 64 NW words,
    // one class), the scales, zero pad to the 16-byte payload start, the payload
    const uint32_t c = w515 & 7u;
    const size_t nt = (rows / 32) * (K / 256), tw = 64 * nw_of_class(c), offD = offset_D(nt);
    memcpy(d, f, 2060);
    memset(d + 2060, 0, 4);
    for (size_t i = 0; i < nt; ++i) {
        const uint32_t m = (uint32_t)(i * tw) | (c << 29);
        memcpy(d + kHeaderBytes + 4 * i, &m, 4);
    }
    memcpy(d + kHeaderBytes + 4 * nt, f + kHeaderBytes, 64 * nt);
    memset(d + kHeaderBytes + 68 * nt, 0, offD - (kHeaderBytes + 68 * nt));
    memcpy(d + offD, f + kHeaderBytes + 64 * nt, fbytes - kHeaderBytes - 64 * nt);
    return P8X_OK;
}

void p8x_vr_close(p8x_vr_file *F) {
    if (!F) return;
    for (int fd : F->fds) close(fd);
    delete F;
}

int p8x_vr_open(const char *const *paths, int npaths, p8x_vr_file **out) {
    if (!paths || npaths < 1 || !out) return set_error(P8X_ERR_ARG, "p8x_vr_open: bad arguments");
    *out = nullptr;
    p8x_vr_file *F = new p8x_vr_file();
    auto bail = [&](int rc) { p8x_vr_close(F); return rc; };
    int rc;
    for (int i = 0; i < npaths; ++i)
        if (!paths[i] || (rc = parse_gguf(F, i, paths[i], i == 0))) return bail(rc ? rc : set_error(P8X_ERR_ARG, "p8x_vr_open: null path"));
    if (!F->kv.count("vr.format")) return bail(set_error(P8X_ERR_FORMAT, "p8x_vr_open: the file has no vr.format entry, so it is not a Pingala-8 model"));
    const GgufValue *ns = kv_u32(F, "vr.ns");
    if (!ns) return bail(set_error(P8X_ERR_FORMAT, "p8x_vr_open: the uint32 entry vr.ns is absent (this library reads files with 108 trellis states)"));
    if (ns->u != kNS) return bail(set_error(P8X_ERR_FORMAT, "p8x_vr_open: the file declares %llu trellis states; this library decodes %u only", (unsigned long long)ns->u, kNS));
    const GgufValue *trl = kv_u32(F, "vr.trl"), *nlin = kv_u32(F, "vr.n_linear");
    if (!trl || trl->u != kTRL || !nlin) return bail(set_error(P8X_ERR_FORMAT, "p8x_vr_open: expected entries vr.trl == 2 and vr.n_linear"));
    {
        const auto it = F->kv.find("vr.layout");
        if (it != F->kv.end() && it->second.type != kGgufU32) return bail(set_error(P8X_ERR_FORMAT, "p8x_vr_open: the entry vr.layout has a type other than uint32"));
        F->layout = it == F->kv.end() ? 2 : (int)it->second.u;
        if (F->layout != 2 && F->layout != 3) return bail(set_error(P8X_ERR_FORMAT, "p8x_vr_open: unknown side-data layout %d (this library reads 2 and 3)", F->layout));
    }
    long long n_layer = -1;
    {
        const auto a = F->kv.find("general.architecture");
        if (a != F->kv.end() && a->second.type == kGgufStr) {
            const GgufValue *bc = kv_u32(F, (a->second.s + ".block_count").c_str());
            if (bc) n_layer = (long long)bc->u;
        }
    }
    auto find = [&](const std::string &n) -> const GgufTensor * {
        const auto it = F->tensors.find(n);
        return it == F->tensors.end() ? nullptr : &it->second;
    };
    for (const auto &it : F->tensors) {
        if (!ends_with(it.first, ".vr_c")) continue;
        const std::string base = it.first.substr(0, it.first.size() - 5);
        p8x_vr_entry e;
        e.name = base + ".weight";
        const GgufTensor *w = find(e.name);
        if (!w) return bail(fail("p8x_vr_open: '%s': a vr_c tensor without its weight tensor", base));
        if (w->type != kGgmlI8 || w->ne.size() != 1) return bail(fail("p8x_vr_open: '%s': the weight bytes must be a one-dimensional I8 tensor", e.name));
        e.w = *w;
        e.c = it.second;
        if (e.c.type != kGgmlF16) return bail(fail("p8x_vr_open: '%s': vr_c is not F16", base));
        p8x_vr_desc &d = e.d;
        memset(&d, 0, sizeof d);
        d.layout = F->layout;
        d.K = (int)std::min<uint64_t>(e.c.ne[0], 1u << 30);
        d.fbytes = (size_t)w->ne[0];
        if (F->layout == 2) {
            const GgufTensor *p = find(base + ".vr_prm");
            if (!p || p->type != kGgmlI16) return bail(fail("p8x_vr_open: '%s': vr_c must be F16 and vr_prm I16", base));
            e.prm = *p;
            e.has_prm = true;
            d.rows = (int)std::min<uint64_t>(p->ne[0], 1u << 30);
            d.kbytes = d.fbytes;
        } else {   // VR3: rows from the file size, K and header word 515; identity permutation, no vr_prm tensor
            if (find(base + ".vr_prm")) return bail(fail("p8x_vr_open: '%s': layout 3 keeps the row order inside the weight, yet a vr_prm tensor is present", base));
            uint32_t w515 = 0;
            if (d.fbytes >= kHeaderBytes && (rc = read_at(F, e.w, 2060, &w515, 4))) return bail(rc);
            d.rows = (int)p8x_vr3_rows(d.fbytes, (size_t)d.K, w515, &d.kbytes);
            if (d.rows == 0)
                return bail(set_error(P8X_ERR_FORMAT, "p8x_vr_open: '%s': not a layout-3 weight (%zu bytes, K %d, header word 515 = 0x%08x)", e.name.c_str(), d.fbytes, d.K, w515));
        }
        if (d.K % 256 || d.K <= 0 || d.rows % 32 || d.rows <= 0 || d.rows >= 32768)
            return bail(set_error(P8X_ERR_FORMAT, "p8x_vr_open: '%s': shape K %d x rows %d is outside the format (K %% 256, rows %% 32, rows < 32768)", base.c_str(), d.K, d.rows));
        const GgufTensor *di = find(base + ".vr_didx"), *dv = find(base + ".vr_dval");
        if (!di != !dv) return bail(fail("p8x_vr_open: '%s': clamp-delta tensors come in pairs (vr_didx with vr_dval)", base));
        if (di) {
            if (di->type != kGgmlI16 || dv->type != kGgmlF32 || di->ne.size() < 2 || di->ne[0] != dv->ne[0] || di->ne[1] != 2)
                return bail(fail("p8x_vr_open: '%s': clamp-delta tensors must be vr_didx I16 [n][2] and vr_dval F32 [n]", base));
            if (dv->ne[0] >= (1u << 30)) return bail(fail("p8x_vr_open: '%s' too many delta entries", base));
            e.didx = *di;
            e.dval = *dv;
            e.has_delta = true;
            d.nd = (int)dv->ne[0];
        }
        const size_t need = p8x_need(d.kbytes, d.rows, d.K, d.nd);
        for (const SlotType &st : kSlotTypes)
            if ((size_t)(d.K / 256) * st.block_bytes * d.rows >= need) {
                d.slot_type = st.type;
                d.slot_bytes = (size_t)(d.K / 256) * st.block_bytes * d.rows;
                break;
            }
        if (!d.slot_bytes) return bail(set_error(P8X_ERR_FORMAT, "p8x_vr_open: '%s': %zu bytes exceed every slot size", e.name.c_str(), need));
        F->vr.push_back(std::move(e));
    }
    const GgufTensor *sg = find("vr.had_signs");
    if (!sg || sg->type != kGgmlI8 || sg->ne[0] != 256) return bail(set_error(P8X_ERR_FORMAT, "p8x_vr_open: the rotation signs (vr.had_signs) must be 256 I8 values"));
    F->signs = *sg;
    if (F->vr.size() != nlin->u || (long long)nlin->u != 7 * n_layer)
        return bail(set_error(P8X_ERR_FORMAT, "p8x_vr_open: found %zu weight tensors; vr.n_linear says %llu and 7 per layer over %lld layers are expected", F->vr.size(), (unsigned long long)nlin->u, n_layer));
    for (auto &e : F->vr) e.d.name = e.name.c_str();
    *out = F;
    return P8X_OK;
}

int p8x_vr_count(const p8x_vr_file *F) { return F ? (int)F->vr.size() : 0; }

int p8x_vr_find(const p8x_vr_file *F, const char *name) {
    if (!F || !name) return -1;
    for (size_t i = 0; i < F->vr.size(); ++i)
        if (F->vr[i].name == name) return (int)i;
    return -1;
}

int p8x_vr_describe(const p8x_vr_file *F, int i, p8x_vr_desc *out) {
    if (!F || !out || i < 0 || i >= (int)F->vr.size()) return set_error(P8X_ERR_ARG, "p8x_vr_describe: bad arguments");
    *out = F->vr[i].d;
    return P8X_OK;
}

int p8x_vr_load(p8x_vr_file *F, int i, void *slot, size_t cap) {
    if (!F || !slot || i < 0 || i >= (int)F->vr.size()) return set_error(P8X_ERR_ARG, "p8x_vr_load: bad arguments");
    const p8x_vr_entry &e = F->vr[i];
    const p8x_vr_desc &d = e.d;
    const size_t n = d.slot_bytes;
    if (cap < n) return set_error(P8X_ERR_ARG, "p8x_vr_load: '%s' needs %zu bytes, %zu given", d.name, n, cap);
    uint8_t *buf = static_cast<uint8_t *>(slot);
    memset(buf, 0, n);
    int rc;
    if (d.layout == 2) {
        if ((rc = read_at(F, e.w, 0, buf, d.kbytes))) return rc;
    } else {   // VR3 file bytes expanded to the layout-2 kernel bytes
        std::vector<uint8_t> f3(d.fbytes);
        if ((rc = read_at(F, e.w, 0, f3.data(), d.fbytes))) return rc;
        uint32_t w515;
        memcpy(&w515, f3.data() + 2060, 4);
        size_t kb = 0;
        if (p8x_vr3_rows(d.fbytes, (size_t)d.K, w515, &kb) != (size_t)d.rows || kb != d.kbytes || d.kbytes > n)
            return set_error(P8X_ERR_FORMAT, "p8x_vr_load: '%s': the layout-3 header differs from what p8x_vr_open read", d.name);
        if ((rc = p8x_vr3_expand(f3.data(), d.fbytes, d.rows, d.K, buf, n))) return rc;
    }
    const uint32_t *hw = reinterpret_cast<const uint32_t *>(buf);
    if (d.kbytes < kHeaderBytes || hw[513] != kNS || hw[514] != kTRL)
        return set_error(P8X_ERR_FORMAT, "p8x_vr_load: '%s': header declares %u states and trellis rate %u; this library needs %u and %u", d.name, d.kbytes >= kHeaderBytes ? hw[513] : 0u,
                         d.kbytes >= kHeaderBytes ? hw[514] : 0u, kNS, kTRL);
    {
        std::lock_guard<std::mutex> lk(F->mu);
        if (F->hdr0.empty()) F->hdr0.assign(buf, buf + 2052);
        else if (memcmp(F->hdr0.data(), buf, 2052) != 0) return set_error(P8X_ERR_FORMAT, "p8x_vr_load: '%s': its codebook tables are not those of the first weight (one codebook per file)", d.name);
    }
    const size_t nt = (size_t)(d.rows / 32) * (d.K / 256);
    if (kHeaderBytes + 4 * nt > d.kbytes) return set_error(P8X_ERR_FORMAT, "p8x_vr_load: '%s': the tile-word table runs past the weight bytes", d.name);
    size_t words = 0;
    for (size_t t = 0; t < nt; ++t) {
        uint32_t m;
        memcpy(&m, buf + kHeaderBytes + 4 * t, 4);
        words += 64 * nw_of_class(m >> 29);
    }
    if (kernel_bytes(d.rows, d.K, words) != d.kbytes)
        return set_error(P8X_ERR_FORMAT, "p8x_vr_load: '%s': %zu weight bytes, but the tile words describe %zu", d.name, d.kbytes, kernel_bytes(d.rows, d.K, words));
    size_t off[6];   // delta, c16, prm, pinv, signs, trailer
    side_offsets(n, (size_t)d.rows, (size_t)d.K, (size_t)d.nd, off);
    if (d.kbytes > off[0]) return set_error(P8X_ERR_FORMAT, "p8x_vr_load: '%s': the weight bytes run into the side data", d.name);
    if ((rc = read_at(F, e.c, 0, buf + off[1], 2 * (size_t)d.K))) return rc;
    int16_t *p = reinterpret_cast<int16_t *>(buf + off[2]);
    if (e.has_prm) {
        if ((rc = read_at(F, e.prm, 0, p, 2 * (size_t)d.rows))) return rc;
    } else {
        for (int r = 0; r < d.rows; ++r) p[r] = (int16_t)r;   // VR3: natural rows
    }
    {   // prm must be a permutation of 0..rows-1; pinv = its inverse
        std::vector<uint8_t> seen(d.rows, 0);
        for (int r = 0; r < d.rows; ++r)
            if (p[r] < 0 || p[r] >= d.rows || seen[p[r]]++) return set_error(P8X_ERR_FORMAT, "p8x_vr_load: '%s': the row order repeats or skips a row", d.name);
        int16_t *q = reinterpret_cast<int16_t *>(buf + off[3]);
        for (int r = 0; r < d.rows; ++r) q[p[r]] = (int16_t)r;
    }
    if (d.nd > 0) {   // vr_didx I16 [nd, 2]: original rows then original cols (u16); vr_dval F32 [nd]
        if ((rc = read_at(F, e.didx, 0, buf + off[0], 4 * (size_t)d.nd))) return rc;
        if ((rc = read_at(F, e.dval, 0, buf + off[0] + 4 * (size_t)d.nd, 4 * (size_t)d.nd))) return rc;
        const uint16_t *dr = reinterpret_cast<const uint16_t *>(buf + off[0]), *dc = dr + d.nd;
        for (int k = 0; k < d.nd; ++k)
            if (dr[k] >= d.rows || dc[k] >= d.K) return set_error(P8X_ERR_FORMAT, "p8x_vr_load: '%s': a clamp-delta entry points outside the matrix", d.name);
    }
    if ((rc = read_at(F, F->signs, 0, buf + off[4], 256))) return rc;
    for (int k = 0; k < 256; ++k) {
        const int8_t v = (int8_t)buf[off[4] + k];
        if (v != 1 && v != -1) return set_error(P8X_ERR_FORMAT, "p8x_vr_load: a rotation sign other than +1 or -1");
    }
    const uint32_t tr[8] = {kMagic0, kMagic1, (uint32_t)d.kbytes, (uint32_t)d.nd, (uint32_t)d.rows, (uint32_t)d.K, kNS, 1u};
    memcpy(buf + off[5], tr, sizeof tr);
    return P8X_OK;
}

}  // extern "C"
