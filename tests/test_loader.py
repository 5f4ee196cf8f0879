"""Native model files (GGUF, vr.layout 2 and 3) to slot bytes: p8x_vr_open / p8x_vr_load / p8x_vr3_* against the
layout the reference's loader builds (llama_model_loader::vr_native_init / vr_native_load, CPU.patch:4700-4869;
llama-vr3.h, CPU.patch:4916-4950), on files written by tests/gguf_writer.py. CPU only, except the last test.

The VR3 checks restate the reference's own C test (research/detail/b3p_vr3_test.c): the expansion of a VR3 file
tensor equals the layout-2 bytes of the same natural-order tensor with every output byte written (the destination
prefilled), and three malformed inputs are rejected (size off by 4, wrong tag, class 0)."""
import os

import numpy as np
import pytest

import gguf_writer as G
import p8x
import slotgen

SLOT_BLOCKS = [(16, 66), (10, 84), (11, 110), (12, 144), (13, 176), (14, 210)]   # IQ2_XXS, Q2_K .. Q6_K per 256 weights
LAYER = [("attn_q", 128, 512), ("attn_k", 32, 512), ("attn_v", 32, 512), ("attn_output", 128, 512),
         ("ffn_gate", 256, 512), ("ffn_up", 256, 512), ("ffn_down", 128, 1024)]


def slot_size(kbytes, rows, K, nd):
    """the reference loader's slot: the smallest quant type whose tensor holds the need (None, need if none does:
    tiny tensors of the widest classes, which the loader rejects)"""
    need = slotgen.need(kbytes, rows, K, nd)
    for t, bb in SLOT_BLOCKS:
        if K // 256 * bb * rows >= need:
            return t, K // 256 * bb * rows
    return None, need


class Linear:
    """one linear: its parts and the in-memory slot the reference's loader would build"""

    def __init__(self, rng, rows, K, A, cs, sg, natural, cls=None, nd=0):
        ng, nb = rows // 32, K // 256
        self.rows, self.K, self.nd = rows, K, nd
        self.cls = np.full((ng, nb), cls, np.int64) if cls else rng.choice([1, 2, 3, 4, 5], size=(ng, nb))
        nwords = int(sum(64 * slotgen.NW[c] for c in self.cls.reshape(-1)))
        self.payload = rng.integers(0, 1 << 32, size=nwords, dtype=np.uint64).astype(np.uint32)
        self.S = rng.uniform(2e-4, 3e-4, size=(nb, rows)).astype(np.float16).view(np.uint16)
        self.c16 = rng.uniform(0.5, 2.0, size=K).astype(np.float16).view(np.uint16)
        self.prm = np.arange(rows, dtype=np.int16) if natural else rng.permutation(rows).astype(np.int16)
        flat = np.sort(rng.choice(rows * K, size=nd, replace=False)) if nd else np.zeros(0, np.int64)
        self.drow, self.dcol = (flat // K).astype(np.uint16), (flat % K).astype(np.uint16)
        self.dval = rng.uniform(-0.05, 0.05, size=nd).astype(np.float32)
        nt = ng * nb
        self.kbytes = slotgen.a16(2064 + 68 * nt) + 4 * nwords
        self.slot_type, self.slot_bytes = slot_size(self.kbytes, rows, K, nd)
        extra = self.slot_bytes - slotgen.need(self.kbytes, rows, K, nd)
        d = (self.drow, self.dcol, self.dval) if nd else (None, None, None)
        self.slot = slotgen.build_slot(A, cs, self.cls, self.payload, self.S, self.c16, self.prm, sg, *d, extra=extra)
        assert self.slot.size == self.slot_bytes

    def vr3_bytes(self):
        """the VR3 file tensor: header (2060 B) | tag | class, the scales, the payload"""
        nt = self.cls.size
        f = np.concatenate([self.slot[:2060], np.array([p8x.VR3_TAG | int(self.cls.flat[0])], np.uint32).view(np.uint8),
                            self.slot[2064 + 4 * nt:2064 + 68 * nt], self.payload.view(np.uint8)])
        return f


def tensors_of(base, lin, layout, with_prm=None):
    out = [(base + ".weight", G.GGML_I8, [lin.kbytes if layout == 2 else lin.vr3_bytes().size],
            lin.slot[:lin.kbytes] if layout == 2 else lin.vr3_bytes()),
           (base + ".vr_c", G.GGML_F16, [lin.K], G.as_bytes(lin.c16))]
    if (layout == 2) if with_prm is None else with_prm:
        out.append((base + ".vr_prm", G.GGML_I16, [lin.rows], G.as_bytes(lin.prm)))
    if lin.nd:
        out.append((base + ".vr_didx", G.GGML_I16, [lin.nd, 2], G.as_bytes(np.concatenate([lin.drow, lin.dcol]))))
        out.append((base + ".vr_dval", G.GGML_F32, [lin.nd], G.as_bytes(lin.dval)))
    return out


def model(tmp_path, layout=2, seed=0, kv_edit=None, tensor_edit=None, name="m.gguf"):
    """a one-layer model file: 7 linears, an unrelated F32 tensor, the signs and the VR metadata"""
    rng = np.random.default_rng(seed)
    A, cs = slotgen.shipped_tables()
    sg = np.where(rng.integers(0, 2, 256) == 1, 1, -1).astype(np.int8)
    lins = {}
    for i, (kind, rows, K) in enumerate(LAYER):
        lins[f"blk.0.{kind}"] = Linear(rng, rows, K, A, cs, sg, natural=layout == 3, cls=3 if layout == 3 and i % 2 else
                                       (6 if layout == 3 else None), nd=(0, 3, 1, 0, 5, 2, 4)[i])
    kvs = [("general.architecture", G.STR, "llama"), ("llama.block_count", G.U32, 1),
           ("vr.format", G.STR, "VRii-C Pingala-8 (test)"), ("vr.ns", G.U32, 108), ("vr.trl", G.U32, 2),
           ("vr.n_linear", G.U32, 7), ("tokenizer.ggml.tokens", G.ARR, (G.STR, ["a", "bc"]))]
    if layout == 3:
        kvs.append(("vr.layout", G.U32, 3))
    tensors = [("token_embd.weight", G.GGML_F32, [16, 4], G.as_bytes(rng.standard_normal(64).astype(np.float32)))]
    for base, lin in lins.items():
        tensors += tensors_of(base, lin, layout)
    tensors.append(("vr.had_signs", G.GGML_I8, [256], G.as_bytes(sg)))
    if kv_edit:
        kvs = kv_edit(kvs)
    if tensor_edit:
        tensors = tensor_edit(tensors)
    path = os.path.join(tmp_path, name)
    G.write(path, kvs, tensors)
    return path, lins


@pytest.mark.parametrize("c", [1, 2, 3, 4, 5, 6, 7])
def test_vr3_expand_like_reference_test(c):
    rng = np.random.default_rng(c)
    A, cs = slotgen.shipped_tables()
    sg = np.ones(256, np.int8)
    for rows, K in ((32, 256), (96, 1024)):
        lin = Linear(rng, rows, K, A, cs, sg, natural=True, cls=c)
        f = lin.vr3_bytes()
        w515 = int(f[2060:2064].view(np.uint32)[0])
        r, kb = p8x.vr3_rows(f.size, K, w515)
        assert (r, kb) == (rows, lin.kbytes)
        for fill in (0xA5, 0x5A):   # every output byte written: two different prefills give the same bytes
            d = np.full(kb, fill, np.uint8)
            p8x.vr3_expand(f, rows, K, d)
            assert np.array_equal(d, lin.slot[:kb]), (c, rows, K, fill)
        # negative cases of the reference test: size off by 4, wrong tag, class 0
        assert p8x.vr3_rows(f.size - 4, K, w515)[0] == 0
        assert p8x.vr3_rows(f.size, K, w515 ^ 0x100)[0] == 0
        assert p8x.vr3_rows(f.size, K, w515 & ~7)[0] == 0


@pytest.mark.parametrize("layout", [2, 3])
def test_load_matches_reference_slot(tmp_path, layout):
    path, lins = model(tmp_path, layout)
    f = p8x.VrFile(path)
    assert len(f) == 7
    for base, lin in lins.items():
        i = f.find(base + ".weight")
        assert i >= 0
        d = f.describe(i)
        assert (d["rows"], d["K"], d["nd"], d["layout"], d["kbytes"]) == (lin.rows, lin.K, lin.nd, layout, lin.kbytes)
        assert (d["slot_type"], d["slot_bytes"]) == (lin.slot_type, lin.slot_bytes)
        assert np.array_equal(f.load(i), lin.slot), base
        assert p8x.lib().p8x_probe(lin.slot.ctypes.data, lin.slot.size, lin.rows, lin.K) == 1
    assert f.find("token_embd.weight") == -1
    f.close()


def test_load_from_shards(tmp_path):
    """the side tensors in a second file (metadata from the first)"""
    path, lins = model(tmp_path, 2)
    rng = np.random.default_rng(0)
    kvs = [("general.architecture", G.STR, "llama"), ("llama.block_count", G.U32, 1), ("vr.format", G.STR, "x"),
           ("vr.ns", G.U32, 108), ("vr.trl", G.U32, 2), ("vr.n_linear", G.U32, 7)]
    A, cs = slotgen.shipped_tables()
    sg = np.where(rng.integers(0, 2, 256) == 1, 1, -1).astype(np.int8)
    main, side = [], []
    for base, lin in lins.items():
        ts = tensors_of(base, lin, 2)
        main.append(ts[0])
        side += ts[1:]
    side.append(("vr.had_signs", G.GGML_I8, [256], G.as_bytes(np.frombuffer(lins["blk.0.attn_q"].slot[-288:-32].tobytes(), np.int8))))
    p1, p2 = os.path.join(tmp_path, "s1.gguf"), os.path.join(tmp_path, "s2.gguf")
    G.write(p1, kvs, main)
    G.write(p2, [("split.no", G.U16, 1)], side)
    f = p8x.VrFile([p1, p2])
    for base, lin in lins.items():
        assert np.array_equal(f.load(f.find(base + ".weight")), lin.slot)


def _drop(name):
    return lambda ts: [t for t in ts if t[0] != name]


def _kv_set(key, t, v):
    return lambda kvs: [k for k in kvs if k[0] != key] + ([(key, t, v)] if v is not None else [])


OPEN_ERRORS = [
    ("no vr.format", dict(kv_edit=_kv_set("vr.format", G.STR, None)), "vr.format"),
    ("no vr.ns", dict(kv_edit=_kv_set("vr.ns", G.U32, None)), "vr.ns"),
    ("vr.ns 100", dict(kv_edit=_kv_set("vr.ns", G.U32, 100)), "declares 100 trellis states"),
    ("vr.trl 3", dict(kv_edit=_kv_set("vr.trl", G.U32, 3)), "vr.trl == 2"),
    ("vr.layout 4", dict(kv_edit=_kv_set("vr.layout", G.U32, 4)), "unknown side-data layout 4"),
    ("vr.layout string", dict(kv_edit=_kv_set("vr.layout", G.STR, "3")), "vr.layout has a type other than uint32"),
    ("n_linear 6", dict(kv_edit=_kv_set("vr.n_linear", G.U32, 6)), "over 1 layers"),
    ("no block_count", dict(kv_edit=_kv_set("llama.block_count", G.U32, None)), "over -1 layers"),
    ("no vr_prm", dict(tensor_edit=_drop("blk.0.attn_q.vr_prm")), "vr_prm I16"),
    ("no weight", dict(tensor_edit=_drop("blk.0.attn_k.weight")), "vr_c tensor without its weight"),
    ("didx without dval", dict(tensor_edit=_drop("blk.0.ffn_gate.vr_dval")), "come in pairs"),
    ("no signs", dict(tensor_edit=_drop("vr.had_signs")), "had_signs"),
    ("weight F16", dict(tensor_edit=lambda ts: [(n, G.GGML_F16 if n == "blk.0.attn_v.weight" else t, [ne[0] // 2] if n == "blk.0.attn_v.weight" else ne, r)
                                                  for n, t, ne, r in ts]), "one-dimensional I8"),
]


@pytest.mark.parametrize("what,edit,msg", OPEN_ERRORS, ids=[e[0] for e in OPEN_ERRORS])
def test_open_rejects(tmp_path, what, edit, msg):
    path, _ = model(tmp_path, 2, **edit)
    with pytest.raises(p8x.P8xError, match=msg):
        p8x.VrFile(path)


def test_open_rejects_vr3_specific(tmp_path):
    def add_prm(ts):
        return ts + [("blk.0.attn_q.vr_prm", G.GGML_I16, [128], G.as_bytes(np.arange(128, dtype=np.int16)))]
    path, _ = model(tmp_path, 3, tensor_edit=add_prm)
    with pytest.raises(p8x.P8xError, match="a vr_prm tensor is present"):
        p8x.VrFile(path)

    def shorten(ts):
        return [(n, t, [ne[0] - 4] if n == "blk.0.attn_q.weight" else ne, r[:-4] if n == "blk.0.attn_q.weight" else r) for n, t, ne, r in ts]
    path, _ = model(tmp_path, 3, tensor_edit=shorten)
    with pytest.raises(p8x.P8xError, match="not a layout-3 weight"):
        p8x.VrFile(path)


def _edit_tensor(name, fn):
    return lambda ts: [(n, t, ne, fn(np.frombuffer(bytes(r), np.uint8).copy()).tobytes() if n == name else r) for n, t, ne, r in ts]


def _bad_prm(b):
    v = b.view(np.int16)
    v[1] = v[0]
    return b


def _bad_didx(b):
    v = b.view(np.uint16)
    v[0] = 60000
    return b


def _bad_sign(b):
    b[7] = 0
    return b


def _bad_tables(b):
    b[100] ^= 1   # a byte of A
    return b


def _bad_ns(b):
    b[2052] = 104
    return b


def _bad_class(b):
    b[2064 + 3] ^= 0x20   # class bits of tile 0's M word: the M-implied size changes
    return b


LOAD_ERRORS = [
    ("prm duplicate", "blk.0.attn_q.vr_prm", _bad_prm, "blk.0.attn_q.weight", "repeats or skips a row"),
    ("delta row out of range", "blk.0.attn_k.vr_didx", _bad_didx, "blk.0.attn_k.weight", "points outside the matrix"),
    ("sign zero", "vr.had_signs", _bad_sign, "blk.0.attn_q.weight", "rotation sign other than"),
    ("header NS", "blk.0.attn_q.weight", _bad_ns, "blk.0.attn_q.weight", "declares 104 states"),
    ("M class", "blk.0.attn_q.weight", _bad_class, "blk.0.attn_q.weight", "tile words describe"),
]


@pytest.mark.parametrize("what,tname,fn,load,msg", LOAD_ERRORS, ids=[e[0] for e in LOAD_ERRORS])
def test_load_rejects(tmp_path, what, tname, fn, load, msg):
    path, _ = model(tmp_path, 2, tensor_edit=_edit_tensor(tname, fn))
    f = p8x.VrFile(path)
    with pytest.raises(p8x.P8xError, match=msg):
        f.load(f.find(load))


def test_load_rejects_different_tables(tmp_path):
    """every tensor must carry the first loaded tensor's codebook tables"""
    path, _ = model(tmp_path, 2, tensor_edit=_edit_tensor("blk.0.attn_k.weight", _bad_tables))
    f = p8x.VrFile(path)
    f.load(f.find("blk.0.attn_q.weight"))
    with pytest.raises(p8x.P8xError, match="codebook tables"):
        f.load(f.find("blk.0.attn_k.weight"))


def test_load_rejects_short_buffer(tmp_path):
    path, lins = model(tmp_path, 2)
    f = p8x.VrFile(path)
    buf = np.empty(16, np.uint8)
    assert p8x.lib().p8x_vr_load(f.h, 0, buf.ctypes.data, buf.size) == p8x.P8X_ERR_ARG


@pytest.mark.gpu
@pytest.mark.parametrize("layout", [2, 3])
def test_loaded_model_on_gpu(tmp_path, layout):
    """file -> slot -> p8x_prepare -> GEMV and dequantize against the oracle of the same slot"""
    import oracle as O
    path, lins = model(tmp_path, layout, seed=5)
    f = p8x.VrFile(path)
    rng = np.random.default_rng(5)
    for base, lin in lins.items():
        slot = f.load(f.find(base + ".weight"))
        t = p8x.Tensor(slot, lin.rows, lin.K)
        orc = O.Oracle(slot, lin.rows, lin.K)
        x = rng.standard_normal(lin.K).astype(np.float32)
        y = t.mul_mat_vec(x)[0]
        ref = orc.gemv_f64(x)
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-5, base
        assert np.array_equal(t.dequantize(p8x.F32).view(np.uint32), orc.dequant().view(np.uint32)), base


def test_open_rejects_tensor_no_slot_fits(tmp_path):
    """a 32 x 256 class-7 VR3 tensor needs more bytes than a Q6_K tensor of its shape holds (the 2 KB header):
    the reference's loader has no slot type for it"""
    def tiny(ts):
        rng = np.random.default_rng(1)
        A, cs = slotgen.shipped_tables()
        lin = Linear(rng, 32, 256, A, cs, np.ones(256, np.int8), natural=True, cls=7)
        assert lin.slot_type is None
        return [t for t in ts if not t[0].startswith("blk.0.attn_k.")] + tensors_of("blk.0.attn_k", lin, 3)
    path, _ = model(tmp_path, 3, tensor_edit=tiny)
    with pytest.raises(p8x.P8xError, match="exceed every slot size"):
        p8x.VrFile(path)
