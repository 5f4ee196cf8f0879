"""ctypes wrappers for the CPU oracle (oracle/p8x_oracle.c) and for the reference's own CPU core
compiled by oracle/Makefile into oracle/_ref/ (when the reference tree was present at build time).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
always as the checker (or the CPU baseline), never as the product path.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "libp8x_oracle.so")
REF_DIR = os.path.join(HERE, "_ref")

_c_u8p = ctypes.POINTER(ctypes.c_uint8)


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


class OrcTensor(ctypes.Structure):
    _fields_ = [
        ("base", ctypes.c_void_p), ("n", ctypes.c_size_t),
        ("rows", ctypes.c_int), ("K", ctypes.c_int), ("nb", ctypes.c_int), ("ng", ctypes.c_int),
        ("nsl", ctypes.c_int), ("nd", ctypes.c_int),
        ("nt", ctypes.c_size_t), ("kbytes", ctypes.c_size_t),
        ("A", ctypes.c_void_p), ("cs", ctypes.c_uint32), ("M", ctypes.c_void_p), ("S", ctypes.c_void_p),
        ("D", ctypes.c_void_p), ("c16", ctypes.c_void_p), ("prm", ctypes.c_void_p), ("pinv", ctypes.c_void_p),
        ("sg", ctypes.c_void_p), ("drow", ctypes.c_void_p), ("dcol", ctypes.c_void_p), ("dval", ctypes.c_void_p),
        ("ic", ctypes.c_void_p), ("cp", ctypes.c_void_p), ("cc", ctypes.c_void_p), ("cv", ctypes.c_void_p),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"oracle library missing: {ORACLE_SO} (run make -C oracle)")
        L = ctypes.CDLL(ORACLE_SO)
        vp, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        L.orc_open.argtypes = [ctypes.POINTER(OrcTensor), vp, sz, i, i]
        L.orc_close.argtypes = [ctypes.POINTER(OrcTensor)]
        L.orc_need.argtypes = [sz, sz, sz, sz]; L.orc_need.restype = sz
        L.orc_offsets.argtypes = [sz, sz, sz, sz, vp]
        L.orc_trellis_word.argtypes = [ctypes.c_uint32]; L.orc_trellis_word.restype = ctypes.c_uint32
        L.orc_trellis_serial.argtypes = [ctypes.c_uint32]; L.orc_trellis_serial.restype = ctypes.c_uint32
        L.orc_weight_int.argtypes = [ctypes.POINTER(OrcTensor), i, i]
        L.orc_decode_tile.argtypes = [ctypes.POINTER(OrcTensor), i, i, vp]
        L.orc_decode_all.argtypes = [ctypes.POINTER(OrcTensor), vp]
        L.orc_dequant_f32.argtypes = [ctypes.POINTER(OrcTensor), vp]
        L.orc_fwht256.argtypes = [vp]
        L.orc_prep_q8_128.argtypes = [ctypes.POINTER(OrcTensor), vp, vp, vp, vp]
        L.orc_prep_x16.argtypes = [ctypes.POINTER(OrcTensor), vp, vp, vp, vp, vp, vp, vp]
        L.orc_quantize_q8_1.argtypes = [ctypes.POINTER(OrcTensor), vp, vp]
        L.orc_rotate_act.argtypes = [ctypes.POINTER(OrcTensor), vp, vp]
        L.orc_partials_q8_128.argtypes = [ctypes.POINTER(OrcTensor), vp, vp]
        L.orc_partials_q8_1.argtypes = [ctypes.POINTER(OrcTensor), vp, vp]
        L.orc_gemv_q8_128_f64.argtypes = [ctypes.POINTER(OrcTensor), vp, vp]
        L.orc_gemv_q8_1_f64.argtypes = [ctypes.POINTER(OrcTensor), vp, vp]
        L.orc_gemv_x16_f64.argtypes = [ctypes.POINTER(OrcTensor), vp, vp]
        L.orc_gemv_q8_128_f64_cols.argtypes = [ctypes.POINTER(OrcTensor), vp, i, sz, vp]
        L.orc_dense_f64.argtypes = [vp, i, i, vp, i, vp]
        L.orc_h2f.argtypes = [ctypes.c_uint16]; L.orc_h2f.restype = ctypes.c_float
        L.orc_f2h.argtypes = [ctypes.c_float]; L.orc_f2h.restype = ctypes.c_uint16
        _lib = L
    return _lib


class Oracle:
    """One parsed tensor slot. `buf` is a uint8 numpy array holding the slot bytes."""

    def __init__(self, buf, rows, K):
        self.buf = np.ascontiguousarray(buf, dtype=np.uint8)
        self.rows, self.K = rows, K
        self.t = OrcTensor()
        rc = lib().orc_open(ctypes.byref(self.t), _p(self.buf), self.buf.size, rows, K)
        if rc:
            raise ValueError(f"orc_open failed rc={rc}")
        self.nb, self.ng, self.nsl, self.nd = K // 256, rows // 32, K // 128, self.t.nd

    def close(self):
        if self.t.ic:
            lib().orc_close(ctypes.byref(self.t))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def decode_tile(self, g, b):
        out = np.empty((32, 256), np.int16)
        lib().orc_decode_tile(ctypes.byref(self.t), g, b, _p(out))
        return out

    def decode_all(self):
        out = np.empty((self.rows, self.K), np.int16)
        lib().orc_decode_all(ctypes.byref(self.t), _p(out))
        return out

    def weight_int(self, r, col):
        return lib().orc_weight_int(ctypes.byref(self.t), r, col)

    def dequant(self):
        W = np.empty((self.rows, self.K), np.float32)
        lib().orc_dequant_f32(ctypes.byref(self.t), _p(W))
        return W

    def prep_q8_128(self, x):
        x = np.ascontiguousarray(x, np.float32)
        q = np.empty(self.K, np.int8); d = np.empty(self.nsl, np.float32); sx = np.empty(self.nsl, np.int32)
        lib().orc_prep_q8_128(ctypes.byref(self.t), _p(x), _p(q), _p(d), _p(sx))
        return q, d, sx

    def prep_x16(self, x):
        x = np.ascontiguousarray(x, np.float32)
        qh = np.empty(self.K, np.int8); dh = np.empty(self.nsl, np.float32); sh = np.empty(self.nsl, np.int32)
        ql = np.empty(self.K, np.int8); dl = np.empty(self.nsl, np.float32); sl = np.empty(self.nsl, np.int32)
        lib().orc_prep_x16(ctypes.byref(self.t), _p(x), _p(qh), _p(dh), _p(sh), _p(ql), _p(dl), _p(sl))
        return qh, dh, sh, ql, dl, sl

    def quantize_q8_1(self, x):
        x = np.ascontiguousarray(x, np.float32)
        blk = np.empty(36 * (self.K // 32), np.uint8)
        lib().orc_quantize_q8_1(ctypes.byref(self.t), _p(x), _p(blk))
        return blk

    def rotate(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(self.K, np.float32)
        lib().orc_rotate_act(ctypes.byref(self.t), _p(x), _p(out))
        return out

    def partials_q8_128(self, q):
        q = np.ascontiguousarray(q, np.int8)
        out = np.empty((self.rows, self.nsl), np.int32)
        lib().orc_partials_q8_128(ctypes.byref(self.t), _p(q), _p(out))
        return out

    def partials_q8_1(self, blk):
        blk = np.ascontiguousarray(blk, np.uint8)
        out = np.empty((self.rows, self.K // 32), np.int32)
        lib().orc_partials_q8_1(ctypes.byref(self.t), _p(blk), _p(out))
        return out

    def gemv_f64(self, x, act="q8_128"):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(self.rows, np.float64)
        fn = {"q8_128": lib().orc_gemv_q8_128_f64, "q8_1": lib().orc_gemv_q8_1_f64, "x16": lib().orc_gemv_x16_f64}[act]
        fn(ctypes.byref(self.t), _p(x), _p(y))
        return y

    def gemv_f64_cols(self, X):
        """fp64 GEMV of every row of X [ncols][K] (8-bit-per-128 activations), each tile decoded once"""
        X = np.ascontiguousarray(np.atleast_2d(X), np.float32)
        Y = np.zeros((X.shape[0], self.rows), np.float64)
        lib().orc_gemv_q8_128_f64_cols(ctypes.byref(self.t), _p(X), X.shape[0], X.shape[1], _p(Y))
        return Y

    @property
    def ic(self):
        return np.ctypeslib.as_array(ctypes.cast(self.t.ic, ctypes.POINTER(ctypes.c_float)), (self.K,)).copy()


def trellis_word(z):
    return lib().orc_trellis_word(z)


def trellis_serial(z):
    return lib().orc_trellis_serial(z)


def fwht256(v):
    v = np.array(v, np.float32)
    lib().orc_fwht256(_p(v))
    return v


def dense_f64(W, x):
    W = np.ascontiguousarray(W, np.float32); x = np.ascontiguousarray(x, np.float32)
    N = x.shape[0]; rows, K = W.shape
    y = np.empty((N, rows), np.float64)
    lib().orc_dense_f64(_p(W), rows, K, _p(x), N, _p(y))
    return y


# ------------------------------------------------------------------------------ reference core (oracle/_ref)
def ref_available(variant="scalar"):
    return os.path.exists(os.path.join(REF_DIR, f"libvrref_{variant}.so"))


def cpu_flags():
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("flags"):
                    return set(ln.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def best_ref_variant():
    fl = cpu_flags()
    if "avx_vnni" in fl and "avx2" in fl and "fma" in fl and "f16c" in fl and ref_available("vnni"):
        return "vnni"
    if "avx2" in fl and "fma" in fl and "f16c" in fl and ref_available("avx2"):
        return "avx2"
    return "scalar"


class RefCore:
    """The reference CPU core (vr-native-cpu-core.h) behind oracle/ref_driver.c."""

    def __init__(self, variant="scalar"):
        path = os.path.join(REF_DIR, f"libvrref_{variant}.so")
        if not os.path.exists(path):
            raise RuntimeError(f"reference core not built: {path}")
        L = ctypes.CDLL(path)
        vp, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        L.ref_isa.restype = ctypes.c_char_p
        L.ref_open.argtypes = [vp, sz, i, i, ctypes.POINTER(ctypes.c_int)]; L.ref_open.restype = vp
        L.ref_close.argtypes = [vp]
        L.ref_decode_tile.argtypes = [vp, i, i, vp]
        L.ref_dequant.argtypes = [vp, vp]
        L.ref_prep_block.argtypes = [vp, vp, i, vp, vp, vp]
        L.ref_prep_block16.argtypes = [vp, vp, i, vp, vp, vp, vp, vp, vp]
        L.ref_tile.argtypes = [vp, i, i, i, vp, vp, vp, vp]
        L.ref_pool_create.argtypes = [i]; L.ref_pool_create.restype = vp
        L.ref_pool_destroy.argtypes = [vp]
        L.ref_gemv_seq.argtypes = [vp, vp, vp, vp, i, i]
        self.L = L
        self.variant = variant
        self.isa = L.ref_isa().decode()

    def open(self, buf, rows, K):
        rc = ctypes.c_int(0)
        buf = np.ascontiguousarray(buf, np.uint8)
        h = self.L.ref_open(_p(buf), buf.size, rows, K, ctypes.byref(rc))
        if not h:
            raise ValueError(f"ref_open failed rc={rc.value}")
        return RefTensor(self, h, buf, rows, K)


class RefTensor:
    def __init__(self, core, h, buf, rows, K):
        self.core, self.h, self.buf, self.rows, self.K = core, h, buf, rows, K
        self.nb, self.ng, self.nsl = K // 256, rows // 32, K // 128

    def close(self):
        if self.h:
            self.core.L.ref_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def decode_tile(self, g, b):
        out = np.empty((32, 256), np.int16)
        self.core.L.ref_decode_tile(self.h, g, b, _p(out))
        return out

    def dequant(self):
        W = np.empty((self.rows, self.K), np.float32)
        self.core.L.ref_dequant(self.h, _p(W))
        return W

    def prep_q8_128(self, x):
        """returns q [K] (first copy of each doubled half-slice), d [nsl], sx [nsl]"""
        x = np.ascontiguousarray(x, np.float32)
        X2 = np.empty((self.nsl, 256), np.int8); XS = np.empty(self.nsl, np.float32); SX = np.empty(self.nsl, np.int32)
        for b in range(self.nb):
            self.core.L.ref_prep_block(self.h, _p(x), b, _p(X2[2 * b:]), _p(XS[2 * b:]), _p(SX[2 * b:]))
        return X2, XS, SX

    def prep_x16(self, x):
        x = np.ascontiguousarray(x, np.float32)
        Xh = np.empty((self.nsl, 256), np.int8); XSh = np.empty(self.nsl, np.float32); SXh = np.empty(self.nsl, np.int32)
        Xl = np.empty((self.nsl, 256), np.int8); XSl = np.empty(self.nsl, np.float32); SXl = np.empty(self.nsl, np.int32)
        for b in range(self.nb):
            self.core.L.ref_prep_block16(self.h, _p(x), b, _p(Xh[2 * b:]), _p(XSh[2 * b:]), _p(SXh[2 * b:]),
                                         _p(Xl[2 * b:]), _p(XSl[2 * b:]), _p(SXl[2 * b:]))
        return Xh, XSh, SXh, Xl, XSl, SXl


class RefPool:
    """Persistent thread pool running the reference's two-phase GEMV driver (CPU baseline)."""

    def __init__(self, core, nthreads):
        self.core, self.nth = core, nthreads
        self.h = core.L.ref_pool_create(nthreads)

    def gemv_seq(self, tensors, xs, ys, planes=1):
        n = len(tensors)
        metas = (ctypes.c_void_p * n)(*[t.h for t in tensors])
        xp = (ctypes.c_void_p * n)(*[x.ctypes.data for x in xs])
        yp = (ctypes.c_void_p * n)(*[y.ctypes.data for y in ys])
        self.core.L.ref_gemv_seq(self.h, metas, xp, yp, n, planes)

    def close(self):
        if self.h:
            self.core.L.ref_pool_destroy(self.h)
            self.h = None
