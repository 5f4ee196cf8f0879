"""ctypes harness for libp8x (the MI355X Pingala-8 hot path) and a minimal HIP runtime binding.

No torch: device memory, streams and events come straight from libamdhip64. The product library must be
built (`make -C pingala8-llm_amd/csrc`); loading fails loudly when it is missing.
"""
import ctypes
import ctypes.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libp8x.so")

P8X_OK, P8X_ERR_ARG, P8X_ERR_FORMAT, P8X_ERR_HIP, P8X_ERR_UNSUPPORTED, P8X_ERR_NOMEM = range(6)
F32, F16, BF16, I16 = 0, 1, 2, 3
ACT_Q8_128, ACT_Q8_1, ACT_X16 = 0, 1, 2
GEMV_KERNEL_AUTO, GEMV_KERNEL_DOT4, GEMV_KERNEL_MFMA = 0, 1, 2   # p8x_gemv_batch_create_ex
MAX_COLS = 8
VR3_TAG = 0x56523300

EXPORTS = [
    "p8x_version", "p8x_error_string", "p8x_last_error", "p8x_need", "p8x_probe", "p8x_prepare", "p8x_release",
    "p8x_tensor_info", "p8x_dequantize", "p8x_decode_rotated", "p8x_quantize_q8_128", "p8x_quantize_q8_1",
    "p8x_vec_dot", "p8x_mul_mat_vec", "p8x_mul_mat_vec_act", "p8x_mul_mat", "p8x_mul_mat_reserve", "p8x_synth_random",
    "p8x_quantize_tensor", "p8x_slot_bytes", "p8x_gemv_batch_create", "p8x_gemv_batch_run", "p8x_gemv_batch_run_stage",
    "p8x_gemv_batch_run_stage_timed",
    "p8x_gemv_batch_release", "p8x_gemv_batch_info", "p8x_mul_mat_noalloc",
    "p8x_vr_open", "p8x_vr_count", "p8x_vr_find", "p8x_vr_describe", "p8x_vr_load", "p8x_vr_close", "p8x_vr3_rows",
    "p8x_vr3_expand", "p8x_quantize_x16", "p8x_mul_mat_vec_multi", "p8x_mul_mat_vec_glu", "p8x_mul_mat_vec_multi_act",
    "p8x_mul_mat_vec_glu_act", "p8x_gemv_batch_create_act", "p8x_gemv_batch_create_ex", "p8x_graph_begin", "p8x_decode_tiles",
    "p8x_dequantize_rows", "p8x_vec_dot_rows", "p8x_encode_defaults", "p8x_encode_tensor", "p8x_encode_free",
    "p8x_encode_factor", "p8x_encode_alloc", "p8x_step_create", "p8x_step_create_act", "p8x_step_run", "p8x_step_check", "p8x_step_info",
    "p8x_step_release",
]


class P8xError(RuntimeError):
    pass


def _finalizing():
    """True while the interpreter shuts down: objects collected then are not released through HIP (the runtime, or a
    profiler's tool attached to it, may already be gone); owners release them explicitly before that."""
    return sys.is_finalizing()


class Info(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_int), ("K", ctypes.c_int), ("nd", ctypes.c_int), ("ng", ctypes.c_int), ("nb", ctypes.c_int),
                ("n", ctypes.c_size_t), ("kbytes", ctypes.c_size_t), ("stream_bytes", ctypes.c_size_t),
                ("class_tiles", ctypes.c_size_t * 8), ("dev_base", ctypes.c_void_p)]


class VrDesc(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("rows", ctypes.c_int), ("K", ctypes.c_int), ("nd", ctypes.c_int),
                ("layout", ctypes.c_int), ("fbytes", ctypes.c_size_t), ("kbytes", ctypes.c_size_t),
                ("slot_bytes", ctypes.c_size_t), ("slot_type", ctypes.c_int)]


class BatchInfo(ctypes.Structure):
    _fields_ = [(f, ctypes.c_int) for f in ("njobs", "ncols", "class_set", "units", "split_jobs", "small_launch", "waves",
                                            "matrix_cores")]


class EncodeParams(ctypes.Structure):
    _fields_ = [("c16", ctypes.c_void_p), ("signs", ctypes.c_void_p), ("sign_seed", ctypes.c_uint64),
                ("H", ctypes.c_void_p), ("U", ctypes.c_void_p), ("damp", ctypes.c_double), ("classes", ctypes.c_void_p),
                ("bits_per_weight", ctypes.c_double), ("n_salient", ctypes.c_int), ("prm", ctypes.c_void_p),
                ("alpha", ctypes.c_double), ("gain", ctypes.c_void_p), ("dist", ctypes.c_void_p), ("A", ctypes.c_void_p),
                ("cs", ctypes.c_uint32), ("threads", ctypes.c_int)]


class StepStageC(ctypes.Structure):
    _fields_ = [("n", ctypes.c_int), ("tensors", ctypes.c_void_p * 4), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p * 4),
                ("glu_out", ctypes.c_void_p)]


_lib = None


def lib():
    """libp8x.so with argtypes set; raises when the build is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise P8xError(f"libp8x.so not built: {LIB_PATH} (run make -C pingala8-llm_amd/csrc)")
    L = ctypes.CDLL(LIB_PATH)
    vp, i, sz, u64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_uint64
    L.p8x_version.restype = ctypes.c_char_p
    L.p8x_error_string.restype = ctypes.c_char_p
    L.p8x_error_string.argtypes = [i]
    L.p8x_last_error.restype = ctypes.c_char_p
    L.p8x_need.argtypes = [sz, i, i, i]; L.p8x_need.restype = sz
    L.p8x_probe.argtypes = [vp, sz, i, i]
    L.p8x_prepare.argtypes = [vp, sz, i, i, i, ctypes.POINTER(vp)]
    L.p8x_release.argtypes = [vp]; L.p8x_release.restype = None
    L.p8x_tensor_info.argtypes = [vp, ctypes.POINTER(Info)]
    L.p8x_dequantize.argtypes = [vp, i, vp, sz, vp]
    L.p8x_decode_rotated.argtypes = [vp, i, vp, sz, vp]
    L.p8x_quantize_q8_128.argtypes = [vp, vp, i, sz, vp, vp, vp, vp]
    L.p8x_quantize_q8_1.argtypes = [vp, vp, i, sz, vp, vp]
    L.p8x_quantize_x16.argtypes = [vp, vp, i, sz, vp, vp, vp, vp, vp, vp, vp]
    L.p8x_mul_mat_vec_multi.argtypes = [vp, i, vp, sz, vp, vp, vp]
    L.p8x_mul_mat_vec_multi_act.argtypes = [vp, i, i, vp, sz, vp, vp, vp]
    L.p8x_graph_begin.argtypes = []; L.p8x_graph_begin.restype = None
    L.p8x_decode_tiles.argtypes = [vp, i, i, i, i, i, vp, sz, vp]
    L.p8x_dequantize_rows.argtypes = [vp, i, i, i, vp, sz, vp]
    L.p8x_vec_dot_rows.argtypes = [vp, i, vp, vp, i, i, i, vp, sz, vp, sz, vp, vp]
    L.p8x_mul_mat_vec_glu.argtypes = [vp, vp, vp, sz, vp, vp]
    L.p8x_mul_mat_vec_glu_act.argtypes = [vp, vp, i, vp, sz, vp, vp]
    L.p8x_vec_dot.argtypes = [vp, i, vp, vp, i, vp, sz, vp, sz, vp, vp]
    L.p8x_mul_mat_vec.argtypes = [vp, vp, i, sz, vp, sz, vp]
    L.p8x_mul_mat_vec_act.argtypes = [vp, i, vp, i, sz, vp, sz, vp]
    L.p8x_mul_mat.argtypes = [vp, vp, i, i, sz, vp, sz, vp]
    L.p8x_mul_mat_reserve.argtypes = [vp, i]
    L.p8x_mul_mat_noalloc.argtypes = [vp, vp, i, i, sz, vp, sz, vp]
    L.p8x_vr_open.argtypes = [ctypes.POINTER(ctypes.c_char_p), i, ctypes.POINTER(vp)]
    L.p8x_vr_count.argtypes = [vp]
    L.p8x_vr_find.argtypes = [vp, ctypes.c_char_p]
    L.p8x_vr_describe.argtypes = [vp, i, ctypes.POINTER(VrDesc)]
    L.p8x_vr_load.argtypes = [vp, i, vp, sz]
    L.p8x_vr_close.argtypes = [vp]; L.p8x_vr_close.restype = None
    L.p8x_vr3_rows.argtypes = [sz, sz, ctypes.c_uint32, ctypes.POINTER(sz)]; L.p8x_vr3_rows.restype = sz
    L.p8x_vr3_expand.argtypes = [vp, sz, sz, sz, vp, sz]
    L.p8x_synth_random.argtypes = [u64, i, i, vp, i, i, i, vp, sz, ctypes.POINTER(sz)]
    L.p8x_quantize_tensor.argtypes = [vp, i, i, vp, u64, vp, sz, ctypes.POINTER(sz)]
    L.p8x_slot_bytes.argtypes = [i, i, vp, i]; L.p8x_slot_bytes.restype = sz
    L.p8x_encode_defaults.argtypes = [ctypes.POINTER(EncodeParams)]; L.p8x_encode_defaults.restype = None
    L.p8x_encode_tensor.argtypes = [vp, i, i, ctypes.POINTER(EncodeParams), ctypes.POINTER(vp), ctypes.POINTER(sz)]
    L.p8x_encode_free.argtypes = [vp]; L.p8x_encode_free.restype = None
    L.p8x_encode_factor.argtypes = [vp, vp, vp, u64, i, ctypes.c_double, i, vp]
    L.p8x_encode_alloc.argtypes = [vp, i, ctypes.c_double, vp, vp, vp]
    L.p8x_step_create.argtypes = [ctypes.POINTER(StepStageC), i, ctypes.POINTER(vp)]
    L.p8x_step_create_act.argtypes = [ctypes.POINTER(StepStageC), i, i, ctypes.POINTER(vp)]
    L.p8x_step_run.argtypes = [vp, vp]
    L.p8x_step_check.argtypes = [vp]
    L.p8x_step_info.argtypes = [vp, ctypes.POINTER(i), ctypes.POINTER(i), ctypes.POINTER(i)]
    L.p8x_step_release.argtypes = [vp]; L.p8x_step_release.restype = None
    L.p8x_gemv_batch_create.argtypes = [vp, vp, vp, vp, vp, i, i, ctypes.POINTER(vp)]
    L.p8x_gemv_batch_create_act.argtypes = [vp, vp, vp, vp, vp, i, i, i, ctypes.POINTER(vp)]
    L.p8x_gemv_batch_create_ex.argtypes = [vp, vp, vp, vp, vp, i, i, i, i, ctypes.POINTER(vp)]
    L.p8x_gemv_batch_run.argtypes = [vp, vp]
    L.p8x_gemv_batch_run_stage.argtypes = [vp, i, vp]
    L.p8x_gemv_batch_run_stage_timed.argtypes = [vp, i, vp, vp, vp]
    L.p8x_gemv_batch_release.argtypes = [vp]; L.p8x_gemv_batch_release.restype = None
    L.p8x_gemv_batch_info.argtypes = [vp, ctypes.POINTER(BatchInfo)]
    _lib = L
    return L


def check(rc, what=""):
    if rc != P8X_OK:
        L = lib()
        raise P8xError(f"{what}: {L.p8x_error_string(rc).decode()} ({L.p8x_last_error().decode()})")


# --------------------------------------------------------------------------------------------------- HIP runtime
_hip = None


def hip():
    global _hip
    if _hip is None:
        path = None
        for cand in ("/opt/rocm/lib/libamdhip64.so", ctypes.util.find_library("amdhip64")):
            if cand and (os.path.exists(cand) or not cand.startswith("/")):
                path = cand
                break
        H = ctypes.CDLL(path)
        vp, sz, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        H.hipMalloc.argtypes = [ctypes.POINTER(vp), sz]
        H.hipFree.argtypes = [vp]
        H.hipMemcpy.argtypes = [vp, vp, sz, i]
        H.hipMemset.argtypes = [vp, i, sz]
        H.hipDeviceSynchronize.argtypes = []
        H.hipGetErrorString.restype = ctypes.c_char_p
        H.hipGetErrorString.argtypes = [i]
        H.hipStreamCreate.argtypes = [ctypes.POINTER(vp)]
        H.hipStreamDestroy.argtypes = [vp]
        H.hipStreamSynchronize.argtypes = [vp]
        H.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        H.hipEventDestroy.argtypes = [vp]
        H.hipEventRecord.argtypes = [vp, vp]
        H.hipEventSynchronize.argtypes = [vp]
        H.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        H.hipGetDeviceCount.argtypes = [ctypes.POINTER(i)]
        H.hipStreamBeginCapture.argtypes = [vp, i]
        H.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
        H.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, vp, sz]
        H.hipGraphLaunch.argtypes = [vp, vp]
        H.hipGraphExecDestroy.argtypes = [vp]
        H.hipGraphDestroy.argtypes = [vp]
        _hip = H
    return _hip


def hip_check(rc, what=""):
    if rc != 0:
        raise P8xError(f"{what}: HIP error {rc} {hip().hipGetErrorString(rc).decode()}")


def device_count():
    n = ctypes.c_int(0)
    try:
        if hip().hipGetDeviceCount(ctypes.byref(n)) != 0:
            return 0
    except OSError:
        return 0
    return n.value


H2D, D2H, D2D = 1, 2, 3


class DeviceBuffer:
    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = ctypes.c_void_p()
        hip_check(hip().hipMalloc(ctypes.byref(self.ptr), max(self.nbytes, 16)), "hipMalloc")

    @classmethod
    def from_numpy(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            hip_check(hip().hipMemcpy(b.ptr, a.ctypes.data_as(ctypes.c_void_p), a.nbytes, H2D), "hipMemcpy H2D")
        return b

    def to_numpy(self, dtype, shape):
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        if out.nbytes:
            hip_check(hip().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.ptr, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def fill(self, byte):
        hip_check(hip().hipMemset(self.ptr, byte, self.nbytes), "hipMemset")

    def copy_from(self, other, nbytes=None):
        """device-to-device copy (synchronous on the null stream)"""
        n = min(self.nbytes, other.nbytes) if nbytes is None else int(nbytes)
        hip_check(hip().hipMemcpy(self.ptr, other.ptr, n, D2D), "hipMemcpy D2D")

    @property
    def addr(self):
        return self.ptr.value

    def free(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        if _finalizing():
            return
        try:
            self.free()
        except Exception:
            pass


def synchronize():
    hip_check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Stream:
    def __init__(self):
        self.h = ctypes.c_void_p()
        hip_check(hip().hipStreamCreate(ctypes.byref(self.h)), "hipStreamCreate")

    def sync(self):
        hip_check(hip().hipStreamSynchronize(self.h), "hipStreamSynchronize")

    def release(self):
        if self.h:
            hip().hipStreamSynchronize(self.h)
            hip().hipStreamDestroy(self.h)
            self.h = ctypes.c_void_p()

    def __del__(self):
        if _finalizing():
            return
        try:
            self.release()
        except Exception:
            pass


class Graph:
    """A HIP graph of the work `enqueue(stream)` issues on `stream`, captured once (global capture mode: a call
    that is not capture-safe fails the capture) and replayed with launch()."""

    def __init__(self, enqueue, stream):
        H = hip()
        self.g, self.x = ctypes.c_void_p(), ctypes.c_void_p()
        hip_check(H.hipStreamBeginCapture(stream.h, 0), "hipStreamBeginCapture")
        try:
            enqueue(stream)
        finally:
            hip_check(H.hipStreamEndCapture(stream.h, ctypes.byref(self.g)), "hipStreamEndCapture")
        hip_check(H.hipGraphInstantiate(ctypes.byref(self.x), self.g, None, None, 0), "hipGraphInstantiate")

    def launch(self, stream):
        hip_check(hip().hipGraphLaunch(self.x, stream.h), "hipGraphLaunch")

    def release(self):
        if self.x:
            hip().hipGraphExecDestroy(self.x)
            self.x = ctypes.c_void_p()
        if self.g:
            hip().hipGraphDestroy(self.g)
            self.g = ctypes.c_void_p()

    def __del__(self):
        if _finalizing():
            return
        try:
            self.release()
        except Exception:
            pass


class Event:
    def __init__(self):
        self.h = ctypes.c_void_p()
        hip_check(hip().hipEventCreate(ctypes.byref(self.h)), "hipEventCreate")

    def record(self, stream=None):
        hip_check(hip().hipEventRecord(self.h, stream.h if stream else None), "hipEventRecord")

    def elapsed_ms(self, later):
        ms = ctypes.c_float(0)
        hip_check(hip().hipEventSynchronize(later.h), "hipEventSynchronize")
        hip_check(hip().hipEventElapsedTime(ctypes.byref(ms), self.h, later.h), "hipEventElapsedTime")
        return ms.value

    def release(self):
        if self.h:
            hip().hipEventDestroy(self.h)
            self.h = ctypes.c_void_p()

    def __del__(self):
        if _finalizing():
            return
        try:
            self.release()
        except Exception:
            pass


# --------------------------------------------------------------------------------------------------- host producers
CLASS_P_C3 = (0, 0, 0, 1, 0, 0, 0, 0)


def synth_random(seed, rows, K, class_p=CLASS_P_C3, codebook=0, nd=0, permute=True):
    """random valid slot bytes (numpy uint8)"""
    L = lib()
    cp = (ctypes.c_double * 8)(*class_p)
    n = ctypes.c_size_t(0)
    L.p8x_synth_random(seed, rows, K, cp, codebook, nd, int(permute), None, 0, ctypes.byref(n))
    buf = np.empty(n.value, np.uint8)
    check(L.p8x_synth_random(seed, rows, K, cp, codebook, nd, int(permute), buf.ctypes.data, buf.size, ctypes.byref(n)), "synth_random")
    return buf


def encode_tensor(W, c16=None, H=None, U=None, classes=None, bits_per_weight=2.0, n_salient=4, prm=None, alpha=1.05,
                  signs=None, sign_seed=0, damp=0.1, gain=None, dist=None, A=None, cs=0, threads=0):
    """Slot bytes from f32 weights [rows][K] (every class, LDLQ feedback from H or U, class allocation).
    classes: (rows/32, K/256) uint8 per sorted tile or None; H: (K, K) input second moment; U: (K, K) rotated factor."""
    L = lib()
    W = np.ascontiguousarray(W, np.float32)
    rows, K = W.shape
    keep = []

    def ptr(a, dt, shape=None):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dt)
        if shape is not None and a.shape != shape:
            raise P8xError(f"encode_tensor: expected shape {shape}, got {a.shape}")
        keep.append(a)
        return a.ctypes.data

    p = EncodeParams()
    L.p8x_encode_defaults(ctypes.byref(p))
    p.c16 = ptr(c16, np.uint16, (K,))
    p.signs = ptr(signs, np.int8, (256,))
    p.sign_seed = sign_seed
    p.H = ptr(H, np.float32, (K, K))
    p.U = ptr(U, np.float64, (K, K))
    p.damp = damp
    p.classes = ptr(classes, np.uint8, (rows // 32, K // 256))
    p.bits_per_weight = bits_per_weight
    p.n_salient = n_salient
    p.prm = ptr(prm, np.int16, (rows,))
    p.alpha = alpha
    p.gain = ptr(gain, np.float64, (8,))
    p.dist = ptr(dist, np.float64, (8,))
    p.A = ptr(A, np.uint32, (256,))
    p.cs = cs
    p.threads = threads
    out = ctypes.c_void_p()
    n = ctypes.c_size_t(0)
    check(L.p8x_encode_tensor(W.ctypes.data, rows, K, ctypes.byref(p), ctypes.byref(out), ctypes.byref(n)), "encode_tensor")
    try:
        buf = np.frombuffer((ctypes.c_uint8 * n.value).from_address(out.value), np.uint8).copy()
    finally:
        L.p8x_encode_free(out)
    return buf


def encode_factor(H, c16=None, signs=None, sign_seed=0, damp=0.1, threads=0):
    """(K, K) float64 upper factor U of the damped rotated inverse second moment"""
    L = lib()
    H = np.ascontiguousarray(H, np.float32)
    K = H.shape[0]
    c = None if c16 is None else np.ascontiguousarray(c16, np.uint16)
    sg = None if signs is None else np.ascontiguousarray(signs, np.int8)
    U = np.empty((K, K), np.float64)
    check(L.p8x_encode_factor(H.ctypes.data, None if c is None else c.ctypes.data, None if sg is None else sg.ctypes.data,
                              sign_seed, K, damp, threads, U.ctypes.data), "encode_factor")
    return U


def encode_alloc(E, budget_bits, dist=None, floor=None):
    """class per tile (uint8, E's shape) from per-tile distortion weights E within budget_bits"""
    L = lib()
    E = np.ascontiguousarray(E, np.float64)
    d = None if dist is None else np.ascontiguousarray(dist, np.float64)
    f = None if floor is None else np.ascontiguousarray(floor, np.uint8)
    out = np.empty(E.shape, np.uint8)
    check(L.p8x_encode_alloc(E.ctypes.data, E.size, budget_bits, None if d is None else d.ctypes.data,
                             None if f is None else f.ctypes.data, out.ctypes.data), "encode_alloc")
    return out


def quantize_tensor(W, c16=None, sign_seed=0):
    """class-3 slot bytes from f32 weights [rows][K] (plain-MSE Viterbi)"""
    L = lib()
    W = np.ascontiguousarray(W, np.float32)
    rows, K = W.shape
    c = None if c16 is None else np.ascontiguousarray(c16, np.uint16)
    cptr = None if c is None else c.ctypes.data
    n = ctypes.c_size_t(0)
    L.p8x_quantize_tensor(W.ctypes.data, rows, K, cptr, sign_seed, None, 0, ctypes.byref(n))
    buf = np.empty(n.value + 64, np.uint8)
    check(L.p8x_quantize_tensor(W.ctypes.data, rows, K, cptr, sign_seed, buf.ctypes.data, buf.size, ctypes.byref(n)), "quantize_tensor")
    return buf[:n.value].copy()


def side_offsets(n, rows, K, nd):
    """byte offsets of the side regions of an n-byte slot, top-down from its end (delta, c16, prm, pinv, signs,
    trailer), as the tensor contract lays them out"""
    t = n - 32
    sg = t - 256
    q = (sg - 2 * rows) & ~15
    p = (q - 2 * rows) & ~15
    c = (p - 2 * K) & ~15
    e = (c - 8 * nd) & ~15
    return {"E": e, "C": c, "P": p, "Q": q, "SG": sg, "T": t}


def slot_nd(slot):
    """clamp-delta entry count from a slot's trailer"""
    return int(np.frombuffer(np.ascontiguousarray(slot[-32:]).tobytes(), np.uint32)[3])


def share_input(slots, shapes, signs_from=None):
    """Give host slots [(rows, K)] one input rotation in place: the column scales c and Hadamard signs of slots[0]
    (or the signs of signs_from) copied into the others, as a file encodes linears that share an input (one c per
    input, one sign vector for the model). The slots must have equal K."""
    r0, K0 = shapes[0]
    o0 = side_offsets(slots[0].size, r0, K0, slot_nd(slots[0]))
    c16 = slots[0][o0["C"]:o0["C"] + 2 * K0].copy()
    sg = (signs_from if signs_from is not None else slots[0][o0["SG"]:o0["SG"] + 256]).copy()
    for s, (r, K) in zip(slots, shapes):
        assert K == K0
        o = side_offsets(s.size, r, K, slot_nd(s))
        s[o["C"]:o["C"] + 2 * K] = c16
        s[o["SG"]:o["SG"] + 256] = sg


# --------------------------------------------------------------------------------------------------- model files
class VrFile:
    """A native Pingala-8 model file (GGUF; one path, or the shards of one model)."""

    def __init__(self, paths):
        if isinstance(paths, (str, bytes, os.PathLike)):
            paths = [paths]
        arr = (ctypes.c_char_p * len(paths))(*[os.fsencode(p) for p in paths])
        self.h = ctypes.c_void_p()
        check(lib().p8x_vr_open(arr, len(paths), ctypes.byref(self.h)), "p8x_vr_open")

    def __len__(self):
        return lib().p8x_vr_count(self.h)

    def find(self, name):
        return lib().p8x_vr_find(self.h, name.encode())

    def describe(self, i):
        d = VrDesc()
        check(lib().p8x_vr_describe(self.h, i, ctypes.byref(d)), "p8x_vr_describe")
        return {f: (getattr(d, f).decode() if f == "name" else getattr(d, f)) for f, _ in VrDesc._fields_}

    def load(self, i):
        """slot bytes of linear i (numpy uint8), ready for Tensor(slot, rows, K)"""
        n = self.describe(i)["slot_bytes"]
        buf = np.empty(n, np.uint8)
        check(lib().p8x_vr_load(self.h, i, buf.ctypes.data, n), "p8x_vr_load")
        return buf

    def close(self):
        if self.h:
            lib().p8x_vr_close(self.h)
            self.h = ctypes.c_void_p()

    def __del__(self):
        if _finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


def vr3_rows(fbytes, K, w515):
    kb = ctypes.c_size_t(0)
    rows = lib().p8x_vr3_rows(fbytes, K, w515, ctypes.byref(kb))
    return rows, kb.value


def vr3_expand(file_bytes, rows, K, out):
    f = np.ascontiguousarray(file_bytes, np.uint8)
    check(lib().p8x_vr3_expand(f.ctypes.data, f.size, rows, K, out.ctypes.data, out.size), "p8x_vr3_expand")


# --------------------------------------------------------------------------------------------------- tensors
def _vp(x):
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    if isinstance(x, int):
        return ctypes.c_void_p(x)
    return x


class Tensor:
    """A prepared tensor slot (device-resident)."""

    def __init__(self, slot, rows, K, device_slot=None):
        L = lib()
        self.rows, self.K = rows, K
        self.h = ctypes.c_void_p()
        if device_slot is not None:
            check(L.p8x_prepare(device_slot.ptr, device_slot.nbytes, rows, K, 1, ctypes.byref(self.h)), "p8x_prepare")
            self._keep = device_slot
        else:
            slot = np.ascontiguousarray(slot, np.uint8)
            check(L.p8x_prepare(slot.ctypes.data, slot.size, rows, K, 0, ctypes.byref(self.h)), "p8x_prepare")
        inf = Info()
        check(L.p8x_tensor_info(self.h, ctypes.byref(inf)), "p8x_tensor_info")
        self.info = inf
        self.nsl = K // 128

    @property
    def stream_bytes(self):
        return self.info.stream_bytes

    def release(self):
        if self.h:
            lib().p8x_release(self.h)
            self.h = ctypes.c_void_p()

    def __del__(self):
        if _finalizing():
            return
        try:
            self.release()
        except Exception:
            pass

    # ---- device-pointer entry points
    def dequantize_dev(self, dtype, out, ld=None, stream=None):
        check(lib().p8x_dequantize(self.h, dtype, _vp(out), ld or self.K, stream.h if stream else None), "p8x_dequantize")

    def decode_rotated_dev(self, dtype, out, ld=None, stream=None):
        check(lib().p8x_decode_rotated(self.h, dtype, _vp(out), ld or self.K, stream.h if stream else None), "p8x_decode_rotated")

    def mul_mat_vec_dev(self, x, y, ncols=1, ldx=None, ldy=None, act=ACT_Q8_128, stream=None):
        check(lib().p8x_mul_mat_vec_act(self.h, act, _vp(x), ncols, ldx or self.K, _vp(y), ldy or self.rows,
                                        stream.h if stream else None), "p8x_mul_mat_vec")

    def quantize_q8_128_dev(self, x, q, d, ncols=1, ldx=None, stream=None):
        check(lib().p8x_quantize_q8_128(self.h, _vp(x), ncols, ldx or self.K, _vp(q), _vp(d), None,
                                        stream.h if stream else None), "p8x_quantize_q8_128")

    def vec_dot_dev(self, act, q, d, y, ncols=1, x=None, ldx=None, ldy=None, stream=None):
        check(lib().p8x_vec_dot(self.h, act, _vp(q), _vp(d), ncols, _vp(x), ldx or self.K, _vp(y), ldy or self.rows,
                                None, stream.h if stream else None), "p8x_vec_dot")

    def mul_mat_reserve(self, n_max):
        check(lib().p8x_mul_mat_reserve(self.h, n_max), "p8x_mul_mat_reserve")

    def mul_mat_dev(self, x, x_dtype, N, y, ldx=None, ldy=None, stream=None):
        check(lib().p8x_mul_mat(self.h, _vp(x), x_dtype, N, ldx or self.K, _vp(y), ldy or self.rows,
                                stream.h if stream else None), "p8x_mul_mat")

    def mul_mat_noalloc_dev(self, x, x_dtype, N, y, ldx=None, ldy=None, stream=None):
        check(lib().p8x_mul_mat_noalloc(self.h, _vp(x), x_dtype, N, ldx or self.K, _vp(y), ldy or self.rows,
                                        stream.h if stream else None), "p8x_mul_mat_noalloc")

    # ---- numpy conveniences (copy in / out, synchronous)
    def dequantize(self, dtype=F32):
        npdt = {F32: np.float32, F16: np.uint16, BF16: np.uint16}[dtype]
        out = DeviceBuffer(self.rows * self.K * np.dtype(npdt).itemsize)
        self.dequantize_dev(dtype, out)
        synchronize()
        return out.to_numpy(npdt, (self.rows, self.K))

    def decode_rotated(self, dtype=I16):
        npdt = {I16: np.int16, F32: np.float32}[dtype]
        out = DeviceBuffer(self.rows * self.K * np.dtype(npdt).itemsize)
        self.decode_rotated_dev(dtype, out)
        synchronize()
        return out.to_numpy(npdt, (self.rows, self.K))

    def quantize_q8_128(self, x):
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        ncols = x.shape[0]
        xd = DeviceBuffer.from_numpy(x)
        q = DeviceBuffer(ncols * self.K); d = DeviceBuffer(4 * ncols * self.nsl); s = DeviceBuffer(4 * ncols * self.nsl)
        check(lib().p8x_quantize_q8_128(self.h, xd.ptr, ncols, self.K, q.ptr, d.ptr, s.ptr, None), "p8x_quantize_q8_128")
        synchronize()
        return (q.to_numpy(np.int8, (ncols, self.K)), d.to_numpy(np.float32, (ncols, self.nsl)),
                s.to_numpy(np.int32, (ncols, self.nsl)))

    def decode_tiles(self, g0, ng, b0, nb, dtype=I16):
        """rotated-domain tiles of row groups g0 .. and blocks b0 ..: [32 ng][256 nb]"""
        npdt = {I16: np.int16, F32: np.float32}[dtype]
        out = DeviceBuffer(32 * ng * 256 * nb * np.dtype(npdt).itemsize)
        check(lib().p8x_decode_tiles(self.h, dtype, g0, ng, b0, nb, out.ptr, 256 * nb, None), "p8x_decode_tiles")
        synchronize()
        return out.to_numpy(npdt, (32 * ng, 256 * nb))

    def dequantize_rows(self, row0, nrows, dtype=F32, ld=None):
        """original rows row0 .. row0 + nrows - 1, [nrows][ld] (ld >= K; the columns past K are left as allocated)"""
        ld = ld or self.K
        npdt = {F32: np.float32, F16: np.uint16, BF16: np.uint16}[dtype]
        out = DeviceBuffer(nrows * ld * np.dtype(npdt).itemsize)
        out.fill(0)
        check(lib().p8x_dequantize_rows(self.h, dtype, row0, nrows, out.ptr, ld, None), "p8x_dequantize_rows")
        synchronize()
        return out.to_numpy(npdt, (nrows, ld))

    def vec_dot_rows(self, act, q, d, g0, ng, x=None):
        """(y [ncols][rows] with only row groups g0 .. written (NaN elsewhere), partials [ncols][32 ng][blocks])"""
        q = np.ascontiguousarray(q)
        ncols = q.shape[0]
        qd = DeviceBuffer.from_numpy(q)
        dd = DeviceBuffer.from_numpy(np.ascontiguousarray(d, np.float32)) if d is not None else None
        xd = DeviceBuffer.from_numpy(np.ascontiguousarray(x, np.float32)) if x is not None else None
        y = DeviceBuffer.from_numpy(np.full((ncols, self.rows), np.nan, np.float32))
        nblk = self.nsl if act == ACT_Q8_128 else self.K // 32
        p = DeviceBuffer(4 * ncols * 32 * ng * nblk)
        check(lib().p8x_vec_dot_rows(self.h, act, qd.ptr, dd.ptr if dd else None, ncols, g0, ng, xd.ptr if xd else None, self.K,
                                     y.ptr, self.rows, p.ptr, None), "p8x_vec_dot_rows")
        synchronize()
        return y.to_numpy(np.float32, (ncols, self.rows)), p.to_numpy(np.int32, (ncols, 32 * ng, nblk))

    def quantize_x16(self, x):
        """(qh, dh, sh, ql, dl, sl) per column: the x16 planes"""
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        ncols = x.shape[0]
        xd = DeviceBuffer.from_numpy(x)
        bufs = [DeviceBuffer(ncols * self.K), DeviceBuffer(4 * ncols * self.nsl), DeviceBuffer(4 * ncols * self.nsl),
                DeviceBuffer(ncols * self.K), DeviceBuffer(4 * ncols * self.nsl), DeviceBuffer(4 * ncols * self.nsl)]
        check(lib().p8x_quantize_x16(self.h, xd.ptr, ncols, self.K, *[b.ptr for b in bufs], None), "p8x_quantize_x16")
        synchronize()
        kinds = [(np.int8, self.K), (np.float32, self.nsl), (np.int32, self.nsl)] * 2
        return tuple(b.to_numpy(dt, (ncols, n)) for b, (dt, n) in zip(bufs, kinds))

    def quantize_q8_1(self, x):
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        ncols = x.shape[0]
        xd = DeviceBuffer.from_numpy(x)
        blk = DeviceBuffer(ncols * 36 * (self.K // 32))
        check(lib().p8x_quantize_q8_1(self.h, xd.ptr, ncols, self.K, blk.ptr, None), "p8x_quantize_q8_1")
        synchronize()
        return blk.to_numpy(np.uint8, (ncols, 36 * (self.K // 32)))

    def vec_dot(self, act, q, d=None, partials=False):
        """y (no delta) and optionally the integer partials, from host-quantized activations"""
        q = np.ascontiguousarray(q)
        ncols = q.shape[0]
        qd = DeviceBuffer.from_numpy(q)
        dd = DeviceBuffer.from_numpy(np.ascontiguousarray(d, np.float32)) if d is not None else None
        y = DeviceBuffer(4 * ncols * self.rows)
        nblk = self.nsl if act == ACT_Q8_128 else self.K // 32
        p = DeviceBuffer(4 * ncols * self.rows * nblk) if partials else None
        check(lib().p8x_vec_dot(self.h, act, qd.ptr, dd.ptr if dd else None, ncols, None, 0, y.ptr, self.rows,
                                p.ptr if p else None, None), "p8x_vec_dot")
        synchronize()
        yo = y.to_numpy(np.float32, (ncols, self.rows))
        if partials:
            return yo, p.to_numpy(np.int32, (ncols, self.rows, nblk))
        return yo

    def mul_mat_vec(self, x, act=ACT_Q8_128):
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        ncols = x.shape[0]
        xd = DeviceBuffer.from_numpy(x)
        y = DeviceBuffer(4 * ncols * self.rows)
        self.mul_mat_vec_dev(xd, y, ncols=ncols, act=act)
        synchronize()
        return y.to_numpy(np.float32, (ncols, self.rows))

    def mul_mat(self, X, dtype=F32):
        X = np.ascontiguousarray(X)
        N = X.shape[0]
        xd = DeviceBuffer.from_numpy(X)
        y = DeviceBuffer(4 * N * self.rows)
        self.mul_mat_dev(xd, dtype, N, y)
        synchronize()
        return y.to_numpy(np.float32, (N, self.rows))


def graph_begin():
    """start of a graph evaluation: later x16 / block_q8_1 calls on the same input reuse its prepared activation"""
    lib().p8x_graph_begin()


def mul_mat_vec_multi_dev(tensors, x, ys, stream=None, act=ACT_Q8_128):
    """y_i = W_i x for tensors sharing K and input rotation, the activation prepared once (device buffers)"""
    n = len(tensors)
    T = (ctypes.c_void_p * n)(*[t.h.value for t in tensors])
    Y = (ctypes.c_void_p * n)(*[y.addr for y in ys])
    LY = (ctypes.c_size_t * n)(*[t.rows for t in tensors])
    st = stream.h if stream else None
    if act == ACT_Q8_128:
        check(lib().p8x_mul_mat_vec_multi(T, n, _vp(x), tensors[0].K, Y, LY, st), "p8x_mul_mat_vec_multi")
    else:
        check(lib().p8x_mul_mat_vec_multi_act(T, n, act, _vp(x), tensors[0].K, Y, LY, st), "p8x_mul_mat_vec_multi_act")


def mul_mat_vec_multi(tensors, x, act=ACT_Q8_128):
    xd = DeviceBuffer.from_numpy(np.ascontiguousarray(x, np.float32))
    ys = [DeviceBuffer(4 * t.rows) for t in tensors]
    mul_mat_vec_multi_dev(tensors, xd, ys, act=act)
    synchronize()
    return [y.to_numpy(np.float32, (t.rows,)) for y, t in zip(ys, tensors)]


def mul_mat_vec_glu_dev(gate, up, x, out, stream=None, act=ACT_Q8_128):
    st = stream.h if stream else None
    if act == ACT_Q8_128:
        check(lib().p8x_mul_mat_vec_glu(gate.h, up.h, _vp(x), gate.K, _vp(out), st), "p8x_mul_mat_vec_glu")
    else:
        check(lib().p8x_mul_mat_vec_glu_act(gate.h, up.h, act, _vp(x), gate.K, _vp(out), st), "p8x_mul_mat_vec_glu_act")


def mul_mat_vec_glu(gate, up, x, act=ACT_Q8_128):
    """silu(gate x) * (up x)"""
    xd = DeviceBuffer.from_numpy(np.ascontiguousarray(x, np.float32))
    out = DeviceBuffer(4 * gate.rows)
    mul_mat_vec_glu_dev(gate, up, xd, out, act=act)
    synchronize()
    return out.to_numpy(np.float32, (gate.rows,))


class Step:
    """A chain of linears in one launch (p8x_step_*). stages: list of (tensors, x, ys) or (tensors, x, None, glu_out)
    with device buffers; stage s may read an earlier stage's output. The step keeps the tensors and buffers alive
    until release() (the library holds their addresses). act: ACT_Q8_128 (one cooperative launch), ACT_Q8_1 or
    ACT_X16 (the stages enqueued as their per-node calls)."""

    def __init__(self, stages, act=ACT_Q8_128):
        self._keep = [list(st) for st in stages]
        arr = (StepStageC * len(stages))()
        for k, st in enumerate(stages):
            tensors, x, ys = st[0], st[1], st[2]
            glu = st[3] if len(st) > 3 else None
            arr[k].n = len(tensors)
            for i, t in enumerate(tensors):
                arr[k].tensors[i] = t.h.value
            arr[k].x = x.addr
            if ys is not None:
                for i, y in enumerate(ys):
                    arr[k].y[i] = y.addr
            arr[k].glu_out = glu.addr if glu is not None else None
        self.h = ctypes.c_void_p()
        check(lib().p8x_step_create_act(arr, len(stages), act, ctypes.byref(self.h)), "p8x_step_create")

    def run(self, stream=None):
        check(lib().p8x_step_run(self.h, stream.h if stream else None), "p8x_step_run")

    def check(self):
        check(lib().p8x_step_check(self.h), "p8x_step_check")

    def info(self):
        """grid (workgroups of the launch), stages, and the class set of the chain's tensors"""
        g, n, cm = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        check(lib().p8x_step_info(self.h, ctypes.byref(g), ctypes.byref(n), ctypes.byref(cm)), "p8x_step_info")
        return {"grid": g.value, "stages": n.value, "class_set": cm.value}

    def release(self):
        if self.h:
            lib().p8x_step_release(self.h)
            self.h = ctypes.c_void_p()
        self._keep = None

    def __del__(self):
        if _finalizing():
            return
        try:
            self.release()
        except Exception:
            pass


class GemvBatch:
    """A grouped launch of independent GEMVs (device buffers x_i, y_i fixed at creation)."""

    stages = 3   # activation prep, fused decode + GEMV, finishing (original rows, clamp delta)

    def __init__(self, tensors, xs, ys, ncols=1, act=ACT_Q8_128, kernel=0):
        n = len(tensors)
        T = (ctypes.c_void_p * n)(*[t.h.value for t in tensors])
        X = (ctypes.c_void_p * n)(*[x.addr for x in xs])
        Y = (ctypes.c_void_p * n)(*[y.addr for y in ys])
        LX = (ctypes.c_size_t * n)(*[t.K for t in tensors])
        LY = (ctypes.c_size_t * n)(*[t.rows for t in tensors])
        self.h = ctypes.c_void_p()
        check(lib().p8x_gemv_batch_create_ex(T, X, LX, Y, LY, n, ncols, act, kernel, ctypes.byref(self.h)), "p8x_gemv_batch_create")
        self._keep = (tensors, xs, ys)

    def info(self):
        inf = BatchInfo()
        check(lib().p8x_gemv_batch_info(self.h, ctypes.byref(inf)), "p8x_gemv_batch_info")
        return {f: getattr(inf, f) for f, _ in BatchInfo._fields_}

    def run(self, stream=None):
        check(lib().p8x_gemv_batch_run(self.h, stream.h if stream else None), "p8x_gemv_batch_run")

    def run_stage(self, stage, stream=None, events=None):
        """events = (start, stop) Event pair recorded at the stage kernel's own start and end"""
        if events is None:
            check(lib().p8x_gemv_batch_run_stage(self.h, stage, stream.h if stream else None), "p8x_gemv_batch_run_stage")
        else:
            check(lib().p8x_gemv_batch_run_stage_timed(self.h, stage, stream.h if stream else None, events[0].h, events[1].h),
                  "p8x_gemv_batch_run_stage_timed")

    def release(self):
        if self.h:
            lib().p8x_gemv_batch_release(self.h)
            self.h = ctypes.c_void_p()

    def __del__(self):
        if _finalizing():
            return
        try:
            self.release()
        except Exception:
            pass
