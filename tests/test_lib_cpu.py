"""libp8x host-side checks that need no GPU: the C ABI loads and exports every declared symbol, the host
producers write slots the oracle accepts, and the class-3 quantizer's Viterbi is optimal."""
import os
import re

import numpy as np
import pytest

import oracle as O
import p8x
import slotgen

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    txt = open(os.path.join(ROOT, "include", "p8x.h")).read()
    return sorted(set(re.findall(r"\b(p8x_[a-z0-9_]+)\s*\(", txt)))


def test_header_declares_python_exports():
    assert sorted(p8x.EXPORTS) == declared_symbols()


def test_library_exports_every_declared_symbol():
    L = p8x.lib()
    for name in declared_symbols():
        assert hasattr(L, name), name
    assert L.p8x_version().decode().startswith("p8x")


def test_need_matches_contract():
    L = p8x.lib()
    for kb, rows, K, nd in ((4335632, 4096, 4096, 0), (1000, 32, 256, 3), (77777, 1024, 2560, 17)):
        assert L.p8x_need(kb, rows, K, nd) == slotgen.need(kb, rows, K, nd)


def test_probe_on_fixture():
    z = np.load(os.path.join(ROOT, "tests", "golden", "case_mixed.npz"))
    slot = np.ascontiguousarray(z["slot"])
    L = p8x.lib()
    assert L.p8x_probe(slot.ctypes.data, slot.size, int(z["rows"]), int(z["K"])) == 1
    assert L.p8x_probe(slot.ctypes.data, slot.size, int(z["rows"]) + 32, int(z["K"])) == 0


@pytest.mark.parametrize("classes,nd,cb", [((3,), 0, 0), ((0, 1, 2, 3, 4, 5, 6, 7), 9, 0), ((1, 4, 7), 4, 1)])
def test_synth_random_is_valid(classes, nd, cb):
    p = [0.0] * 8
    for c in classes:
        p[c] = 1.0
    slot = p8x.synth_random(7, 128, 1024, class_p=p, codebook=cb, nd=nd)
    orc = O.Oracle(slot, 128, 1024)
    assert orc.nd == nd
    ints = orc.decode_all()
    assert ints.shape == (128, 1024)
    # deterministic
    assert np.array_equal(slot, p8x.synth_random(7, 128, 1024, class_p=p, codebook=cb, nd=nd))


def _viterbi_ref(X, cb):
    """independent 8-state DP on one half-slice: X [32,4] targets, cb [2][256][4]; returns min cost"""
    cost = np.empty((32, 2, 2))
    for h in range(2):
        d = ((X[:, None, :] - cb[h][None, :, :]) ** 2).sum(-1)   # [32, 256]
        cost[:, h, 0] = d[:, :128].min(1)
        cost[:, h, 1] = d[:, 128:].min(1)
    pm = {0: 0.0}
    for t in range(32):
        nm = {}
        for s, v in pm.items():
            h = (s >> 1) & 1
            for m in (0, 1):
                u = m ^ (s & 1) ^ ((s >> 2) & 1)
                s2 = ((s << 1) | u) & 7
                c = v + cost[t, h, m]
                if c < nm.get(s2, 1e300):
                    nm[s2] = c
        pm = nm
    return min(pm.values())


def test_quantizer_viterbi_optimal_and_accurate():
    rng = np.random.default_rng(0)
    rows, K = 32, 512
    W = (rng.standard_normal((rows, K)) * 0.02).astype(np.float32)
    slot = p8x.quantize_tensor(W, sign_seed=3)
    orc = O.Oracle(slot, rows, K)
    Wd = orc.dequant()
    rel = np.linalg.norm(Wd - W) / np.linalg.norm(W)
    assert rel < 0.45, rel   # ~2 bpw code: SNR ~ 9-11 dB
    # optimality: achieved half-slice cost == independent DP minimum
    A, c = slotgen.shipped_tables()
    A8 = A.view(np.int8).reshape(256, 4).astype(np.float64)
    c8 = np.frombuffer(np.uint32(c).tobytes(), np.int8).astype(np.float64)
    cb = np.stack([A8, A8 + c8[None, :]])
    ints = orc.decode_all().astype(np.float64)
    nt = (rows // 32) * (K // 256)
    S = slot[2064 + 4 * nt:2064 + 68 * nt].view(np.float16).astype(np.float64).reshape(K // 256, rows)
    o = slotgen.offsets(slot.size, rows, K, orc.nd)
    sg = slot[o["SG"]:o["SG"] + 256].view(np.int8).astype(np.float64)
    from scipy.linalg import hadamard
    H = hadamard(256) / 16.0
    for r in (0, 5, 31):
        for b in range(K // 256):
            T = H @ (W[r, 256 * b:256 * b + 256].astype(np.float64) * sg)
            sc = S[b, r]
            for hs in range(2):
                X = (T[128 * hs:128 * hs + 128] / sc).reshape(32, 4)
                got = ((X - ints[r, 256 * b + 128 * hs:256 * b + 128 * hs + 128].reshape(32, 4)) ** 2).sum()
                ref = _viterbi_ref(X, cb)
                assert got == pytest.approx(ref, rel=1e-9, abs=1e-9)


def test_quantizer_outliers_get_clamp_delta():
    rng = np.random.default_rng(1)
    rows, K = 64, 512
    W = (rng.standard_normal((rows, K)) * 0.02).astype(np.float32)
    mask = rng.random((rows, K)) < 0.001
    W[mask] *= 10
    slot = p8x.quantize_tensor(W, sign_seed=1)
    orc = O.Oracle(slot, rows, K)
    Wd = orc.dequant()
    wmax = np.float32(np.float16(np.abs(W).max() * np.float32(1.001)))
    assert np.abs(Wd).max() <= wmax * (1 + 1e-6)


def test_product_library_has_no_timeline_instrumentation():
    """the launch-timeline stamps live only in the separate analysis build (make timeline)"""
    L = p8x.lib()
    assert not hasattr(L, "p8x_timeline_read")
    path = os.path.join(os.path.dirname(p8x.LIB_PATH), "libp8x_timeline.so")
    if os.path.exists(path):
        import ctypes
        T = ctypes.CDLL(path)
        assert hasattr(T, "p8x_timeline_read") and hasattr(T, "p8x_timeline_reset")


def test_timeline_module_parses_arguments():
    import subprocess
    import sys
    r = subprocess.run([sys.executable, "-m", "p8x.timeline", "--help"], cwd=os.path.join(ROOT, "pingala8-llm_amd"),
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "--layers" in r.stdout
