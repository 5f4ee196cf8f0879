"""Grouped GEMV on the matrix cores (k_gemv_wave_mx: class-3 batches of 2..8 q8/128 columns, tile products as
v_mfma_i32_32x32x32_i8) against the v_dot4 kernel of the same batch (bit for bit: the integer tile sums are exact
and the float steps are the same) and against the fp64 oracle."""
import numpy as np
import pytest

import oracle as O
import p8x

pytestmark = pytest.mark.gpu

C3 = (0, 0, 0, 1, 0, 0, 0, 0)


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def run_batch(tensors, xs, rows, ncols, mx, act=p8x.ACT_Q8_128):
    """one grouped launch on the matrix-core kernel (mx) or the v_dot4 kernel, chosen at creation"""
    ys = [p8x.DeviceBuffer(4 * ncols * r) for r in rows]
    batch = p8x.GemvBatch(tensors, xs, ys, ncols=ncols, act=act, kernel=p8x.GEMV_KERNEL_MFMA if mx else p8x.GEMV_KERNEL_DOT4)
    info = batch.info()
    out = []
    for rep in range(2):   # twice: the unit counters are put back for the next launch
        batch.run()
        p8x.synchronize()
        out.append([y.to_numpy(np.float32, (ncols, r)) for y, r in zip(ys, rows)])
    batch.release()
    for y in ys:
        y.free()
    for a, b in zip(out[0], out[1]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return info, out[0]


@pytest.mark.parametrize("ncols", [2, 3, 4, 5, 6, 7, 8])
def test_mx_batch_matches_dot4_and_oracle(ncols):
    """mixed shapes (a 32 x 256 tensor, long K with K-split units, clamp-delta rows): the matrix-core launch gives
    the v_dot4 launch's bits, and each column is within 1e-5 of the fp64 oracle"""
    shapes = [(1024, 4096), (512, 14336), (32, 256), (2048, 2560), (96, 768)]
    rng = np.random.default_rng(500 + ncols)
    tensors, orcs, xs, hx = [], [], [], []
    for i, (rows, K) in enumerate(shapes):
        slot = p8x.synth_random(900 + 7 * ncols + i, rows, K, class_p=C3, nd=3)
        tensors.append(p8x.Tensor(slot, rows, K))
        orcs.append(O.Oracle(slot, rows, K))
        X = rng.standard_normal((ncols, K)).astype(np.float32)
        hx.append(X)
        xs.append(p8x.DeviceBuffer.from_numpy(X))
    rows = [r for r, _ in shapes]
    info_mx, y_mx = run_batch(tensors, xs, rows, ncols, True)
    info_d4, y_d4 = run_batch(tensors, xs, rows, ncols, False)
    assert info_mx["matrix_cores"] == 1 and info_d4["matrix_cores"] == 0
    for i in range(len(shapes)):
        assert np.array_equal(y_mx[i].view(np.uint32), y_d4[i].view(np.uint32)), i
        for n in range(ncols):
            assert rel_l2(y_mx[i][n], orcs[i].gemv_f64(hx[i][n])) < 1e-5, (i, n)
    for t in tensors:
        t.release()
    for x in xs:
        x.free()


@pytest.mark.parametrize("ncols", [1, 2, 3, 4])
def test_mx_batch_x16_matches_dot4_and_oracle(ncols):
    """x16 activations (both planes as virtual columns): the matrix-core launch gives the v_dot4 launch's bits, and
    each column is within 1e-5 of the oracle's x16 GEMV"""
    shapes = [(1024, 4096), (512, 14336), (32, 256)]
    rng = np.random.default_rng(700 + ncols)
    tensors, orcs, xs, hx = [], [], [], []
    for i, (rows, K) in enumerate(shapes):
        slot = p8x.synth_random(950 + 5 * ncols + i, rows, K, class_p=C3, nd=2)
        tensors.append(p8x.Tensor(slot, rows, K))
        orcs.append(O.Oracle(slot, rows, K))
        X = rng.standard_normal((ncols, K)).astype(np.float32)
        hx.append(X)
        xs.append(p8x.DeviceBuffer.from_numpy(X))
    rows = [r for r, _ in shapes]
    info_mx, y_mx = run_batch(tensors, xs, rows, ncols, True, act=p8x.ACT_X16)
    info_d4, y_d4 = run_batch(tensors, xs, rows, ncols, False, act=p8x.ACT_X16)
    assert info_mx["matrix_cores"] == 1 and info_d4["matrix_cores"] == 0
    for i in range(len(shapes)):
        assert np.array_equal(y_mx[i].view(np.uint32), y_d4[i].view(np.uint32)), i
        for n in range(ncols):
            assert rel_l2(y_mx[i][n], orcs[i].gemv_f64(hx[i][n], act="x16")) < 1e-5, (i, n)
    for t in tensors:
        t.release()
    for x in xs:
        x.free()


def test_mx_plan_choice():
    """by default the matrix cores take class-3 batches of 4..8 multiplied columns (q8/128 columns, or x16 columns
    with their two planes); one to three, and non-class-3 sets, stay on the v_dot4 kernel"""
    rows, K = 256, 2048
    t3 = p8x.Tensor(p8x.synth_random(31, rows, K, class_p=C3, nd=1), rows, K)
    t6 = p8x.Tensor(p8x.synth_random(32, rows, K, class_p=(0, 0, 0, 0, 0, 0, 1, 0), nd=1), rows, K)
    x8 = p8x.DeviceBuffer.from_numpy(np.ones((8, K), np.float32))
    y8 = p8x.DeviceBuffer(4 * 8 * rows)
    for ts, ncols, act, want in (([t3], 1, p8x.ACT_Q8_128, 0), ([t3], 2, p8x.ACT_Q8_128, 0), ([t3], 3, p8x.ACT_Q8_128, 0),
                                 ([t6], 4, p8x.ACT_Q8_128, 0), ([t3], 4, p8x.ACT_Q8_128, 1), ([t3], 8, p8x.ACT_Q8_128, 1),
                                 ([t3], 1, p8x.ACT_X16, 0), ([t3], 2, p8x.ACT_X16, 1), ([t3], 4, p8x.ACT_X16, 1)):
        b = p8x.GemvBatch(ts, [x8], [y8], ncols=ncols, act=act)
        assert b.info()["matrix_cores"] == want, (ncols, act)
        b.release()
    t3.release()
    t6.release()
    x8.free()
    y8.free()


def test_mx_kernel_choice_rejected_outside_its_set():
    """asking for the matrix-core kernel where it does not apply (one multiplied column, a non-class-3 set) fails at
    creation; an unknown kernel value too"""
    rows, K = 256, 2048
    t3 = p8x.Tensor(p8x.synth_random(33, rows, K, class_p=C3, nd=1), rows, K)
    t6 = p8x.Tensor(p8x.synth_random(34, rows, K, class_p=(0, 0, 0, 0, 0, 0, 1, 0), nd=1), rows, K)
    x = p8x.DeviceBuffer.from_numpy(np.ones((8, K), np.float32))
    y = p8x.DeviceBuffer(4 * 8 * rows)
    for ts, ncols in (([t3], 1), ([t6], 4)):
        with pytest.raises(p8x.P8xError, match="matrix-core kernel"):
            p8x.GemvBatch(ts, [x], [y], ncols=ncols, kernel=p8x.GEMV_KERNEL_MFMA)
    with pytest.raises(p8x.P8xError, match="kernel 7"):
        p8x.GemvBatch([t3], [x], [y], ncols=2, kernel=7)
    t3.release()
    t6.release()
    x.free()
    y.free()
