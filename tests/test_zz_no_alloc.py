"""p8x_mul_mat_noalloc (prompt GEMM with its workspace in the library's fixed per-GPU scratch array) against
p8x_mul_mat (the allocating entry point, same kernels): bitwise equal outputs, on two calls in a row, the second
with a smaller input; both also against the fp64 oracle at the GEMM bar (1e-3 relative L2). Oversized requests are
rejected on the host before any GPU work."""
import numpy as np
import pytest

import oracle as O
import p8x

pytestmark = pytest.mark.gpu


def bf16(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def run_both(t, X, dtype):
    N = X.shape[0]
    xd = p8x.DeviceBuffer.from_numpy(X)
    y_ref = p8x.DeviceBuffer(4 * N * t.rows)
    y_na = p8x.DeviceBuffer(4 * N * t.rows)
    y_na.fill(0xFF)
    t.mul_mat_dev(xd, dtype, N, y_ref)
    t.mul_mat_noalloc_dev(xd, dtype, N, y_na)
    p8x.synchronize()
    return y_na.to_numpy(np.float32, (N, t.rows)), y_ref.to_numpy(np.float32, (N, t.rows))


def test_noalloc_matches_mul_mat_two_calls():
    rng = np.random.default_rng(71)
    # call 1: the 512-token Llama FFN up-projection (14336 x 4096, bf16 activations, permuted rows, clamp delta)
    rows, K, N = 14336, 4096, 512
    slot = p8x.synth_random(71, rows, K, nd=8)
    t = p8x.Tensor(slot, rows, K)
    X = bf16(rng.standard_normal((N, K)))
    Y, R = run_both(t, X, p8x.BF16)
    assert np.array_equal(Y.view(np.uint32), R.view(np.uint32))
    orc = O.Oracle(slot, rows, K)
    sample = [0, 1, 255, 511]
    Xs = (X[sample].astype(np.uint32) << 16).view(np.float32)
    assert rel_l2(Y[sample], O.dense_f64(orc.dequant(), Xs)) < 1e-3
    # call 2, smaller: a 1024 x 2560 tensor of every class, 40 f32 tokens (less scratch than call 1 left behind)
    rows2, K2, N2 = 1024, 2560, 40
    slot2 = p8x.synth_random(72, rows2, K2, class_p=(1, 1, 1, 1, 1, 1, 1, 1), nd=5)
    t2 = p8x.Tensor(slot2, rows2, K2)
    X2 = rng.standard_normal((N2, K2)).astype(np.float32)
    Y2, R2 = run_both(t2, X2, p8x.F32)
    assert np.array_equal(Y2.view(np.uint32), R2.view(np.uint32))
    orc2 = O.Oracle(slot2, rows2, K2)
    assert rel_l2(Y2, O.dense_f64(orc2.dequant(), X2)) < 1e-3


def test_noalloc_runs_the_ffn_down_shape():
    """the 512-token Llama FFN down-projection (4096 x 14336, class 3, bf16): its K-split plan fits the scratch next
    to x', and both entry points run that same plan (bitwise equal outputs)"""
    rng = np.random.default_rng(74)
    rows, K, N = 4096, 14336, 512
    slot = p8x.synth_random(74, rows, K, nd=8)
    t = p8x.Tensor(slot, rows, K)
    X = bf16(rng.standard_normal((N, K)))
    Y, R = run_both(t, X, p8x.BF16)
    assert np.array_equal(Y.view(np.uint32), R.view(np.uint32))
    orc = O.Oracle(slot, rows, K)
    sample = [0, 3, 510]
    Xs = (X[sample].astype(np.uint32) << 16).view(np.float32)
    assert rel_l2(Y[sample], O.dense_f64(orc.dequant(), Xs)) < 1e-3


def test_noalloc_rejects_oversized_request():
    """4096 tokens of a 4096 x 14336 tensor need 117 MB of rotated activations alone: rejected before any launch"""
    rows, K, N = 4096, 14336, 4096
    t = p8x.Tensor(p8x.synth_random(73, rows, K, nd=1), rows, K)
    xd = p8x.DeviceBuffer(2 * N * K)
    yd = p8x.DeviceBuffer(4 * N * rows)
    with pytest.raises(p8x.P8xError, match="scratch"):
        t.mul_mat_noalloc_dev(xd, p8x.BF16, N, yd)
