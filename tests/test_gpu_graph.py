"""HIP graph capture of the device entry points: a captured sequence of single GEMV calls (one and several
columns) and a captured grouped launch replay bit-identically to the same calls made eagerly, with eager work
and synchronisations between the replays. The launches record no memset nodes (the grouped launch's unit
counters are put back by its own last waves)."""
import numpy as np
import pytest

import p8x

pytestmark = pytest.mark.gpu

SHAPES = [(1024, 4096, (0, 0, 0, 1, 0, 0, 0, 0)), (512, 14336, (0, 0, 1, 8, 1, 0, 0, 0)),
          (2048, 2560, (0, 0, 0, 0, 0, 0, 1, 0)), (96, 768, (1, 1, 1, 1, 1, 1, 1, 1))]


def make(ncols, seed):
    rng = np.random.default_rng(seed)
    tensors, xs, ys = [], [], []
    for i, (rows, K, cp) in enumerate(SHAPES):
        tensors.append(p8x.Tensor(p8x.synth_random(300 + i, rows, K, class_p=cp, nd=3), rows, K))
        xs.append(p8x.DeviceBuffer.from_numpy(rng.standard_normal((ncols, K)).astype(np.float32)))
        ys.append(p8x.DeviceBuffer(4 * ncols * rows))
    return tensors, xs, ys


def outputs(tensors, ys, ncols):
    return [y.to_numpy(np.float32, (ncols, t.rows)).copy() for t, y in zip(tensors, ys)]


def clear(ys):
    for y in ys:
        y.fill(0xFF)   # NaN patterns: a replay that skips a row shows
    p8x.synchronize()


@pytest.mark.parametrize("ncols", [1, 3])
def test_captured_single_calls_replay_bitwise(ncols):
    tensors, xs, ys = make(ncols, 11 + ncols)
    st = p8x.Stream()

    def enqueue(stream):
        for t, x, y in zip(tensors, xs, ys):
            t.mul_mat_vec_dev(x, y, ncols=ncols, stream=stream)

    enqueue(st)
    st.sync()
    ref = outputs(tensors, ys, ncols)
    g = p8x.Graph(enqueue, st)
    try:
        for rep in range(3):
            clear(ys)
            g.launch(st)
            st.sync()
            got = outputs(tensors, ys, ncols)
            for i, (a, b) in enumerate(zip(got, ref)):
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (rep, i)
            enqueue(st)   # eager work between replays
            st.sync()
    finally:
        g.release()


@pytest.mark.parametrize("ncols", [1, 2])
def test_captured_grouped_launch_replay_bitwise(ncols):
    tensors, xs, ys = make(ncols, 21 + ncols)
    st = p8x.Stream()
    batch = p8x.GemvBatch(tensors, xs, ys, ncols=ncols)
    batch.run(st)
    st.sync()
    ref = outputs(tensors, ys, ncols)
    g = p8x.Graph(lambda s: batch.run(s), st)
    try:
        for rep in range(3):
            clear(ys)
            g.launch(st)
            st.sync()
            got = outputs(tensors, ys, ncols)
            for i, (a, b) in enumerate(zip(got, ref)):
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (rep, i)
            batch.run(st)   # eager launches between replays reuse the same unit counters
            st.sync()
    finally:
        g.release()
        batch.release()
