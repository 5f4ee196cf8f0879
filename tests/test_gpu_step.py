"""The decode-step object (p8x_step_*): a chain of linears in one cooperative launch, each stage reading an earlier
stage's output, against the same chain run as one launch per node (p8x_mul_mat_vec_multi / p8x_mul_mat_vec /
p8x_mul_mat_vec_glu), which the parity tests pin to the oracle. Bar: every stage's output bit-identical to the
per-node chain, on consecutive runs; one stage also against the fp64 oracle.

Shapes reach every stage variant: q/k/v as one multi-linear stage, gate/up with teams of waves (more row groups than
CUs), down with two K-chunks (K = 8192, the split-K fix-up), two head shards."""
import numpy as np
import pytest

import oracle as O
import p8x

pytestmark = pytest.mark.gpu

HIDDEN, KV, FFN = 1024, 256, 8192
HEAD = (16384, 16384)
C3 = [0, 0, 0, 1, 0, 0, 0, 0]
MIXED = [0.05, 0.1, 0.1, 0.35, 0.1, 0.1, 0.15, 0.05]


def group(seed, shapes, class_p):
    slots = [p8x.synth_random(seed + i, r, K, class_p=class_p, nd=1) for i, (r, K) in enumerate(shapes)]
    o = p8x.side_offsets(slots[0].size, shapes[0][0], shapes[0][1], 1)
    p8x.share_input(slots, shapes, signs_from=slots[0][o["SG"]:o["SG"] + 256].copy())
    return slots


def build(class_p, layers=2, seed=100):
    L, host = [], {}
    for l in range(layers):
        qkv = group(seed, [(HIDDEN, HIDDEN), (KV, HIDDEN), (KV, HIDDEN)], class_p)
        o = group(seed + 10, [(HIDDEN, HIDDEN)], class_p)
        gu = group(seed + 20, [(FFN, HIDDEN), (FFN, HIDDEN)], class_p)
        d = group(seed + 30, [(HIDDEN, FFN)], class_p)
        seed += 100
        shapes = [(HIDDEN, HIDDEN), (KV, HIDDEN), (KV, HIDDEN), (HIDDEN, HIDDEN), (FFN, HIDDEN), (FFN, HIDDEN), (HIDDEN, FFN)]
        slots = qkv + o + gu + d
        L.append([p8x.Tensor(s, r, K) for s, (r, K) in zip(slots, shapes)])
        if l == 0:
            host["o"] = (slots[3], HIDDEN, HIDDEN)
    hs = group(seed, [(r, HIDDEN) for r in HEAD], class_p)
    head = [p8x.Tensor(s, r, HIDDEN) for s, r in zip(hs, HEAD)]
    return L, head, host


def chain(L, head, x0):
    """stages and the buffers of each stage's outputs"""
    stages, outs = [], []
    cur = x0
    for q, k, v, o, gate, up, down in L:
        yq, yk, yv = (p8x.DeviceBuffer(4 * t.rows) for t in (q, k, v))
        yo, yg, yd = p8x.DeviceBuffer(4 * o.rows), p8x.DeviceBuffer(4 * gate.rows), p8x.DeviceBuffer(4 * down.rows)
        stages += [([q, k, v], cur, [yq, yk, yv]), ([o], yq, [yo]), ([gate, up], yo, None, yg), ([down], yg, [yd])]
        outs += [(yq, q.rows), (yk, k.rows), (yv, v.rows), (yo, o.rows), (yg, gate.rows), (yd, down.rows)]
        cur = yd
    yh = [p8x.DeviceBuffer(4 * t.rows) for t in head]
    stages.append((head, cur, yh))
    outs += [(y, t.rows) for y, t in zip(yh, head)]
    return stages, outs


def run_per_node(stages):
    for st in stages:
        ts, x, ys = st[0], st[1], st[2]
        if len(st) > 3:
            p8x.mul_mat_vec_glu_dev(ts[0], ts[1], x, st[3])
        elif len(ts) == 1:
            ts[0].mul_mat_vec_dev(x, ys[0])
        else:
            p8x.mul_mat_vec_multi_dev(ts, x, ys)
    p8x.synchronize()


def read(outs):
    return [b.to_numpy(np.float32, (n,)).copy() for b, n in outs]


@pytest.mark.parametrize("mix", ["c3", "mixed"])
def test_step_equals_per_node_chain(mix):
    L, head, host = build(C3 if mix == "c3" else MIXED)
    rng = np.random.default_rng(1)
    x0 = p8x.DeviceBuffer.from_numpy(rng.standard_normal(HIDDEN).astype(np.float32))
    stages, outs = chain(L, head, x0)
    run_per_node(stages)
    want = read(outs)
    assert all(np.isfinite(w).all() for w in want)
    step = p8x.Step(stages)
    info = step.info()
    assert info["stages"] == len(stages) and info["grid"] >= 1
    assert info["class_set"] == (8 if mix == "c3" else 0xFE)
    for rep in range(3):
        for b, _ in outs:   # poison the outputs (NaN bytes): the step must write every value
            b.fill(0xFF)
        step.run()
        step.check()
        got = read(outs)
        for i, (g, w) in enumerate(zip(got, want)):
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (mix, rep, i)
    # the first o stage against the fp64 oracle on its own input (the q output)
    slot, rows, K = host["o"]
    orc = O.Oracle(slot, rows, K)
    yo = got[3]
    ref = orc.gemv_f64(got[0])
    assert np.linalg.norm(yo - ref) / np.linalg.norm(ref) < 1e-3
    step.release()


def test_step_rejects_mismatched_stage():
    L, head, _ = build(C3, layers=1)
    x0 = p8x.DeviceBuffer(4 * HIDDEN)
    q, k, v, o, gate, up, down = L[0]
    with pytest.raises(p8x.P8xError, match="K"):
        p8x.Step([([q, down], x0, [p8x.DeviceBuffer(4 * HIDDEN), p8x.DeviceBuffer(4 * HIDDEN)])])
    with pytest.raises(p8x.P8xError, match="swiglu"):
        p8x.Step([([gate], x0, None, p8x.DeviceBuffer(4 * FFN))])
