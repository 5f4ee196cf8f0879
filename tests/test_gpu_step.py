"""The decode-step object (p8x_step_*): a chain of linears in one cooperative launch, each stage reading an earlier
stage's output, stages separated by grid barriers.

Every stage's output is bit-identical to the per-node chain (p8x_mul_mat_vec_multi / p8x_mul_mat_vec /
p8x_mul_mat_vec_glu) on consecutive runs and on HIP graph replays (the barrier's run counter lives on the device), and
for class-3 chains also checked against the fp64 oracle on that stage's actual input (1e-5 relative L2, as the
single-call GEMV tests), including the swiglu output.

Shapes reach every stage variant: q/k/v as one multi-linear stage, gate/up with several row groups per workgroup,
down with two K-chunks (K = 8192), two head shards."""
import numpy as np
import pytest

import oracle as O
import p8x

pytestmark = pytest.mark.gpu

HIDDEN, KV, FFN = 1024, 256, 8192
HEAD = (16384, 16384)
C3 = [0, 0, 0, 1, 0, 0, 0, 0]
MIXED = [0.05, 0.1, 0.1, 0.35, 0.1, 0.1, 0.15, 0.05]
SHAPES = [(HIDDEN, HIDDEN), (KV, HIDDEN), (KV, HIDDEN), (HIDDEN, HIDDEN), (FFN, HIDDEN), (FFN, HIDDEN), (HIDDEN, FFN)]


def group(seed, shapes, class_p):
    slots = [p8x.synth_random(seed + i, r, K, class_p=class_p, nd=1) for i, (r, K) in enumerate(shapes)]
    o = p8x.side_offsets(slots[0].size, shapes[0][0], shapes[0][1], 1)
    p8x.share_input(slots, shapes, signs_from=slots[0][o["SG"]:o["SG"] + 256].copy())
    return slots


def build(class_p, layers=2, seed=100):
    """device tensors per layer, head shards, and the host slots of every tensor (same order)"""
    L, hosts = [], []
    for _ in range(layers):
        qkv = group(seed, SHAPES[0:3], class_p)
        o = group(seed + 10, SHAPES[3:4], class_p)
        gu = group(seed + 20, SHAPES[4:6], class_p)
        d = group(seed + 30, SHAPES[6:7], class_p)
        seed += 100
        slots = qkv + o + gu + d
        L.append([p8x.Tensor(s, r, K) for s, (r, K) in zip(slots, SHAPES)])
        hosts.append(list(zip(slots, SHAPES)))
    hs = group(seed, [(r, HIDDEN) for r in HEAD], class_p)
    head = [p8x.Tensor(s, r, HIDDEN) for s, r in zip(hs, HEAD)]
    return L, head, hosts, [(s, (r, HIDDEN)) for s, r in zip(hs, HEAD)]


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


def rel(a, ref):
    return float(np.linalg.norm(a.astype(np.float64) - ref) / np.linalg.norm(ref))


def check_against_oracle(got, x0, hosts, head_hosts):
    """every stage's output vs the fp64 oracle on that stage's input as the step wrote it"""
    orc = [[O.Oracle(s, r, K) for s, (r, K) in layer] for layer in hosts]
    orh = [O.Oracle(s, r, K) for s, (r, K) in head_hosts]
    cur = x0
    for l, layer in enumerate(orc):
        yq, yk, yv, yo, yg, yd = got[6 * l:6 * l + 6]
        for y, o, name in ((yq, layer[0], "q"), (yk, layer[1], "k"), (yv, layer[2], "v")):
            assert rel(y, o.gemv_f64(cur)) < 1e-5, (l, name)
        assert rel(yo, layer[3].gemv_f64(yq)) < 1e-5, (l, "o")
        g, u = layer[4].gemv_f64(yo), layer[5].gemv_f64(yo)
        assert rel(yg, g / (1.0 + np.exp(-g)) * u) < 1e-5, (l, "swiglu")
        assert rel(yd, layer[6].gemv_f64(yg)) < 1e-5, (l, "down")
        cur = yd
    for i, o in enumerate(orh):
        assert rel(got[6 * len(orc) + i], o.gemv_f64(cur)) < 1e-5, ("head", i)


@pytest.mark.parametrize("mix", ["c3", "mixed"])
def test_step_chain(mix):
    L, head, hosts, head_hosts = build(C3 if mix == "c3" else MIXED)
    rng = np.random.default_rng(1)
    x0h = rng.standard_normal(HIDDEN).astype(np.float32)
    x0 = p8x.DeviceBuffer.from_numpy(x0h)
    stages, outs = chain(L, head, x0)
    run_per_node(stages)
    want = read(outs)
    assert all(np.isfinite(w).all() for w in want)
    step = p8x.Step(stages)
    info = step.info()
    assert info["stages"] == len(stages) and info["grid"] >= 1
    assert info["class_set"] == (8 if mix == "c3" else 0xFE)
    first = None
    for rep in range(3):
        for b, _ in outs:   # poison the outputs (NaN bytes): the step must write every value
            b.fill(0xFF)
        step.run()
        step.check()
        got = read(outs)
        if first is None:
            first = got
        for i, (g, f) in enumerate(zip(got, first)):
            assert np.array_equal(g.view(np.uint32), f.view(np.uint32)), (mix, rep, i)   # deterministic
    for i, (g, w) in enumerate(zip(first, want)):
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (mix, i)
    if mix == "c3":
        check_against_oracle(first, x0h, hosts, head_hosts)
    # replays of one HIP graph capture, with eager runs and synchronizations between them
    st = p8x.Stream()
    graph = p8x.Graph(lambda s: step.run(s), st)
    for rep in range(3):
        for b, _ in outs:
            b.fill(0xFF)
        graph.launch(st)
        st.sync()
        step.check()
        got = read(outs)
        for i, (g, f) in enumerate(zip(got, first)):
            assert np.array_equal(g.view(np.uint32), f.view(np.uint32)), (mix, "replay", rep, i)
        step.run(st)
        st.sync()
    graph.release()
    step.release()


def test_step_rejects_mismatched_stage():
    L, head, _, _ = build(C3, layers=1)
    x0 = p8x.DeviceBuffer(4 * HIDDEN)
    q, k, v, o, gate, up, down = L[0]
    with pytest.raises(p8x.P8xError, match="K"):
        p8x.Step([([q, down], x0, [p8x.DeviceBuffer(4 * HIDDEN), p8x.DeviceBuffer(4 * HIDDEN)])])
    with pytest.raises(p8x.P8xError, match="swiglu"):
        p8x.Step([([gate], x0, None, p8x.DeviceBuffer(4 * FFN))])
    with pytest.raises(p8x.P8xError, match="twice"):
        p8x.Step([([gate, gate], x0, None, p8x.DeviceBuffer(4 * FFN))])


def test_step_keeps_stage_order_for_aliased_outputs():
    """A chain whose stage reads an output that a later stage writes again: the barrier orders the read before the
    write, so the results equal the per-node chain's."""
    L, head, _, _ = build(C3, layers=1)
    q, k, v, o, gate, up, down = L[0]
    rng = np.random.default_rng(2)
    xh = rng.standard_normal(HIDDEN).astype(np.float32)
    x0 = p8x.DeviceBuffer.from_numpy(xh)
    yq = p8x.DeviceBuffer(4 * HIDDEN)
    # stage 0 reads x0, stage 1 reads q's output and writes x0, stage 2 reads x0 again
    yk = p8x.DeviceBuffer(4 * 256)
    stages = [([q], x0, [yq]), ([o], yq, [x0]), ([k], x0, [yk])]
    run_per_node(stages)
    want = read([(yq, HIDDEN), (x0, HIDDEN), (yk, 256)])
    x0.copy_from(p8x.DeviceBuffer.from_numpy(xh))   # the per-node chain overwrote it
    step = p8x.Step(stages)
    step.run()
    step.check()
    got = read([(yq, HIDDEN), (x0, HIDDEN), (yk, 256)])
    for g, w in zip(got, want):
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32))
    step.release()


@pytest.mark.parametrize("act", [p8x.ACT_X16, p8x.ACT_Q8_1])
def test_step_chain_act(act):
    """x16 and block_q8_1 steps: every stage's output equals the per-node call of that mode bit for bit (poisoned
    outputs, consecutive runs, HIP graph replays), and each stage is within 1e-5 of the oracle's GEMV of that mode on
    the stage's input as the step wrote it"""
    name = "x16" if act == p8x.ACT_X16 else "q8_1"
    L, head, hosts, head_hosts = build(C3, layers=1, seed=300 + act)
    rng = np.random.default_rng(10 + act)
    x0h = rng.standard_normal(HIDDEN).astype(np.float32)
    x0 = p8x.DeviceBuffer.from_numpy(x0h)
    stages, outs = chain(L, head, x0)
    for st in stages:   # the per-node calls of this mode
        ts, x, ys = st[0], st[1], st[2]
        if len(st) > 3:
            p8x.mul_mat_vec_glu_dev(ts[0], ts[1], x, st[3], act=act)
        else:
            p8x.mul_mat_vec_multi_dev(ts, x, ys, act=act)
    p8x.synchronize()
    want = read(outs)
    step = p8x.Step(stages, act=act)
    info = step.info()
    assert info["stages"] == len(stages) and info["grid"] == 0 and info["class_set"] == 8
    st = p8x.Stream()
    graph = p8x.Graph(lambda s: step.run(s), st)
    for rep in range(3):
        for b, _ in outs:
            b.fill(0xFF)
        if rep == 1:
            graph.launch(st)
            st.sync()
        else:
            step.run()
            step.check()
        got = read(outs)
        for i, (g, w) in enumerate(zip(got, want)):
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (name, rep, i)
    graph.release()
    step.release()
    orc = [O.Oracle(s, r, K) for s, (r, K) in hosts[0]]
    orh = [O.Oracle(s, r, K) for s, (r, K) in head_hosts]
    yq, yk, yv, yo, yg, yd = want[:6]
    for y, o, nm in ((yq, orc[0], "q"), (yk, orc[1], "k"), (yv, orc[2], "v")):
        assert rel(y, o.gemv_f64(x0h, act=name)) < 1e-5, (name, nm)
    assert rel(yo, orc[3].gemv_f64(yq, act=name)) < 1e-5, (name, "o")
    g, u = orc[4].gemv_f64(yo, act=name), orc[5].gemv_f64(yo, act=name)
    assert rel(yg, g / (1.0 + np.exp(-g)) * u) < 1e-5, (name, "swiglu")
    assert rel(yd, orc[6].gemv_f64(yg, act=name)) < 1e-5, (name, "down")
    for i, o in enumerate(orh):
        assert rel(want[6 + i], o.gemv_f64(yd, act=name)) < 1e-5, (name, "head", i)
    for b, _ in outs:
        b.free()
    for t in [t for layer in L for t in layer] + head:
        t.release()
    x0.free()


def test_step_act_rejects_unknown_mode():
    L, head, _, _ = build(C3, layers=1, seed=400)
    x0 = p8x.DeviceBuffer.from_numpy(np.ones(HIDDEN, np.float32))
    stages, outs = chain(L, head, x0)
    with pytest.raises(p8x.P8xError, match="act 5"):
        p8x.Step(stages, act=5)
    for b, _ in outs:
        b.free()
    for t in [t for layer in L for t in layer] + head:
        t.release()
    x0.free()
