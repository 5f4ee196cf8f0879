"""Several linears on one activation vector in one launch (p8x_mul_mat_vec_multi: q/k/v, gate/up) and the gated
FFN input silu(gate x) * (up x) (p8x_mul_mat_vec_glu), against the fp64 oracle of each tensor on the same 8-bit
activations (bar 1e-3 relative L2, asserted at 1e-5), and the rejections of tensors that cannot share an input.
The same calls with the other activation modes (p8x_mul_mat_vec_multi_act / _glu_act: x16, the reference CPU path's
default, and block_q8_1) against the oracle's GEMV in that mode, and the grouped launch with x16 activations."""
import numpy as np
import pytest

import oracle as O
import p8x
import slotgen

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def shared_input(specs, seed):
    """slots for [(rows, K, class_p, nd)] with tensor 0's column scales c and Hadamard signs copied into the others
    (one input rotation, as a file encodes the linears that share an input)"""
    slots = [p8x.synth_random(seed + i, r, K, class_p=cp, nd=nd) for i, (r, K, cp, nd) in enumerate(specs)]
    r0, K0, _, nd0 = specs[0]
    o0 = slotgen.offsets(slots[0].size, r0, K0, nd0)
    c16, sg = slots[0][o0["C"]:o0["C"] + 2 * K0].copy(), slots[0][o0["SG"]:o0["SG"] + 256].copy()
    for s, (r, K, _, nd) in zip(slots[1:], specs[1:]):
        o = slotgen.offsets(s.size, r, K, nd)
        s[o["C"]:o["C"] + 2 * K] = c16
        s[o["SG"]:o["SG"] + 256] = sg
    return slots


C3 = (0, 0, 0, 1, 0, 0, 0, 0)
MIX = (0, 0, 1, 6, 1, 0, 1, 0)


@pytest.mark.parametrize("specs", [
    [(4096, 4096, C3, 3), (1024, 4096, C3, 1), (1024, 4096, (0, 0, 0, 0, 0, 0, 1, 0), 2)],   # Llama q / k / v
    [(4096, 2560, C3, 2), (1024, 2560, C3, 0), (1024, 2560, C3, 4)],                         # Qwen3-4B q / k / v
    [(512, 14336, MIX, 5), (256, 14336, MIX, 3)],                                           # long K: the K-split path
    [(96, 1024, (1, 1, 1, 1, 1, 1, 1, 1), 2), (64, 1024, C3, 1), (32, 1024, C3, 0), (128, 1024, MIX, 3)],
], ids=["llama_qkv", "qwen4b_qkv", "ksplit", "four_mixed"])
def test_multi_matches_oracle(specs):
    slots = shared_input(specs, 60)
    ts = [p8x.Tensor(s, r, K) for s, (r, K, _, _) in zip(slots, specs)]
    x = np.random.default_rng(61).standard_normal(specs[0][1]).astype(np.float32)
    for rep in range(2):
        ys = p8x.mul_mat_vec_multi(ts, x)
        for i, (s, (r, K, _, _)) in enumerate(zip(slots, specs)):
            assert rel_l2(ys[i], O.Oracle(s, r, K).gemv_f64(x)) < 1e-5, (rep, i)


def silu_up(g, u):
    return g / (1.0 + np.exp(-g)) * u


@pytest.mark.parametrize("rows,K,cp,nd", [(14336, 4096, C3, 6), (9728, 2560, C3, 3), (1024, 14336, MIX, 4), (96, 512, (1, 1, 1, 1, 1, 1, 1, 1), 2)],
                         ids=["llama_ffn", "qwen4b_ffn", "ksplit", "small_mixed"])
def test_glu_matches_oracle(rows, K, cp, nd):
    slots = shared_input([(rows, K, cp, nd), (rows, K, cp, nd + 1)], 70)
    gate, up = p8x.Tensor(slots[0], rows, K), p8x.Tensor(slots[1], rows, K)
    x = np.random.default_rng(71).standard_normal(K).astype(np.float32)
    ref = silu_up(O.Oracle(slots[0], rows, K).gemv_f64(x), O.Oracle(slots[1], rows, K).gemv_f64(x))
    first = None
    for rep in range(3):   # the per-row counters go back to 0: repeated calls agree bit for bit
        out = p8x.mul_mat_vec_glu(gate, up, x)
        assert rel_l2(out, ref) < 1e-5, rep
        if first is None:
            first = out
        else:
            assert np.array_equal(out.view(np.uint32), first.view(np.uint32)), rep


ACTS = [(p8x.ACT_X16, "x16"), (p8x.ACT_Q8_1, "q8_1")]


@pytest.mark.parametrize("act,name", ACTS, ids=[a[1] for a in ACTS])
@pytest.mark.parametrize("specs", [
    [(4096, 4096, C3, 3), (1024, 4096, C3, 1), (1024, 4096, (0, 0, 0, 0, 0, 0, 1, 0), 2)],   # Llama q / k / v
    [(512, 14336, MIX, 5), (256, 14336, MIX, 3)],                                           # long K: the K-split path
], ids=["llama_qkv", "ksplit"])
def test_multi_act_matches_oracle(specs, act, name):
    slots = shared_input(specs, 62)
    ts = [p8x.Tensor(s, r, K) for s, (r, K, _, _) in zip(slots, specs)]
    x = np.random.default_rng(63).standard_normal(specs[0][1]).astype(np.float32)
    for rep in range(2):
        ys = p8x.mul_mat_vec_multi(ts, x, act=act)
        for i, (s, (r, K, _, _)) in enumerate(zip(slots, specs)):
            orc = O.Oracle(s, r, K)
            assert rel_l2(ys[i], orc.gemv_f64(x, act=name)) < 1e-5, (rep, i)
            # the same values as the single call in that mode
            assert np.array_equal(ys[i].view(np.uint32), ts[i].mul_mat_vec(x, act=act)[0].view(np.uint32)), (rep, i)


@pytest.mark.parametrize("act,name", ACTS, ids=[a[1] for a in ACTS])
@pytest.mark.parametrize("rows,K,cp,nd", [(14336, 4096, C3, 6), (1024, 14336, MIX, 4)], ids=["llama_ffn", "ksplit"])
def test_glu_act_matches_oracle(rows, K, cp, nd, act, name):
    slots = shared_input([(rows, K, cp, nd), (rows, K, cp, nd + 1)], 72)
    gate, up = p8x.Tensor(slots[0], rows, K), p8x.Tensor(slots[1], rows, K)
    x = np.random.default_rng(73).standard_normal(K).astype(np.float32)
    ref = silu_up(O.Oracle(slots[0], rows, K).gemv_f64(x, act=name), O.Oracle(slots[1], rows, K).gemv_f64(x, act=name))
    first = None
    for rep in range(2):
        out = p8x.mul_mat_vec_glu(gate, up, x, act=act)
        assert rel_l2(out, ref) < 1e-5, rep
        if first is None:
            first = out
        else:
            assert np.array_equal(out.view(np.uint32), first.view(np.uint32)), rep


@pytest.mark.parametrize("ncols", [1, 2, 4])
def test_batch_x16_matches_oracle(ncols):
    """the grouped launch with x16 activations: a q/k/v group (one input), a long-K job (split along K by the plan)
    and a mixed-class job, ncols columns each; every column against the oracle's x16 GEMV"""
    specs = [(4096, 4096, C3, 3), (1024, 4096, C3, 1), (1024, 4096, (0, 0, 0, 0, 0, 0, 1, 0), 2)]
    slots = shared_input(specs, 64) + [p8x.synth_random(66, 512, 14336, class_p=MIX, nd=4), p8x.synth_random(67, 96, 1024, class_p=(1, 1, 1, 1, 1, 1, 1, 1), nd=2)]
    shapes = [(r, K) for r, K, _, _ in specs] + [(512, 14336), (96, 1024)]
    ts = [p8x.Tensor(s, r, K) for s, (r, K) in zip(slots, shapes)]
    rng = np.random.default_rng(65)
    xh = [rng.standard_normal((ncols, K)).astype(np.float32) for _, K in shapes]
    xs = [p8x.DeviceBuffer.from_numpy(x) for x in xh]
    ys = [p8x.DeviceBuffer(4 * ncols * r) for r, _ in shapes]
    b = p8x.GemvBatch(ts, xs, ys, ncols=ncols, act=p8x.ACT_X16)
    for rep in range(2):
        for y in ys:
            y.fill(0xFF)
        b.run()
        p8x.synchronize()
        for i, ((r, K), s) in enumerate(zip(shapes, slots)):
            got = ys[i].to_numpy(np.float32, (ncols, r))
            orc = O.Oracle(s, r, K)
            for n in range(ncols):
                assert rel_l2(got[n], orc.gemv_f64(xh[i][n], act="x16")) < 1e-5, (rep, i, n)
    b.release()


def test_multi_and_glu_reject_unshared_inputs():
    a, b = p8x.synth_random(80, 256, 1024), p8x.synth_random(81, 256, 1024)   # own c16 and signs each
    ta, tb = p8x.Tensor(a, 256, 1024), p8x.Tensor(b, 256, 1024)
    x = np.zeros(1024, np.float32)
    with pytest.raises(p8x.P8xError, match="rotates its input differently"):
        p8x.mul_mat_vec_multi([ta, tb], x)
    with pytest.raises(p8x.P8xError, match="rotates its input differently"):
        p8x.mul_mat_vec_glu(ta, tb, x)
    tc = p8x.Tensor(p8x.synth_random(82, 256, 2048), 256, 2048)
    with pytest.raises(p8x.P8xError, match="has K 2048"):
        p8x.mul_mat_vec_multi([ta, tc], x)
    s = shared_input([(256, 1024, C3, 0), (128, 1024, C3, 0)], 83)
    with pytest.raises(p8x.P8xError, match="rows"):
        p8x.mul_mat_vec_glu(p8x.Tensor(s[0], 256, 1024), p8x.Tensor(s[1], 128, 1024), x)


@pytest.mark.parametrize("act,name", ACTS, ids=[a[1] for a in ACTS])
def test_prepared_activation_reuse(act, name):
    """p8x_graph_begin: within one evaluation a call on the same input and rotation reuses the activation the previous
    call prepared (shown by changing x in place: the next call still sees the old x), a tensor with another rotation
    prepares its own, and the next p8x_graph_begin starts over. Every result equals the oracle on the x it used."""
    # no clamp deltas: those read the live x (as the reference's do), and the reuse shows in the rest of the row sum
    slots = shared_input([(1024, 4096, C3, 0), (512, 4096, C3, 0)], 90)
    ta, tb = p8x.Tensor(slots[0], 1024, 4096), p8x.Tensor(slots[1], 512, 4096)
    other = p8x.synth_random(92, 256, 4096, nd=1)   # its own column scales and signs
    tc = p8x.Tensor(other, 256, 4096)
    oa, ob, oc = O.Oracle(slots[0], 1024, 4096), O.Oracle(slots[1], 512, 4096), O.Oracle(other, 256, 4096)
    rng = np.random.default_rng(91)
    x1 = rng.standard_normal(4096).astype(np.float32)
    x2 = rng.standard_normal(4096).astype(np.float32)
    xd = p8x.DeviceBuffer.from_numpy(x1)
    ya, yb, yc = p8x.DeviceBuffer(4 * 1024), p8x.DeviceBuffer(4 * 512), p8x.DeviceBuffer(4 * 256)

    def run(t, y, n):
        t.mul_mat_vec_dev(xd, y, act=act)
        p8x.synchronize()
        return y.to_numpy(np.float32, (n,)).copy()

    p8x.graph_begin()
    a1 = run(ta, ya, 1024)
    b1 = run(tb, yb, 512)                      # reuses ta's prepared x1
    assert rel_l2(a1, oa.gemv_f64(x1, act=name)) < 1e-5
    assert rel_l2(b1, ob.gemv_f64(x1, act=name)) < 1e-5
    xd.copy_from(p8x.DeviceBuffer.from_numpy(x2))   # x changed in place, no new evaluation
    b2 = run(tb, yb, 512)
    assert np.array_equal(b2.view(np.uint32), b1.view(np.uint32))   # still x1's activation: reused
    c2 = run(tc, yc, 256)                      # another rotation: prepares x2 itself
    assert rel_l2(c2, oc.gemv_f64(x2, act=name)) < 1e-5
    p8x.graph_begin()
    b3 = run(tb, yb, 512)                      # a new evaluation: x2
    assert rel_l2(b3, ob.gemv_f64(x2, act=name)) < 1e-5
    # the reused result equals a call that prepares for itself
    p8x.graph_begin()
    xd.copy_from(p8x.DeviceBuffer.from_numpy(x1))
    b4 = run(tb, yb, 512)
    assert np.array_equal(b4.view(np.uint32), b1.view(np.uint32))
