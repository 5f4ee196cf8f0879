"""GPU parity of the HIP path against the oracle and the reference-core fixtures (run on an MI355X).

Bars: exact for decoded ints, dequantized f32 bits, activation ints/scales and integer dot partials;
fp32 GEMV outputs within 1e-3 relative L2 of the fp64 oracle that consumes the same 8-bit activations
(they agree to ~1e-7 in practice).
"""
import glob
import os

import numpy as np
import pytest

import oracle as O
import p8x

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
CASES = sorted(glob.glob(os.path.join(HERE, "golden", "case_*.npz")))
REL_L2 = 1e-3


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def load(path):
    z = np.load(path)
    c = {k: z[k] for k in z.files}
    c["rows"], c["K"] = int(c["rows"]), int(c["K"])
    return c


@pytest.fixture(scope="module", params=CASES, ids=[os.path.basename(c)[5:-4] for c in CASES])
def case(request):
    c = load(request.param)
    c["t"] = p8x.Tensor(c["slot"], c["rows"], c["K"])
    return c


def test_decode_ints_exact(case):
    ints = case["t"].decode_rotated(p8x.I16)
    assert np.array_equal(ints, case["ints"])


def test_decode_rotated_f32_exact(case):
    got = case["t"].decode_rotated(p8x.F32)
    rows, K = case["rows"], case["K"]
    nt = (rows // 32) * (K // 256)
    S = case["slot"][2064 + 4 * nt:2064 + 68 * nt].view(np.float16).astype(np.float32).reshape(K // 256, rows)
    ref = case["ints"].astype(np.float32) * np.repeat(S.T, 256, axis=1)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_f32_bit_exact(case):
    W = case["t"].dequantize(p8x.F32)
    assert np.array_equal(W.view(np.uint32), case["dequant"].view(np.uint32))


def test_dequant_f16_bf16_rounding(case):
    ref = case["dequant"]
    h = case["t"].dequantize(p8x.F16)
    assert np.array_equal(h, ref.astype(np.float16).view(np.uint16))
    b = case["t"].dequantize(p8x.BF16)
    u = ref.view(np.uint32).astype(np.uint64)
    rb = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    assert np.array_equal(b, rb)


def test_act_q8_128_exact(case):
    q, d, s = case["t"].quantize_q8_128(case["x"])
    assert np.array_equal(q[0], case["q8"])
    assert np.array_equal(d[0].view(np.uint32), case["q8_d"].view(np.uint32))
    assert np.array_equal(s[0], case["q8_sum"])


def test_act_q8_1_exact(case):
    orc = O.Oracle(case["slot"], case["rows"], case["K"])
    blk = case["t"].quantize_q8_1(case["x"])
    assert np.array_equal(blk[0], orc.quantize_q8_1(case["x"]))


def test_vec_dot_partials_exact(case):
    orc = O.Oracle(case["slot"], case["rows"], case["K"])
    q, d, _ = orc.prep_q8_128(case["x"])
    y, part = case["t"].vec_dot(p8x.ACT_Q8_128, q[None, :], d[None, :], partials=True)
    assert np.array_equal(part[0], orc.partials_q8_128(q))
    blk = orc.quantize_q8_1(case["x"])
    y1, part1 = case["t"].vec_dot(p8x.ACT_Q8_1, blk[None, :], None, partials=True)
    assert np.array_equal(part1[0], orc.partials_q8_1(blk))


def test_gemv_matches_fp64(case):
    orc = O.Oracle(case["slot"], case["rows"], case["K"])
    y = case["t"].mul_mat_vec(case["x"])[0]
    ref = orc.gemv_f64(case["x"])
    assert rel_l2(y, ref) < REL_L2
    assert rel_l2(y, ref) < 1e-5
    y1 = case["t"].mul_mat_vec(case["x"], act=p8x.ACT_Q8_1)[0]
    assert rel_l2(y1, orc.gemv_f64(case["x"], act="q8_1")) < 1e-5
    # and the reference core's own fp32 two-phase GEMV
    assert rel_l2(y, case["y_q8"]) < 1e-5


@pytest.mark.parametrize("ncols", [1, 2, 3, 4, 5, 6, 7, 8])
def test_gemv_multicolumn(ncols):
    rng = np.random.default_rng(100 + ncols)
    rows, K = 256, 2560
    slot = p8x.synth_random(ncols, rows, K, class_p=(1, 1, 1, 4, 1, 1, 1, 1), nd=6)
    t = p8x.Tensor(slot, rows, K)
    orc = O.Oracle(slot, rows, K)
    X = rng.standard_normal((ncols, K)).astype(np.float32)
    Y = t.mul_mat_vec(X)
    for n in range(ncols):
        assert rel_l2(Y[n], orc.gemv_f64(X[n])) < 1e-5, n


@pytest.mark.parametrize("rows,K,classes", [(4096, 4096, (3,)), (1024, 14336, (2, 3, 4)), (2048, 1024, tuple(range(8))),
                                            (512, 6144, (3,)), (256, 28672, (3, 6)), (64, 30720, (3,))])
def test_large_shapes(rows, K, classes):
    p = [0.0] * 8
    for c in classes:
        p[c] = 1.0
    slot = p8x.synth_random(rows + K, rows, K, class_p=p, nd=11)
    t = p8x.Tensor(slot, rows, K)
    orc = O.Oracle(slot, rows, K)
    x = np.random.default_rng(rows).standard_normal(K).astype(np.float32)
    y = t.mul_mat_vec(x)[0]
    assert rel_l2(y, orc.gemv_f64(x)) < 1e-5
    W = t.dequantize(p8x.F32)
    assert np.array_equal(W.view(np.uint32), orc.dequant().view(np.uint32))


def test_gemv_linear_in_x_exactly():
    """y(2x) == 2 y(x) bit for bit: quantization scales by exact powers of two (size-independent property)."""
    rows, K = 14336, 4096
    slot = p8x.synth_random(5, rows, K, nd=20)
    t = p8x.Tensor(slot, rows, K)
    x = np.random.default_rng(5).standard_normal(K).astype(np.float32)
    y1 = t.mul_mat_vec(x)[0]
    y2 = t.mul_mat_vec(2 * x)[0]
    assert np.array_equal((2 * y1).view(np.uint32), y2.view(np.uint32))


def test_gemv_deterministic():
    rows, K = 4096, 14336
    slot = p8x.synth_random(9, rows, K, nd=3)
    t = p8x.Tensor(slot, rows, K)
    x = np.random.default_rng(9).standard_normal((2, K)).astype(np.float32)
    a = t.mul_mat_vec(x)
    b = t.mul_mat_vec(x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_quantized_4096_config():
    """4096 x 4096, N(0, 0.02^2) with 0.1% outliers x10, through the class-3 quantizer; CPU dequant vs GPU; the GEMV
    with both activation formats the reference offers for it: 8 bits per 128 columns and ggml's block_q8_1 (blocks
    bit-exact, integer partials exact, the GEMV within the fp64 bar)."""
    rng = np.random.default_rng(2024)
    W = (rng.standard_normal((4096, 4096)) * 0.02).astype(np.float32)
    m = rng.random(W.shape) < 0.001
    W[m] *= 10
    slot = p8x.quantize_tensor(W, sign_seed=0)
    t = p8x.Tensor(slot, 4096, 4096)
    orc = O.Oracle(slot, 4096, 4096)
    Wd = t.dequantize(p8x.F32)
    assert np.array_equal(Wd.view(np.uint32), orc.dequant().view(np.uint32))
    x = rng.standard_normal(4096).astype(np.float32)
    assert rel_l2(t.mul_mat_vec(x)[0], orc.gemv_f64(x)) < 1e-5
    blk = t.quantize_q8_1(x)[0]
    assert np.array_equal(blk, orc.quantize_q8_1(x))
    _, part = t.vec_dot(p8x.ACT_Q8_1, blk[None, :], None, partials=True)
    assert np.array_equal(part[0], orc.partials_q8_1(blk))
    assert rel_l2(t.mul_mat_vec(x, act=p8x.ACT_Q8_1)[0], orc.gemv_f64(x, act="q8_1")) < 1e-5


def test_encoded_ldlq_slot_all_classes():
    """A 512 x 2048 slot from the host encoder with H-weighted feedback and allocated classes (mixed 0..7, sorted
    rows, clamp deltas): GPU decode and dequant bit-exact to the oracle, GEMV within the fp64 bar."""
    rng = np.random.default_rng(77)
    rows, K = 512, 2048
    W = (rng.standard_normal((rows, K)) * 0.02).astype(np.float32)
    W *= rng.lognormal(0, 1.0, rows).astype(np.float32)[:, None]      # row energies spread: classes 0..7 all used
    W[rng.random(W.shape) < 0.002] *= 12
    W[:4] = np.where(W[:4] > 0, 1, -1) * np.abs(W).max()            # |W| = max: overshoots become clamp deltas
    X = rng.standard_normal((2 * K, K)).astype(np.float32)
    X[:, 1:] += 0.8 * X[:, :-1]
    H = (X.T @ X / X.shape[0]).astype(np.float32)
    c16 = rng.uniform(0.6, 1.8, K).astype(np.float16).view(np.uint16)
    slot = p8x.encode_tensor(W, c16=c16, H=H, bits_per_weight=2.5, n_salient=8, sign_seed=5)
    t = p8x.Tensor(slot, rows, K)
    info = t.info
    assert sum(1 for c in range(8) if info.class_tiles[c]) >= 6, list(info.class_tiles)
    orc = O.Oracle(slot, rows, K)
    assert orc.nd > 0
    assert np.array_equal(t.decode_rotated(p8x.I16), orc.decode_all())
    assert np.array_equal(t.dequantize(p8x.F32).view(np.uint32), orc.dequant().view(np.uint32))
    x = rng.standard_normal(K).astype(np.float32)
    assert rel_l2(t.mul_mat_vec(x)[0], orc.gemv_f64(x)) < REL_L2


@pytest.mark.parametrize("tables", ["shipped", "random", "wrapping"])
def test_dequant_classes_0_to_3(tables):
    """tensors of classes 0-3 only (the integer-butterfly dequantizer): f32 bit-exact to the oracle, f16 / bf16 its
    RNE roundings, with clamp deltas, permuted rows, any int8 codebook (wrapping A + c included) and row ranges"""
    import slotgen
    rng = np.random.default_rng({"shipped": 1, "random": 2, "wrapping": 3}[tables])
    rows, K = 256, 2048
    slot = slotgen.random_slot(rng, rows, K, classes=(0, 1, 2, 3), class_p=(0.1, 0.2, 0.2, 0.5), tables=tables, nd=40)
    t = p8x.Tensor(slot, rows, K)
    W = O.Oracle(slot, rows, K).dequant()
    got = t.dequantize(p8x.F32)
    assert np.array_equal(got.view(np.uint32), W.view(np.uint32))
    assert np.array_equal(t.dequantize(p8x.F16), W.astype(np.float16).view(np.uint16))
    u = W.view(np.uint32).astype(np.uint64)
    assert np.array_equal(t.dequantize(p8x.BF16), ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16))
    for row0, nrows in ((0, 1), (77, 50), (255, 1)):
        r = t.dequantize_rows(row0, nrows, ld=K + 32)
        assert np.array_equal(r[:, :K].view(np.uint32), W[row0:row0 + nrows].view(np.uint32)), (row0, nrows)
        assert not r[:, K:].any()


def test_dequant_class3_ffn_shape():
    """the benchmarked 14336 x 4096 class-3 tensor with clamp deltas, f16 against the oracle's f32 rounded"""
    rows, K = 14336, 4096
    slot = p8x.synth_random(rows + K, rows, K, nd=8)
    t = p8x.Tensor(slot, rows, K)
    W = O.Oracle(slot, rows, K).dequant()
    assert np.array_equal(t.dequantize(p8x.F16), W.astype(np.float16).view(np.uint16))


def test_prepare_rejects_bad_slots():
    rng = np.random.default_rng(3)
    import slotgen
    buf = slotgen.random_slot(rng, 64, 512, classes=(3,), nd=1)
    p8x.Tensor(buf, 64, 512).release()
    bad = buf.copy(); bad[-32] ^= 1
    with pytest.raises(p8x.P8xError, match="contract"):
        p8x.Tensor(bad, 64, 512)
    with pytest.raises(p8x.P8xError, match="invalid argument"):
        p8x.Tensor(buf, 64, 500)
    # device-resident slot
    dev = p8x.DeviceBuffer.from_numpy(buf)
    t = p8x.Tensor(None, 64, 512, device_slot=dev)
    assert np.array_equal(t.decode_rotated(p8x.I16), O.Oracle(buf, 64, 512).decode_all())


@pytest.mark.parametrize("ncols", [1, 3, 8])
def test_batch_matches_single(ncols):
    """one grouped launch over mixed shapes and class mixes == fp64 oracle per job"""
    shapes = [(1024, 4096, (0, 0, 0, 1, 0, 0, 0, 0)), (512, 14336, (0, 0, 1, 8, 1, 0, 0, 0)),
              (2048, 2560, (0, 0, 0, 0, 0, 0, 1, 0)), (96, 768, (1, 1, 1, 1, 1, 1, 1, 1))]
    rng = np.random.default_rng(40 + ncols)
    tensors, orcs, xs, ys, hx = [], [], [], [], []
    for i, (rows, K, cp) in enumerate(shapes):
        slot = p8x.synth_random(77 + i, rows, K, class_p=cp, nd=3)
        tensors.append(p8x.Tensor(slot, rows, K))
        orcs.append(O.Oracle(slot, rows, K))
        X = rng.standard_normal((ncols, K)).astype(np.float32)
        hx.append(X)
        xs.append(p8x.DeviceBuffer.from_numpy(X))
        ys.append(p8x.DeviceBuffer(4 * ncols * rows))
    batch = p8x.GemvBatch(tensors, xs, ys, ncols=ncols)
    for rep in range(2):
        batch.run()
        p8x.synchronize()
        for i, (rows, K, _) in enumerate(shapes):
            Y = ys[i].to_numpy(np.float32, (ncols, rows))
            for n in range(ncols):
                assert rel_l2(Y[n], orcs[i].gemv_f64(hx[i][n])) < 1e-5, (i, n, rep)


@pytest.mark.parametrize("ncols", [1, 2])
def test_batch_timed_stages_match_run(ncols):
    """p8x_gemv_batch_run_stage_timed: the three stages with kernel-attached events give the bits of
    p8x_gemv_batch_run, and each event pair spans a positive time no longer than the whole step"""
    shapes = [(1024, 4096), (4096, 1024), (256, 14336)]
    rng = np.random.default_rng(60 + ncols)
    tensors, xs, ys = [], [], []
    for i, (rows, K) in enumerate(shapes):
        tensors.append(p8x.Tensor(p8x.synth_random(90 + i, rows, K, nd=2), rows, K))
        xs.append(p8x.DeviceBuffer.from_numpy(rng.standard_normal((ncols, K)).astype(np.float32)))
        ys.append(p8x.DeviceBuffer(4 * ncols * rows))
    batch = p8x.GemvBatch(tensors, xs, ys, ncols=ncols)
    stream = p8x.Stream()
    batch.run(stream)
    stream.sync()
    want = [y.to_numpy(np.float32, (ncols * r,)).copy() for y, (r, _) in zip(ys, shapes)]
    for y in ys:
        y.fill(0xFF)
    ev = [(p8x.Event(), p8x.Event()) for _ in range(3)]
    a, b = p8x.Event(), p8x.Event()
    a.record(stream)
    for stage in range(3):
        batch.run_stage(stage, stream, events=ev[stage])
    b.record(stream)
    stream.sync()
    for y, w, (r, _) in zip(ys, want, shapes):
        assert np.array_equal(y.to_numpy(np.float32, (ncols * r,)).view(np.uint32), w.view(np.uint32))
    whole = a.elapsed_ms(b)
    for s, t in ev:
        assert 0.0 < s.elapsed_ms(t) <= whole
    batch.release()


@pytest.mark.parametrize("one_block", [False, True])
@pytest.mark.parametrize("cp", [(0, 0, 0, 1, 0, 0, 0, 0), (0, 0, 0, 0, 0, 0, 1, 0), (0, 0, 1, 6, 1, 0, 0, 0)])
def test_batch_one_column_class_sets(cp, one_block):
    """one-column grouped launches per class set (class 3, class 6, classes 2-4): units of unequal length (split
    along K at the end), three runs in a row (the unit counters reset themselves), bitwise equal runs, fp64 oracle
    per job, with and without one-block units."""
    shapes = [(2048, 4096), (512, 4096), (1024, 14336), (64, 2560)] + ([(96, 256)] if one_block else [])
    rng = np.random.default_rng(sum(cp))
    tensors, orcs, xs, ys, hx = [], [], [], [], []
    for i, (rows, K) in enumerate(shapes):
        slot = p8x.synth_random(500 + i, rows, K, class_p=cp, nd=2)
        tensors.append(p8x.Tensor(slot, rows, K))
        orcs.append(O.Oracle(slot, rows, K))
        X = rng.standard_normal((1, K)).astype(np.float32)
        hx.append(X)
        xs.append(p8x.DeviceBuffer.from_numpy(X))
        ys.append(p8x.DeviceBuffer(4 * rows))
    batch = p8x.GemvBatch(tensors, xs, ys, ncols=1)
    first = None
    for rep in range(3):
        for y in ys:
            y.fill(0)
        batch.run()
        p8x.synchronize()
        out = [y.to_numpy(np.float32, (rows,)) for y, (rows, _) in zip(ys, shapes)]
        if first is None:
            first = out
            for i in range(len(shapes)):
                assert rel_l2(out[i], orcs[i].gemv_f64(hx[i][0])) < 1e-5, i
        else:
            for a, c in zip(first, out):
                assert np.array_equal(a.view(np.uint32), c.view(np.uint32)), rep


def test_batch_fewer_units_than_waves():
    """a grouped launch with 3 row groups in all: most waves find no unit and leave; a second run still works"""
    slot = p8x.synth_random(901, 96, 512, class_p=(0, 0, 0, 1, 0, 0, 0, 0), nd=1)
    t = p8x.Tensor(slot, 96, 512)
    orc = O.Oracle(slot, 96, 512)
    X = np.random.default_rng(901).standard_normal((1, 512)).astype(np.float32)
    x = p8x.DeviceBuffer.from_numpy(X)
    y = p8x.DeviceBuffer(4 * 96)
    batch = p8x.GemvBatch([t], [x], [y], ncols=1)
    for rep in range(2):
        y.fill(0)
        batch.run()
        p8x.synchronize()
        assert rel_l2(y.to_numpy(np.float32, (96,)), orc.gemv_f64(X[0])) < 1e-5, rep


@pytest.mark.parametrize("cp", [(1, 0, 0, 1, 0, 0, 0, 0), (1, 0, 1, 6, 1, 0, 1, 0), (0, 0, 1, 6, 1, 0, 1, 0)])
def test_class_zero_tiles_and_mixed_sets(cp):
    """tensors with all-zero (class 0) tiles among class-3 tiles, and the classes 2-4 + 6 set: single calls
    (one and three columns) and a grouped launch against the fp64 oracle"""
    rows, K = 512, 4096
    slot = p8x.synth_random(808, rows, K, class_p=cp, nd=5)
    t = p8x.Tensor(slot, rows, K)
    orc = O.Oracle(slot, rows, K)
    rng = np.random.default_rng(9)
    X = rng.standard_normal((3, K)).astype(np.float32)
    assert rel_l2(t.mul_mat_vec(X[0])[0], orc.gemv_f64(X[0])) < 1e-5
    Y = t.mul_mat_vec(X)
    for n in range(3):
        assert rel_l2(Y[n], orc.gemv_f64(X[n])) < 1e-5, n
    for ncols in (1, 2):
        xb = p8x.DeviceBuffer.from_numpy(X[:ncols].copy())
        yb = p8x.DeviceBuffer(4 * ncols * rows)
        batch = p8x.GemvBatch([t], [xb], [yb], ncols=ncols)
        batch.run()
        p8x.synchronize()
        Yb = yb.to_numpy(np.float32, (ncols, rows))
        for n in range(ncols):
            assert rel_l2(Yb[n], orc.gemv_f64(X[n])) < 1e-5, (ncols, n)
        batch.release()


@pytest.mark.parametrize("rows,K,cp,ncols", [(1024, 14336, (0, 0, 0, 1, 0, 0, 0, 0), 2), (1024, 14336, (0, 0, 0, 1, 0, 0, 0, 0), 3),
                                             (1024, 14336, (0, 0, 0, 1, 0, 0, 0, 0), 8), (2048, 4096, (0, 0, 0, 1, 0, 0, 0, 0), 2),
                                             (512, 8192, (0, 0, 0, 0, 0, 0, 1, 0), 2), (256, 30720, (0, 0, 0, 1, 0, 0, 0, 0), 1),
                                             (512, 4096, (0, 0, 0, 0, 0, 0, 1, 0), 4), (256, 28672, (0, 0, 0, 1, 0, 0, 0, 0), 7),
                                             (32, 8192, (0, 0, 0, 1, 0, 0, 0, 0), 1), (32, 8192, (0, 0, 0, 1, 0, 0, 0, 0), 2),
                                             (32, 256, (0, 0, 0, 1, 0, 0, 0, 0), 2), (32, 256, (0, 0, 0, 1, 0, 0, 0, 0), 1)])
def test_single_call_columns_row_group_kernel(rows, K, cp, ncols):
    """single calls on one-class tensors: two columns with K <= 8192 and one column of any K (K-chunks past 112
    blocks) run the row-group kernel, the others the multi-column task kernel; all against fp64"""
    slot = p8x.synth_random(rows * 7 + K, rows, K, class_p=cp, nd=6)
    t = p8x.Tensor(slot, rows, K)
    orc = O.Oracle(slot, rows, K)
    X = np.random.default_rng(ncols).standard_normal((ncols, K)).astype(np.float32)
    for rep in range(2):   # the K-chunk arrival counters are put back for the next call
        Y = t.mul_mat_vec(X)
        for n in range(ncols):
            assert rel_l2(Y[n], orc.gemv_f64(X[n])) < 1e-5, (rep, n)


@pytest.mark.parametrize("rows,K,cp", [(9728, 512, (0, 0, 0, 1, 0, 0, 0, 0)), (24576, 256, (0, 0, 0, 1, 0, 0, 0, 0)),
                                       (32000, 512, (1, 1, 1, 1, 1, 1, 1, 1))])
def test_single_call_many_row_groups(rows, K, cp):
    """more row groups than CUs: a workgroup streams 2-4 row groups at once (teams of waves); one and two columns"""
    slot = p8x.synth_random(rows + 3 * K, rows, K, class_p=cp, nd=9)
    t = p8x.Tensor(slot, rows, K)
    orc = O.Oracle(slot, rows, K)
    X = np.random.default_rng(rows).standard_normal((2, K)).astype(np.float32)
    assert rel_l2(t.mul_mat_vec(X[0])[0], orc.gemv_f64(X[0])) < 1e-5
    Y = t.mul_mat_vec(X)
    for n in range(2):
        assert rel_l2(Y[n], orc.gemv_f64(X[n])) < 1e-5, n


def test_activation_ties_match_oracle():
    """x' exactly on k + 1/2 with d = 1: block_q8_1 rounds half away from zero (+-(k+1)) and stores s = d * sum q;
    the 8-bit-per-128 prep rounds half to even (+-k) like the reference core; GPU blocks bitwise equal to the oracle"""
    import slotgen
    buf, x, k = slotgen.tie_case(np.random.default_rng(12), K=512, k=2)
    t = p8x.Tensor(buf, 32, 512)
    orc = O.Oracle(buf, 32, 512)
    blk = t.quantize_q8_1(x)[0]
    assert np.array_equal(blk, orc.quantize_q8_1(x))
    q = blk.reshape(-1, 36)[:, 4:].view(np.int8)
    assert np.all(q[:8, 1::2] == k + 1) and np.all(q[8:16, 1::2] == -(k + 1))
    q8, d8, s8 = t.quantize_q8_128(x)
    oq, od, osx = orc.prep_q8_128(x)
    assert np.array_equal(q8[0], oq) and np.array_equal(d8[0], od) and np.array_equal(s8[0], osx)
    assert np.all(q8[0][1:256:2] == k) and np.all(q8[0][257:512:2] == -k)
    # the products on these activations
    assert rel_l2(t.mul_mat_vec(x)[0], orc.gemv_f64(x)) < 1e-5
    assert rel_l2(t.mul_mat_vec(x, act=p8x.ACT_Q8_1)[0], orc.gemv_f64(x, act="q8_1")) < 1e-5


def test_wrapping_codebook():
    """a codebook whose A + c leaves the int8 range: every kernel decodes through the bytewise (wrapping) coset add
    of the reference CPU core, so ints, dequantized bits, GEMV and GEMM agree with the oracle"""
    import slotgen
    rng = np.random.default_rng(14)
    rows, K = 256, 2048
    buf = slotgen.random_slot(rng, rows, K, classes=(1, 2, 3, 4, 5, 6, 7), tables="wrapping", nd=4)
    t = p8x.Tensor(buf, rows, K)
    orc = O.Oracle(buf, rows, K)
    assert np.array_equal(t.decode_rotated(p8x.I16), orc.decode_all())
    W = orc.dequant()
    assert np.array_equal(t.dequantize(p8x.F32).view(np.uint32), W.view(np.uint32))
    X = rng.standard_normal((3, K)).astype(np.float32)
    Y = t.mul_mat_vec(X)
    for n in range(3):
        assert rel_l2(Y[n], orc.gemv_f64(X[n])) < 1e-5, n
    Xm = rng.standard_normal((40, K)).astype(np.float32)
    assert rel_l2(t.mul_mat(Xm, p8x.F32), O.dense_f64(W, Xm)) < 1e-3


def test_act_x16_exact(case):
    """x16 planes bit-exact to the reference core's vrc_prep_block16 (fixtures)"""
    qh, dh, sh, ql, dl, sl = case["t"].quantize_x16(case["x"])
    assert np.array_equal(qh[0], case["x16_hi"]) and np.array_equal(ql[0], case["x16_lo"])
    assert np.array_equal(dh[0].view(np.uint32), case["x16_hi_d"].view(np.uint32))
    assert np.array_equal(dl[0].view(np.uint32), case["x16_lo_d"].view(np.uint32))
    assert np.array_equal(sh[0], case["x16_hi_sum"]) and np.array_equal(sl[0], case["x16_lo_sum"])


def test_gemv_x16(case):
    """x16 products against the fp64 oracle on the same planes and the reference core's own x16 GEMV"""
    orc = O.Oracle(case["slot"], case["rows"], case["K"])
    y = case["t"].mul_mat_vec(case["x"], act=p8x.ACT_X16)[0]
    assert rel_l2(y, orc.gemv_f64(case["x"], act="x16")) < 1e-5
    assert rel_l2(y, case["y_x16"]) < 1e-5


@pytest.mark.parametrize("rows,K,ncols", [(256, 2560, 1), (256, 2560, 2), (256, 2560, 3), (256, 2560, 4), (4096, 14336, 1),
                                          (14336, 4096, 2)])
def test_gemv_x16_columns_and_shapes(rows, K, ncols):
    slot = p8x.synth_random(rows + ncols, rows, K, class_p=(1, 1, 1, 4, 1, 1, 1, 1) if rows == 256 else (0, 0, 0, 1, 0, 0, 0, 0), nd=6)
    t = p8x.Tensor(slot, rows, K)
    orc = O.Oracle(slot, rows, K)
    X = np.random.default_rng(ncols).standard_normal((ncols, K)).astype(np.float32)
    Y = t.mul_mat_vec(X, act=p8x.ACT_X16)
    for n in range(ncols):
        assert rel_l2(Y[n], orc.gemv_f64(X[n], act="x16")) < 1e-5, n
    with pytest.raises(p8x.P8xError, match="x16 takes at most 4"):
        t.mul_mat_vec(np.zeros((5, K), np.float32), act=p8x.ACT_X16)


@pytest.mark.parametrize("permute", [True, False])
def test_tile_and_row_ranges(permute):
    """the per-tile / per-row forms: decode_tiles windows and single tiles bit-exact to the oracle's tile decode,
    dequantize_rows bit-exact to the oracle's rows (identity and permuted rows), vec_dot_rows equal to the whole
    call on those rows with exact partials"""
    rows, K = 512, 2048
    slot = p8x.synth_random(900 + permute, rows, K, class_p=(1, 1, 1, 4, 1, 1, 1, 1), nd=9, permute=permute)
    t = p8x.Tensor(slot, rows, K)
    orc = O.Oracle(slot, rows, K)
    ints = orc.decode_all()
    for g0, ng, b0, nb in ((0, 1, 0, 1), (3, 1, 5, 1), (2, 5, 1, 3), (0, 16, 0, 8), (15, 1, 7, 1)):
        got = t.decode_tiles(g0, ng, b0, nb)
        assert np.array_equal(got, ints[32 * g0:32 * (g0 + ng), 256 * b0:256 * (b0 + nb)]), (g0, ng, b0, nb)
    assert np.array_equal(t.decode_tiles(4, 1, 2, 1), orc.decode_tile(4, 2))
    W = orc.dequant()
    for row0, nrows in ((0, rows), (0, 1), (37, 1), (100, 57), (480, 32), (511, 1)):
        got = t.dequantize_rows(row0, nrows, ld=K + 64)
        assert np.array_equal(got[:, :K].view(np.uint32), W[row0:row0 + nrows].view(np.uint32)), (row0, nrows)
        assert not got[:, K:].any()   # only the K columns are written
    h = t.dequantize_rows(200, 40, dtype=p8x.F16)
    assert np.array_equal(h, W[200:240].astype(np.float16).view(np.uint16))
    x = np.random.default_rng(5).standard_normal((2, K)).astype(np.float32)
    q = np.stack([orc.prep_q8_128(x[n])[0] for n in range(2)])
    d = np.stack([orc.prep_q8_128(x[n])[1] for n in range(2)])
    yall, pall = t.vec_dot(p8x.ACT_Q8_128, q, d, partials=True)
    prm = np.frombuffer(slot[slotgen_offsets(slot, rows, K)["P"]:][:2 * rows].tobytes(), np.int16)
    for g0, ng in ((0, 16), (3, 2), (15, 1)):
        y, part = t.vec_dot_rows(p8x.ACT_Q8_128, q, d, g0, ng)
        orig = prm[32 * g0:32 * (g0 + ng)]
        assert np.array_equal(y[:, orig].view(np.uint32), yall[:, orig].view(np.uint32)), (g0, ng)
        others = np.setdiff1d(np.arange(rows), orig)
        assert np.isnan(y[:, others]).all()
        assert np.array_equal(part, pall[:, 32 * g0:32 * (g0 + ng)]), (g0, ng)
    blk = orc.quantize_q8_1(x[0])
    y1, p1 = t.vec_dot_rows(p8x.ACT_Q8_1, blk[None, :], None, 6, 3)
    assert np.array_equal(p1[0], orc.partials_q8_1(blk)[192:288])


def slotgen_offsets(slot, rows, K):
    import slotgen
    nd = int(np.frombuffer(slot[-32:].tobytes(), np.uint32)[3])
    return slotgen.offsets(slot.size, rows, K, nd)


@pytest.mark.parametrize("cls", [3, 6])
def test_one_class_tiles_out_of_order(cls):
    """A one-class tensor whose tiles lie in D out of (row group, block) order: the one-class kernels compute payload
    offsets, so the host must route it to the kernels that read the tile words. Same tensor stored both ways: equal
    results (single calls, two columns, several linears in one launch, swiglu, dequantize) and the fp64 oracle."""
    import slotgen
    rng = np.random.default_rng(90 + cls)
    rows, K = 256, 8192   # 8 row groups, 32 blocks: the single call splits K in two (pair meet)
    slot = slotgen.random_slot(rng, rows, K, classes=(cls,), nd=3)
    shuf = slotgen.shuffle_tiles(slot, rows, K, rng)
    assert not np.array_equal(shuf, slot)
    t_in, t_sh = p8x.Tensor(slot, rows, K), p8x.Tensor(shuf, rows, K)
    orc = O.Oracle(shuf, rows, K)
    X = rng.standard_normal((2, K)).astype(np.float32)
    y_in, y_sh = t_in.mul_mat_vec(X[0])[0], t_sh.mul_mat_vec(X[0])[0]
    assert rel_l2(y_sh, orc.gemv_f64(X[0])) < REL_L2
    assert np.array_equal(y_sh, y_in)
    Y = t_sh.mul_mat_vec(X)
    for n in range(2):
        assert rel_l2(Y[n], orc.gemv_f64(X[n])) < REL_L2
    a, b = p8x.mul_mat_vec_multi([t_in, t_sh], X[0])
    assert np.array_equal(a, y_in) and np.array_equal(b, y_sh)
    g = p8x.mul_mat_vec_glu(t_in, t_sh, X[0])
    ref = (y_in.astype(np.float64) / (1.0 + np.exp(-y_in.astype(np.float64)))) * y_sh
    assert rel_l2(g, ref) < 1e-6
    assert np.array_equal(t_sh.dequantize(p8x.F32).view(np.uint32), t_in.dequantize(p8x.F32).view(np.uint32))
