"""Pins the CPU oracle (oracle/p8x_oracle.c) before anything is compared against it.

Each check is chosen so that a plausible slip (dropped term, wrong sign or index, transposed operand)
fails: golden fixtures written by the reference's own CPU core, closed forms, an independent bit-by-bit
decoder, brute force on small inputs.
"""
import glob
import os

import numpy as np
import pytest

import oracle as O
import slotgen

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = sorted(glob.glob(os.path.join(HERE, "golden", "case_*.npz")))


def load(path):
    z = np.load(path)
    return {k: z[k] for k in z.files}


@pytest.fixture(scope="module", params=CASES, ids=[os.path.basename(c)[5:-4] for c in CASES])
def case(request):
    c = load(request.param)
    c["rows"], c["K"] = int(c["rows"]), int(c["K"])
    c["orc"] = O.Oracle(c["slot"], c["rows"], c["K"])
    return c


def test_fixtures_present():
    assert len(CASES) == 9
    tab = np.fromfile(os.path.join(HERE, "golden", "tables_vrc.bin"), np.int8)
    assert tab.size == 1028
    # the shipped coset vector, as the reference runtime log prints it ("c = ebf9fcfe")
    assert tab[1024:].view(np.uint32)[0] == 0xEBF9FCFE
    A = tab[:1024].reshape(256, 4).astype(int)
    assert A.min() >= -64 and A.max() <= 64
    s = A + tab[1024:].astype(int)[None, :]
    assert s.min() >= -128 and s.max() <= 127  # A + c never wraps in int8


def test_trellis_exhaustive_16bit():
    for z in range(1 << 16):
        assert O.trellis_word(z) == O.trellis_serial(z)


def test_trellis_random_words():
    rng = np.random.default_rng(0)
    for z in rng.integers(0, 1 << 32, 20000, dtype=np.uint64):
        assert O.trellis_word(int(z)) == O.trellis_serial(int(z))


def test_trellis_known_values():
    # single label at t = 0: u = 1 + x + x^2 + x^4 + x^7 + ... (inverse of 1 + x + x^3), h = u << 2
    u = [0] * 32
    for t in range(32):
        u[t] = (1 if t == 0 else 0) ^ (u[t - 1] if t >= 1 else 0) ^ (u[t - 3] if t >= 3 else 0)
    h = sum(u[t - 2] << t for t in range(2, 32))
    assert O.trellis_word(1) == h
    assert O.trellis_word(0) == 0


def test_fwht_matches_hadamard():
    from scipy.linalg import hadamard
    H = hadamard(256).astype(np.float64)
    rng = np.random.default_rng(1)
    v = rng.standard_normal(256).astype(np.float32)
    got = O.fwht256(v)
    ref = H @ v.astype(np.float64) / 16.0
    assert np.allclose(got, ref, rtol=0, atol=1e-5)
    back = O.fwht256(got)  # H H = 256 I
    assert np.allclose(back, v, atol=1e-5)


def test_decode_matches_reference_fixture(case):
    ints = case["orc"].decode_all()
    assert np.array_equal(ints, case["ints"])


def test_bitwise_decoder_matches(case):
    orc = case["orc"]
    rng = np.random.default_rng(7)
    R = rng.integers(0, case["rows"], 400)
    C = rng.integers(0, case["K"], 400)
    for r, c in zip(R, C):
        assert orc.weight_int(int(r), int(c)) == int(case["ints"][r, c])


def test_dequant_bit_exact(case):
    W = case["orc"].dequant()
    assert np.array_equal(W.view(np.uint32), case["dequant"].view(np.uint32))


def test_prep_q8_bit_exact(case):
    q, d, sx = case["orc"].prep_q8_128(case["x"])
    assert np.array_equal(q, case["q8"])
    assert np.array_equal(d.view(np.uint32), case["q8_d"].view(np.uint32))
    assert np.array_equal(sx, case["q8_sum"])


def test_prep_x16_bit_exact(case):
    qh, dh, sh, ql, dl, sl = case["orc"].prep_x16(case["x"])
    assert np.array_equal(qh, case["x16_hi"]) and np.array_equal(ql, case["x16_lo"])
    assert np.array_equal(dh.view(np.uint32), case["x16_hi_d"].view(np.uint32))
    assert np.array_equal(dl.view(np.uint32), case["x16_lo_d"].view(np.uint32))
    assert np.array_equal(sh, case["x16_hi_sum"]) and np.array_equal(sl, case["x16_lo_sum"])


def test_gemv_x16_f64_matches_reference_gemv(case):
    """fp64 GEMV on the x16 planes vs the reference core's own fp32 two-phase GEMV in its x16 mode (y_x16), and a
    negative control: the q8 GEMV differs from y_x16 by far more (the modes quantize the activations differently)"""
    y = case["orc"].gemv_f64(case["x"], act="x16")
    ref = case["y_x16"].astype(np.float64)
    rel = np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30)
    assert rel < 1e-5, rel
    y8 = case["orc"].gemv_f64(case["x"])
    assert np.linalg.norm(y8 - ref) / np.linalg.norm(ref) > 10 * rel


def test_partials_are_integer_matmul(case):
    orc = case["orc"]
    q, d, sx = orc.prep_q8_128(case["x"])
    isum = orc.partials_q8_128(q)
    ints = case["ints"].astype(np.int64).reshape(case["rows"], -1, 128)
    ref = np.einsum("rsk,sk->rs", ints, q.astype(np.int64).reshape(-1, 128))
    assert np.array_equal(isum.astype(np.int64), ref)


def test_gemv_f64_matches_reference_gemv(case):
    """fp64 GEMV of the oracle vs the reference's own fp32 two-phase GEMV (rounding-level agreement)."""
    y = case["orc"].gemv_f64(case["x"])
    ref = case["y_q8"].astype(np.float64)
    rel = np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30)
    assert rel < 2e-6, rel


def test_gemv_f64_closed_form(case):
    """y = Sigma_s S * d_s * (ints . q) in original rows + delta . x, restated with numpy."""
    orc = case["orc"]
    rows, K = case["rows"], case["K"]
    q, d, _ = orc.prep_q8_128(case["x"])
    ints = case["ints"].astype(np.float64)
    buf = case["slot"]
    nt = (rows // 32) * (K // 256)
    S = buf[2064 + 4 * nt:2064 + 68 * nt].view(np.float16).astype(np.float64).reshape(K // 256, rows)
    scale = np.repeat(S.T, 256, axis=1) * np.repeat(d.astype(np.float64), 128)[None, :]
    ysorted = (ints * scale) @ q.astype(np.float64)
    o = slotgen.offsets(buf.size, rows, K, orc.nd)
    prm = buf[o["P"]:o["P"] + 2 * rows].view(np.int16).astype(np.int64)
    y = np.zeros(rows)
    y[prm] = ysorted
    if orc.nd:
        dr = buf[o["E"]:o["E"] + 2 * orc.nd].view(np.uint16).astype(np.int64)
        dc = buf[o["E"] + 2 * orc.nd:o["E"] + 4 * orc.nd].view(np.uint16).astype(np.int64)
        dv = buf[o["E"] + 4 * orc.nd:o["E"] + 8 * orc.nd].view(np.float32).astype(np.float64)
        np.add.at(y, dr, dv * case["x"][dc].astype(np.float64))
    got = orc.gemv_f64(case["x"])
    assert np.allclose(got, y, rtol=1e-12, atol=1e-12)


def test_dequant_is_rotated_ints_closed_form(case):
    """W[prm[r]] = (H256(ints * S) / 16) * sg / c + delta, restated in fp64."""
    from scipy.linalg import hadamard
    H = hadamard(256).astype(np.float64)
    orc = case["orc"]
    rows, K = case["rows"], case["K"]
    buf = case["slot"]
    nt = (rows // 32) * (K // 256)
    S = buf[2064 + 4 * nt:2064 + 68 * nt].view(np.float16).astype(np.float64).reshape(K // 256, rows)
    rot = case["ints"].astype(np.float64) * np.repeat(S.T, 256, axis=1)
    o = slotgen.offsets(buf.size, rows, K, orc.nd)
    c16 = buf[o["C"]:o["C"] + 2 * K].view(np.float16).astype(np.float64)
    sg = buf[o["SG"]:o["SG"] + 256].view(np.int8).astype(np.float64)
    prm = buf[o["P"]:o["P"] + 2 * rows].view(np.int16).astype(np.int64)
    Wsorted = (rot.reshape(rows, -1, 256) @ H / 16.0).reshape(rows, K) * np.tile(sg, K // 256)[None, :] / c16[None, :]
    W = np.zeros((rows, K))
    W[prm] = Wsorted
    if orc.nd:
        dr = buf[o["E"]:o["E"] + 2 * orc.nd].view(np.uint16).astype(np.int64)
        dc = buf[o["E"] + 2 * orc.nd:o["E"] + 4 * orc.nd].view(np.uint16).astype(np.int64)
        dv = buf[o["E"] + 4 * orc.nd:o["E"] + 8 * orc.nd].view(np.float32).astype(np.float64)
        W[dr, dc] += dv
    got = orc.dequant().astype(np.float64)
    assert np.allclose(got, W, rtol=1e-5, atol=1e-6 * np.abs(W).max())


def test_q8_1_blocks_definition(case):
    """ggml block_q8_1 over x': |q| <= 127, max |q| = 127 per non-zero block, d = fp16(amax/127), s = fp16(d sum q)."""
    orc = case["orc"]
    blk = orc.quantize_q8_1(case["x"]).reshape(-1, 36)
    xr = orc.rotate(case["x"]).reshape(-1, 32)
    d = blk[:, 0:2].copy().view(np.float16).reshape(-1).astype(np.float32)
    s = blk[:, 2:4].copy().view(np.float16).reshape(-1).astype(np.float32)
    q = blk[:, 4:].view(np.int8).astype(np.int64)
    amax = np.abs(xr).max(1)
    assert np.array_equal(d, (amax / 127.0).astype(np.float32).astype(np.float16).astype(np.float32))
    assert np.all(np.abs(q).max(1) == 127)
    assert np.allclose(s, (q.sum(1) * (amax / 127.0)).astype(np.float16).astype(np.float32), rtol=2e-3, atol=1e-3)
    err = np.abs(q * (amax / 127.0)[:, None] - xr)
    assert np.all(err <= (amax / 127.0)[:, None] * 0.5 + 1e-6)
    isum = orc.partials_q8_1(blk.reshape(-1))
    ints = case["ints"].astype(np.int64).reshape(case["rows"], -1, 32)
    assert np.array_equal(isum.astype(np.int64), np.einsum("rsk,sk->rs", ints, q))


def test_q8_1_tie_rule_and_sum():
    """ggml block_q8_1 (quantize_row_q8_1_ref, llama.cpp @7ac59a6, the convention followed here): q = roundf(x' * id),
    id = 1/d, d = amax/127, s = fp16(d * sum q). Crafted x' sits exactly on k + 1/2 with d = 1: roundf rounds half
    away from zero (+-(k+1)), where rint / nearbyint would give +-k; s is d * sum q, which differs from sum x'."""
    buf, x, k = slotgen.tie_case(np.random.default_rng(12), K=512, k=2)
    orc = O.Oracle(buf, 32, 512)
    xr = orc.rotate(x)
    assert np.array_equal(xr[0:256:2], np.full(128, 127.0, np.float32))
    assert np.array_equal(xr[1:256:2], np.full(128, k + 0.5, np.float32))
    assert np.array_equal(xr[257:512:2], np.full(128, -(k + 0.5), np.float32))
    blk = orc.quantize_q8_1(x).reshape(-1, 36)
    d = blk[:, 0:2].copy().view(np.float16).reshape(-1)
    s = blk[:, 2:4].copy().view(np.float16).reshape(-1)
    q = blk[:, 4:].view(np.int8).astype(np.int64)
    assert np.all(d[:16] == 1.0) and np.all(d[16:] == 0.0)
    assert np.array_equal(q[:8, 1::2], np.full((8, 16), k + 1)) and np.array_equal(q[8:16, 1::2], np.full((8, 16), -(k + 1)))
    assert np.array_equal(q[:16, 0::2], np.full((16, 16), 127)) and not q[16:].any()
    # s = d * sum q: block 0: 16 * 127 + 16 * (k + 1); sum x' would be 16 * 127 + 16 * (k + 1/2)
    assert np.array_equal(s[:8].astype(np.float64), np.full(8, 16 * 127 + 16 * (k + 1.0)))
    assert np.array_equal(s[8:16].astype(np.float64), np.full(8, 16 * 127 - 16 * (k + 1.0)))
    assert np.all(s[16:] == 0.0)


def test_q8_128_ties_round_half_even():
    """the reference core's own 8-bit-per-128 prep rounds x' * (1/d) with nearbyintf (round half to even, CPU.patch:566-568):
    on the same ties +-(k + 1/2) with k even it gives +-k, not the Q8_1 +-(k + 1)"""
    buf, x, k = slotgen.tie_case(np.random.default_rng(12), K=512, k=2)
    orc = O.Oracle(buf, 32, 512)
    q, d, sx = orc.prep_q8_128(x)
    assert np.array_equal(d, np.array([1, 1, 1, 1], np.float32))
    assert np.all(q[1:256:2] == k) and np.all(q[257:512:2] == -k)
    assert np.array_equal(sx, np.array([64 * 127 + 64 * k] * 2 + [64 * 127 - 64 * k] * 2, np.int32))
    if O.ref_available("scalar"):   # and so does the live reference core (build container only)
        t = O.RefCore("scalar").open(buf, 32, 512)
        X2, XS, SX = t.prep_q8_128(x)
        assert np.array_equal(q, X2[:, :128].reshape(-1)) and np.array_equal(sx, SX)
        t.close()


def test_gemv_f64_cols_equals_single_columns():
    """the multi-column fp64 GEMV (each tile decoded once) equals the one-column one bit for bit"""
    rng = np.random.default_rng(21)
    buf = slotgen.random_slot(rng, 96, 1024, classes=(0, 1, 2, 3, 4, 5, 6, 7), nd=5)
    orc = O.Oracle(buf, 96, 1024)
    X = rng.standard_normal((3, 1024)).astype(np.float32)
    Y = orc.gemv_f64_cols(X)
    for n in range(3):
        assert np.array_equal(Y[n], orc.gemv_f64(X[n])), n


def test_open_rejects_corruption():
    rng = np.random.default_rng(3)
    buf = slotgen.random_slot(rng, 64, 512, classes=(3, 4), nd=2)
    O.Oracle(buf, 64, 512).close()
    bad = buf.copy(); bad[-32] ^= 1                       # trailer magic
    with pytest.raises(ValueError, match="rc=1"):
        O.Oracle(bad, 64, 512)
    with pytest.raises(ValueError, match="rc=1"):         # shape mismatch
        O.Oracle(buf, 32, 512)
    bad = buf.copy(); bad[2052] = 104                     # NS word
    with pytest.raises(ValueError, match="rc=2"):
        O.Oracle(bad, 64, 512)
    bad = buf.copy(); bad[2064 + 3] ^= 0x20               # class of tile 0 changed: kbytes != M-implied size
    with pytest.raises(ValueError, match="rc=4"):
        O.Oracle(bad, 64, 512)


def test_negative_controls_change_decode():
    """one flipped payload bit, one scale and one tile word must each change the decode (research/detail/b3p_native.py:252-262)."""
    rng = np.random.default_rng(4)
    buf = slotgen.random_slot(rng, 32, 256, classes=(3,), nd=0, permute=False)
    base = O.Oracle(buf, 32, 256).dequant()
    offD = slotgen.a16(2064 + 68)
    bad = buf.copy(); bad[offD + 40] ^= 0x04
    assert not np.array_equal(O.Oracle(bad, 32, 256).dequant(), base)
    bad = buf.copy(); bad[2064 + 4 + 10] ^= 0x01          # one fp16 scale
    assert not np.array_equal(O.Oracle(bad, 32, 256).dequant(), base)


@pytest.mark.skipif(not O.ref_available("scalar"), reason="reference core not built here")
def test_live_reference_random_shapes():
    """More random tensors against the live reference core (build container only)."""
    core = O.RefCore("scalar")
    rng = np.random.default_rng(11)
    for rows, K in ((32, 256), (96, 1024), (64, 1536)):
        buf = slotgen.random_slot(rng, rows, K, classes=(0, 1, 2, 3, 4, 5, 6, 7), nd=7)
        x = (rng.standard_normal(K) * rng.uniform(0.1, 10)).astype(np.float32)
        x[:7] = 0.0
        t = core.open(buf, rows, K)
        orc = O.Oracle(buf, rows, K)
        assert np.array_equal(orc.dequant().view(np.uint32), t.dequant().view(np.uint32))
        X2, XS, SX = t.prep_q8_128(x)
        q, d, sx = orc.prep_q8_128(x)
        assert np.array_equal(q, X2[:, :128].reshape(-1)) and np.array_equal(d, XS) and np.array_equal(sx, SX)
        t.close()


@pytest.mark.skipif(not O.ref_available("scalar"), reason="reference core not built here")
def test_live_reference_wrapping_codebook():
    """A codebook whose coset entries A + c leave the int8 range: the reference core adds bytewise and wraps
    (vrc_vadd4, CPU.patch:221, :255); the oracle's decode and dequantize_row do the same (build container only)."""
    core = O.RefCore("scalar")
    rng = np.random.default_rng(13)
    buf = slotgen.random_slot(rng, 64, 512, classes=(1, 2, 3, 4, 5, 6, 7), tables="wrapping", nd=3)
    A, c = slotgen.wrapping_tables(np.random.default_rng(0))
    s = A.view(np.int8).reshape(256, 4).astype(int) + np.array([100, -90, 77, -120])[None, :]
    assert (s > 127).any() and (s < -128).any()   # the table does wrap
    t = core.open(buf, 64, 512)
    orc = O.Oracle(buf, 64, 512)
    for g, b in ((0, 0), (1, 1)):
        assert np.array_equal(orc.decode_tile(g, b), t.decode_tile(g, b))
    assert np.array_equal(orc.dequant().view(np.uint32), t.dequant().view(np.uint32))
    t.close()


def test_zero_block_activation():
    """x = 0 on a block gives d = 0 and q = 0 (CPU.patch:566)."""
    rng = np.random.default_rng(5)
    buf = slotgen.random_slot(rng, 32, 512, classes=(3,))
    orc = O.Oracle(buf, 32, 512)
    x = rng.standard_normal(512).astype(np.float32)
    x[:256] = 0
    q, d, sx = orc.prep_q8_128(x)
    assert d[0] == 0 and d[1] == 0 and not q[:256].any() and sx[0] == 0 and sx[1] == 0
    assert d[2] > 0
