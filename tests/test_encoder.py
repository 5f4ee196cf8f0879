"""The host encoder (p8x_encode_tensor and friends) against the numpy restatement of the reference's tensor
encoder (oracle/encode_oracle.py, research/detail/r48k.py), and that restatement against what the mathematics fixes:

* factor: U upper with U^T U Hq = I for Hq built from an explicit dense rotation (scipy's Sylvester Hadamard matrix);
* alloc: the budget holds, no affordable upgrade is left, the extreme budgets give all-0 / all-7, salient tiles are
  held at class >= 6, more budget never costs distortion;
* identity metric: each half-slice's cost equals an independent dynamic-programming minimum over all label sequences
  of the decoder's trellis (the Viterbi is exact there);
* LDLQ: from the decoded slot alone, E = (Y - Q) U^-1 recovers each step's fed-back target x_t = q_t + e_t U_tt, and
  every chosen codeword is the metric-nearest entry of its half (single-stage classes) or no worse than the greedy
  stage-by-stage pick (multi-stage classes) for that target -- a dropped or misplaced feedback term fails this;
* the decoded slot reproduces the encoder's own reconstruction (format packing and trellis labels agree);
* scales and row order follow their formulas recomputed here from W.
The native slots must equal the oracle's, byte for byte.
"""
import numpy as np
import pytest
from scipy.linalg import hadamard, solve_triangular

import encode_oracle as OE
import oracle as O
import p8x
import slotgen

HAD = hadamard(256).astype(np.float64) / 16.0


def shipped():
    A, cs = slotgen.shipped_tables()
    A8 = A.view(np.int8).reshape(256, 4).astype(np.float64)
    c8 = np.frombuffer(np.uint32(cs).tobytes(), np.int8).astype(np.float64)
    return A, cs, A8, c8


def rand_inputs(rng, rows, K, outliers=0.0):
    W = (rng.standard_normal((rows, K)) * 0.02).astype(np.float32)
    if outliers:
        m = rng.random(W.shape) < outliers
        W[m] *= 12
    c16 = rng.uniform(0.6, 1.8, K).astype(np.float16).view(np.uint16)
    sg = np.where(rng.integers(0, 2, 256) == 1, 1, -1).astype(np.int8)
    return W, c16, sg


def rand_H(rng, K, n=None, corr=0.9):
    """second moment of correlated inputs: AR(1) columns with per-column gains"""
    n = n or 2 * K
    Z = rng.standard_normal((n, K))
    X = np.empty_like(Z)
    X[:, 0] = Z[:, 0]
    for k in range(1, K):
        X[:, k] = corr * X[:, k - 1] + np.sqrt(1 - corr * corr) * Z[:, k]
    X *= rng.uniform(0.3, 3.0, K)[None, :]
    return (X.T @ X / n).astype(np.float32)


def dense_rotation(sg, K):
    R1 = HAD * sg.astype(np.float64)[None, :]
    R = np.zeros((K, K))
    for b in range(K // 256):
        R[256 * b:256 * b + 256, 256 * b:256 * b + 256] = R1
    return R


def slot_from_oracle(res, c16, sg):
    A, cs, _, _ = shipped()
    pay = slotgen.pack_codes(res["idx"], res["cls"], res["prm"])
    return slotgen.build_slot(A, cs, res["cls"], pay, res["S"], c16, res["prm"], sg,
                              res["drow"] if len(res["drow"]) else None, res["dcol"] if len(res["drow"]) else None,
                              res["dval"] if len(res["drow"]) else None)


def oracle_encode(W, c16, sg, U=None, **kw):
    _, _, A8, c8 = shipped()
    return OE.encode_tensor(W, c16, sg, U=U, A=A8, cvec=c8, **kw)


# ----------------------------------------------------------------------------------------------- factor
def test_oracle_factor_inverts_rotated_H():
    rng = np.random.default_rng(11)
    K = 512
    _, c16, sg = rand_inputs(rng, 32, K)
    H = rand_H(rng, K)
    U = OE.factor(H, c16.view(np.float16).astype(np.float64), sg, 0.1)
    assert np.allclose(np.tril(U, -1), 0)
    assert (U.diagonal() > 0).all()
    R = dense_rotation(sg, K)
    c = c16.view(np.float16).astype(np.float64)
    Hp = R @ (H.astype(np.float64) / c[:, None] / c[None, :]) @ R.T
    Hq = Hp + 0.1 * Hp.diagonal().mean() * np.eye(K)
    assert np.abs(U.T @ U @ Hq - np.eye(K)).max() < 1e-8


def test_native_factor_matches_oracle():
    rng = np.random.default_rng(12)
    K = 768
    _, c16, sg = rand_inputs(rng, 32, K)
    H = rand_H(rng, K)
    Un = p8x.encode_factor(H, c16=c16, signs=sg, damp=0.1)
    Uo = OE.factor(H, c16.view(np.float16).astype(np.float64), sg, 0.1)
    assert np.abs(Un - Uo).max() <= 1e-9 * np.abs(Uo).max()


def test_native_factor_rejects_indefinite():
    K = 256
    H = -np.eye(K, dtype=np.float32)
    with pytest.raises(p8x.P8xError, match="positive definite"):
        p8x.encode_factor(H, damp=0.0)


# ----------------------------------------------------------------------------------------------- allocation
def alloc_rate(c):
    return (256.0 * np.asarray(OE.RATE))[c].sum()


def test_oracle_alloc_properties():
    rng = np.random.default_rng(13)
    E = rng.lognormal(0, 2, 40)
    assert (OE.alloc(E, 0.0) == 0).all()
    assert (OE.alloc(E, 1536.0 * E.size) == 7).all()
    prev = None
    for bpw in (0.5, 1.0, 2.0, 2.5, 3.5):
        budget = 256.0 * bpw * E.size
        c = OE.alloc(E, budget)
        assert alloc_rate(c) <= budget
        slack = budget - alloc_rate(c)
        up = [256.0 * (OE.RATE[k] - OE.RATE[ci]) for ci in c for k in range(ci + 1, 8)]
        assert not up or min(up) > slack                     # no affordable upgrade left
        D = (E * np.asarray(OE.DIST)[c]).sum()
        if prev is not None:
            assert D <= prev * (1 + 1e-12)
        prev = D
    fl = np.zeros(E.size, bool)
    fl[[3, 17]] = True
    c = OE.alloc(E, 256.0 * 2.0 * E.size, floor=fl)
    assert (c[fl] >= 6).all()


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_native_alloc_matches_oracle(seed):
    rng = np.random.default_rng(100 + seed)
    E = rng.lognormal(0, 1.5, (6, 9))
    fl = rng.random(E.shape) < 0.1
    for bpw in (1.0, 2.0, 2.75):
        budget = bpw * 32 * 256 * E.size                     # whole-tensor bits; tiles are 32 x 256
        for floor in (None, fl):
            n = p8x.encode_alloc(E, budget, floor=floor)
            o = OE.alloc(E.ravel(), budget / 32.0, floor=None if floor is None else floor.ravel()).reshape(E.shape)
            assert np.array_equal(n, o), (bpw, floor is None)


# ----------------------------------------------------------------------------------------------- oracle pins
def _dp_min(X, tab0, tab1, K1):
    """min over stored-label sequences of sum_t min_{f in half z_t} |X_t - tab_h(f)|^2 with the decoder's trellis
    (u_t = z_t ^ u_{t-1} ^ u_{t-3}, h_t = u_{t-2}), states keyed by (u_{t-1}, u_{t-2}, u_{t-3})"""
    half = K1 // 2
    cost = {}
    for h, tab in ((0, tab0), (1, tab1)):
        d = ((X[:, None, :] - tab[None, :K1, :]) ** 2).sum(-1)
        cost[h] = (d[:, :half].min(1), d[:, half:].min(1))
    pm = {(0, 0, 0): 0.0}
    for t in range(X.shape[0]):
        nm = {}
        for (u1, u2, u3), v in pm.items():
            for z in (0, 1):
                u = z ^ u1 ^ u3
                c = v + cost[u2][z][t]
                key = (u, u1, u2)
                if c < nm.get(key, np.inf):
                    nm[key] = c
        pm = nm
    return min(pm.values())


def test_oracle_identity_viterbi_exact_and_decodable():
    rng = np.random.default_rng(14)
    rows, K = 64, 512
    W, c16, sg = rand_inputs(rng, rows, K)
    cls = np.array([[1, 2], [3, 2]], np.uint8)
    res = oracle_encode(W, c16, sg, classes=cls, n_salient=0)
    slot = slot_from_oracle(res, c16, sg)
    orc = O.Oracle(slot, rows, K)
    ints_sorted = orc.decode_all().astype(np.int64)
    prm = res["prm"].astype(np.int64)
    assert np.array_equal(ints_sorted, res["ints"][prm])            # decoder == encoder reconstruction
    # scales and row order from their formulas
    c = c16.view(np.float16).astype(np.float64)
    Y = np.concatenate([(W[:, 256 * b:256 * b + 256].astype(np.float64) * c[256 * b:256 * b + 256] * sg) @ HAD.T
                        for b in range(K // 256)], axis=1)
    E = (Y.reshape(rows, 2, 256) ** 2).sum(-1)
    key = np.log(np.maximum(E, 1e-30)).mean(1)
    assert np.array_equal(np.argsort(key, kind="stable"), prm)
    _, _, A8, c8 = shipped()
    for rs in range(rows):
        r = prm[rs]
        for b in range(2):
            k = int(cls[rs // 32, b])
            rms = np.sqrt(E[r, b] / 256.0)
            assert res["S"][b, rs] == np.float16(np.float32(1.05 * rms / OE.GAIN[k])).view(np.uint16)
    # exact Viterbi: the achieved half-slice cost is the DP minimum
    S = res["S"].view(np.float16).astype(np.float64)
    for rs in (0, 7, 33, 63):
        r = prm[rs]
        for b in range(2):
            k = int(cls[rs // 32, b])
            K1 = 1 << OE.W1[k]
            for hs in range(2):
                sl = slice(256 * b + 128 * hs, 256 * b + 128 * hs + 128)
                X = (Y[r, sl] / S[b, rs]).reshape(32, 4)
                got = ((X - ints_sorted[rs, sl].reshape(32, 4)) ** 2).sum()
                ref = _dp_min(X, A8, A8 + c8[None, :], K1)
                assert got == pytest.approx(ref, rel=1e-9, abs=1e-12)


@pytest.mark.parametrize("seed", [0, 1])
def test_oracle_ldlq_choices_follow_fed_back_targets(seed):
    rng = np.random.default_rng(20 + seed)
    rows, K = 64, 768
    W, c16, sg = rand_inputs(rng, rows, K)
    H = rand_H(rng, K)
    c = c16.view(np.float16).astype(np.float64)
    U = OE.factor(H, c, sg, 0.1)
    cls = rng.integers(1, 8, (2, 3)).astype(np.uint8)
    cls[0, 0], cls[1, 2], cls[0, 2] = 7, 3, 0
    res = oracle_encode(W, c16, sg, U=U, classes=cls, n_salient=0)
    slot = slot_from_oracle(res, c16, sg)
    _, idx, hb = slotgen.slot_codes(slot, rows, K)
    ints = O.Oracle(slot, rows, K).decode_all().astype(np.float64)
    prm = res["prm"].astype(np.int64)
    S = res["S"].view(np.float16).astype(np.float64)
    Y = (W.astype(np.float64) * c[None, :]) @ dense_rotation(sg, K).T
    Ys = Y[prm]
    Q = ints * np.repeat(S.T, 256, axis=1)                            # rotated-domain reconstruction, sorted rows
    E = solve_triangular(U.T, (Ys - Q).T, lower=True).T               # (Y - Q) = E U
    _, _, A8, c8 = shipped()
    checked = 0
    for rs in range(0, rows, 5):
        for t in range(K // 4):
            b = t // 64
            k = int(cls[rs // 32, b])
            if k == 0:
                continue
            j = 4 * t
            Ub = U[j:j + 4, j:j + 4]
            A4 = np.linalg.inv(Ub)
            x = Q[rs, j:j + 4] + E[rs, j:j + 4] @ Ub                    # the target the encoder saw at this step
            h = hb[rs, t]
            y = x / S[b, rs] - h * OE.mc(k) * c8
            xa = y @ A4
            f1, f2, f3 = idx[rs, t]
            s1, s2 = 1 << OE.SH1[k], 1 << OE.SH2[k]
            base = A8[f1] * s1 + (A8[f2] * s2 if OE.W2[k] else 0) + (A8[f3] if OE.W3[k] else 0)
            assert np.array_equal(base + h * OE.mc(k) * c8, ints[rs, j:j + 4])
            d_got = (((xa - base @ A4)) ** 2).sum()
            K1h = 1 << (OE.W1[k] - 1)
            half = f1 >> (OE.W1[k] - 1)
            tab1 = A8[half * K1h:(half + 1) * K1h] * s1
            d1 = (((xa[None, :] - tab1 @ A4)) ** 2).sum(1)
            tol = 1e-9 * max(1.0, d_got)
            if not OE.W2[k]:
                assert d_got <= d1.min() + tol
            else:                                                      # no worse than greedy stage by stage
                g1 = tab1[np.argmin(d1)]
                r = xa - g1 @ A4
                t2 = A8[:1 << OE.W2[k]] * s2
                g2 = t2[np.argmin(((r[None, :] - t2 @ A4) ** 2).sum(1))]
                gv = g1 + g2
                if OE.W3[k]:
                    r2 = r - g2 @ A4
                    gv = gv + A8[np.argmin(((r2[None, :] - A8 @ A4) ** 2).sum(1))]
                d_greedy = (((xa - gv @ A4)) ** 2).sum()
                assert d_got <= d_greedy + tol
            checked += 1
    assert checked > 500


# ----------------------------------------------------------------------------------------------- native == oracle
CASES = {
    "identity_alloc": dict(seed=1, U=False, classes=None, bpw=2.0, nsal=4, prm=False, W="gauss"),
    "ldlq_given_classes": dict(seed=2, U=True, classes="mix", bpw=2.0, nsal=0, prm=True, W="gauss"),
    "ldlq_alloc_outliers": dict(seed=3, U=True, classes=None, bpw=2.5, nsal=4, prm=False, W="outliers"),
    "ldlq_clamp_deltas": dict(seed=4, U=True, classes=None, bpw=2.0, nsal=0, prm=False, W="flat"),
}


@pytest.mark.parametrize("name", list(CASES))
def test_native_slot_equals_oracle(name):
    cfg = CASES[name]
    rng = np.random.default_rng(cfg["seed"])
    rows, K = 64, 512
    W, c16, sg = rand_inputs(rng, rows, K, 0.002 if cfg["W"] == "outliers" else 0.0)
    if cfg["W"] == "flat":                                   # |W| constant: any overshoot of the code exceeds wmax
        W = np.where(W > 0, np.float32(0.02), np.float32(-0.02))
    c = c16.view(np.float16).astype(np.float64)
    U = OE.factor(rand_H(rng, K), c, sg, 0.1) if cfg["U"] else None
    classes = None
    if cfg["classes"] == "mix":
        classes = np.array([[0, 7], [4, 1]], np.uint8)
    prm = rng.permutation(rows).astype(np.int16) if cfg["prm"] else None
    res = oracle_encode(W, c16, sg, U=U, classes=classes, bits_per_weight=cfg["bpw"], n_salient=cfg["nsal"], prm=prm)
    want = slot_from_oracle(res, c16, sg)
    got = p8x.encode_tensor(W, c16=c16, U=U, classes=classes, bits_per_weight=cfg["bpw"], n_salient=cfg["nsal"],
                            prm=prm, signs=sg)
    assert got.size == want.size
    assert np.array_equal(got, want)
    if cfg["W"] == "flat":
        assert len(res["drow"]) > 100
    Wd = O.Oracle(got, rows, K).dequant()
    assert np.abs(Wd).max() <= res["wmax"]


def test_native_threads_do_not_change_the_slot():
    rng = np.random.default_rng(31)
    rows, K = 96, 512
    W, c16, sg = rand_inputs(rng, rows, K)
    H = rand_H(rng, K)
    a = p8x.encode_tensor(W, c16=c16, H=H, signs=sg, threads=1)
    b = p8x.encode_tensor(W, c16=c16, H=H, signs=sg, threads=7)
    assert np.array_equal(a, b)


def test_ldlq_lowers_the_proxy_loss():
    """tr(dW H dW^T) with H-weighted feedback is well below the plain-MSE code of the same classes"""
    rng = np.random.default_rng(32)
    rows, K = 64, 512
    W, c16, sg = rand_inputs(rng, rows, K)
    H = rand_H(rng, K, corr=0.95)
    cls = np.full((rows // 32, K // 256), 3, np.uint8)
    loss = {}
    for name, h in (("plain", None), ("ldlq", H)):
        slot = p8x.encode_tensor(W, c16=c16, H=h, classes=cls, signs=sg, n_salient=0)
        d = (O.Oracle(slot, rows, K).dequant() - W).astype(np.float64)
        loss[name] = np.einsum("rk,kl,rl->", d, H.astype(np.float64), d)
    assert loss["ldlq"] < 0.8 * loss["plain"], loss


def test_encoded_slot_opens_and_rates():
    rng = np.random.default_rng(33)
    rows, K = 128, 1024
    W, c16, sg = rand_inputs(rng, rows, K, outliers=0.001)
    slot = p8x.encode_tensor(W, c16=c16, H=rand_H(rng, K), bits_per_weight=2.0, signs=sg)
    cls, _, _ = slotgen.slot_codes(slot, rows, K)
    bits = (np.asarray(OE.RATE)[cls] * 32 * 256).sum()
    assert bits <= 2.0 * rows * K
    orc = O.Oracle(slot, rows, K)
    rel = np.linalg.norm(orc.dequant() - W) / np.linalg.norm(W)
    assert rel < 0.5, rel


def test_encoder_rejects_bad_input():
    rng = np.random.default_rng(34)
    W, c16, sg = rand_inputs(rng, 32, 256)
    with pytest.raises(p8x.P8xError, match="shape"):
        p8x.encode_tensor(W[:, :200])
    bad = W.copy(); bad[0, 0] = np.nan
    with pytest.raises(p8x.P8xError, match="not finite"):
        p8x.encode_tensor(bad)
    z = c16.copy(); z[5] = 0
    with pytest.raises(p8x.P8xError, match="column scale"):
        p8x.encode_tensor(W, c16=z)
    with pytest.raises(p8x.P8xError, match="permutation"):
        p8x.encode_tensor(W, prm=np.zeros(32, np.int16))
    with pytest.raises(p8x.P8xError, match="class"):
        p8x.encode_tensor(W, classes=np.full((1, 1), 8, np.uint8))
    A, cs = slotgen.wrapping_tables(rng)
    with pytest.raises(p8x.P8xError, match="int8"):
        p8x.encode_tensor(W, A=A, cs=cs)
