"""Numpy writer of random-valid Pingala-8 native tensor slots (test infrastructure).

Byte layout follows the reference's in-memory contract (patches/llama_cpu_vs_7ac59a6.patch:8-51 and
:3817-3824): header A|B|c|NS|TRL|0, tile words M, fp16 scales S[b][r], 16-aligned payload D, then the
side regions placed top-down from the slot end (delta, c16, prm, pinv, signs, trailer).
Random payload words are always valid codes (every 8-bit index and every label bit is legal), as in the
reference's timing arm (CPU.patch:4391-4458).
"""
import os

import numpy as np

NW = [0, 4, 6, 8, 10, 12, 16, 24]
MAGIC0, MAGIC1 = 0x4E525656, 0x31354952
HERE = os.path.dirname(os.path.abspath(__file__))
TABLES = os.path.join(HERE, "golden", "tables_vrc.bin")


def a16(n):
    return (n + 15) & ~15


def need(kbytes, rows, K, nd):
    return a16(kbytes) + a16(8 * nd) + a16(2 * K) + 2 * a16(2 * rows) + 256 + 32 + 64


def offsets(n, rows, K, nd):
    t = n - 32
    sg = t - 256
    q = (sg - 2 * rows) & ~15
    p = (q - 2 * rows) & ~15
    c = (p - 2 * K) & ~15
    e = (c - 8 * nd) & ~15
    return dict(E=e, C=c, P=p, Q=q, SG=sg, T=t)


def shipped_tables():
    """(A uint32[256], c uint32): the shipped codebook, as raw little-endian int8 (tests/golden/tables_vrc.bin)."""
    raw = np.fromfile(TABLES, np.int8)
    A = raw[:1024].view(np.uint32).copy()
    c = int(raw[1024:1028].view(np.uint32)[0])
    return A, c


def random_tables(rng):
    """A in [-64, 64], c in [-16, 16] (the reference's random-valid arm, CPU.patch:4211-4220)."""
    A = rng.integers(-64, 65, size=(256, 4)).astype(np.int8).view(np.uint32).reshape(256).copy()
    c = int(rng.integers(-16, 17, size=4).astype(np.int8).view(np.uint32)[0])
    return A, c


def wrapping_tables(rng):
    """A over the whole int8 range and a large c, so that many A + c leave [-128, 127] (the bytewise add wraps)"""
    A = rng.integers(-128, 128, size=(256, 4)).astype(np.int8).view(np.uint32).reshape(256).copy()
    c = int(np.array([100, -90, 77, -120], np.int8).view(np.uint32)[0])
    return A, c


def build_slot(A, cs, cls, payload, S, c16, prm, sg, drow=None, dcol=None, dval=None, extra=0):
    """cls int[ng, nb]; payload uint32 in tile order (tile i = g*nb + b has 64*NW(cls) words);
    S uint16 [nb, rows]; c16 uint16 [K]; prm int16 [rows]; sg int8 [256]; delta arrays (original indices)."""
    ng, nb = cls.shape
    rows, K = 32 * ng, 256 * nb
    nt = ng * nb
    nd = 0 if drow is None else len(drow)
    M = np.zeros(nt, np.uint32)
    off = 0
    for i, c in enumerate(cls.reshape(-1)):
        M[i] = off | (int(c) << 29)
        off += 64 * NW[int(c)]
    assert off == payload.size and off < (1 << 29)
    offD = a16(2064 + 68 * nt)
    kbytes = offD + 4 * payload.size
    n = need(kbytes, rows, K, nd) + extra
    buf = np.zeros(n, np.uint8)
    w = buf[:2064].view(np.uint32)
    w[0:256] = A
    w[256:512] = A
    w[512] = cs
    w[513] = 108
    w[514] = 2
    w[515] = 0
    buf[2064:2064 + 4 * nt] = M.view(np.uint8)
    buf[2064 + 4 * nt:2064 + 68 * nt] = np.ascontiguousarray(S, np.uint16).reshape(-1).view(np.uint8)
    buf[offD:kbytes] = payload.view(np.uint8)
    o = offsets(n, rows, K, nd)
    assert kbytes <= o["E"]
    if nd:
        buf[o["E"]:o["E"] + 2 * nd] = np.asarray(drow, np.uint16).view(np.uint8)
        buf[o["E"] + 2 * nd:o["E"] + 4 * nd] = np.asarray(dcol, np.uint16).view(np.uint8)
        buf[o["E"] + 4 * nd:o["E"] + 8 * nd] = np.asarray(dval, np.float32).view(np.uint8)
    buf[o["C"]:o["C"] + 2 * K] = np.ascontiguousarray(c16, np.uint16).view(np.uint8)
    prm = np.asarray(prm, np.int16)
    pinv = np.empty(rows, np.int16)
    pinv[prm.astype(np.int64)] = np.arange(rows, dtype=np.int16)
    buf[o["P"]:o["P"] + 2 * rows] = prm.view(np.uint8)
    buf[o["Q"]:o["Q"] + 2 * rows] = pinv.view(np.uint8)
    buf[o["SG"]:o["SG"] + 256] = np.asarray(sg, np.int8).view(np.uint8)
    buf[o["T"]:o["T"] + 32] = np.array([MAGIC0, MAGIC1, kbytes, nd, rows, K, 108, 1], np.uint32).view(np.uint8)
    return buf


def random_slot(rng, rows, K, classes=(3,), class_p=None, tables="shipped", nd=0, permute=True,
                c16="random", scale_range=(2e-4, 3e-4), extra=0):
    """A random-valid tensor. classes: classes drawn per tile (with probabilities class_p)."""
    ng, nb = rows // 32, K // 256
    A, cs = {"shipped": shipped_tables, "random": lambda: random_tables(rng), "wrapping": lambda: wrapping_tables(rng)}[tables]()
    cls = rng.choice(np.asarray(classes), size=(ng, nb), p=class_p).astype(np.int64)
    nwords = int(sum(64 * NW[c] for c in cls.reshape(-1)))
    payload = rng.integers(0, 1 << 32, size=nwords, dtype=np.uint64).astype(np.uint32)
    S = rng.uniform(*scale_range, size=(nb, rows)).astype(np.float16).view(np.uint16)
    S[np.repeat(cls.T == 0, 32, axis=1)] = 0
    if c16 == "random":
        c16v = rng.uniform(0.5, 2.0, size=K).astype(np.float16).view(np.uint16)
    else:
        c16v = np.full(K, 0x3C00, np.uint16)
    prm = rng.permutation(rows).astype(np.int16) if permute else np.arange(rows, dtype=np.int16)
    sg = np.where(rng.integers(0, 2, 256) == 1, 1, -1).astype(np.int8)
    drow = dcol = dval = None
    if nd:
        flat = rng.choice(rows * K, size=nd, replace=False)
        order = np.argsort(flat)
        flat = flat[order]
        drow = (flat // K).astype(np.uint16)
        dcol = (flat % K).astype(np.uint16)
        dval = rng.uniform(-0.05, 0.05, size=nd).astype(np.float32)
    return build_slot(A, cs, cls, payload, S, c16v, prm, sg, drow, dcol, dval, extra=extra)


def shuffle_tiles(buf, rows, K, rng):
    """The same tensor with its tiles stored in D in a random order (M offsets follow): every tile's class, words
    and decoded values are unchanged; only the physical order differs (the contract allows any order)."""
    ng, nb = rows // 32, K // 256
    nt = ng * nb
    M = buf[2064:2064 + 4 * nt].view(np.uint32).copy()
    offD = a16(2064 + 68 * nt)
    cls = (M >> 29).astype(np.int64)
    size = np.array([64 * NW[c] for c in cls], np.int64)
    old = (M & 0x1FFFFFFF).astype(np.int64)
    D = buf[offD:offD + 4 * int(size.sum())].view(np.uint32)
    newD = np.empty_like(D)
    new = np.zeros(nt, np.int64)
    off = 0
    for t in rng.permutation(nt):
        new[t] = off
        newD[off:off + size[t]] = D[old[t]:old[t] + size[t]]
        off += size[t]
    out = buf.copy()
    out[2064:2064 + 4 * nt] = (new.astype(np.uint32) | (cls.astype(np.uint32) << 29)).view(np.uint8)
    out[offD:offD + 4 * off] = newD.view(np.uint8)
    return out


def tie_case(rng, K=512, k=2):
    """A 32 x K class-3 tensor with c16 = 1 and an activation x whose rotated values x' land exactly on quantizer
    ties. In 256-block b = 0, 1 only x'[0] = a, x'[1] = b are non-zero before the transform, so after FWHT256 / 16
    every even column holds (a + b) / 16 = 127 and every odd column (a - b) / 16 = +-(k + 1/2) (block 0: +, block 1:
    -). Every scale is then d = 127 / 127 = 1 exactly (both per 32 and per 128 columns), so x' / d is exactly
    +-(k + 1/2): round-half-away gives +-(k + 1), round-half-even gives +-k (k even). Blocks past 1 are zero.
    Returns (slot bytes, x, k)."""
    buf = random_slot(rng, 32, K, classes=(3,), c16="ones", permute=False)
    sg = buf[offsets(buf.size, 32, K, 0)["SG"]:][:256].view(np.int8).astype(np.float32)
    a, b = (2032 + 16 * k + 8) // 2, (2032 - 16 * k - 8) // 2      # a + b = 16 * 127, a - b = 16 (k + 1/2)
    x = np.zeros(K, np.float32)
    # x * ic = x * sg / c must be (a, b) at columns 0, 1 of block 0 and (b, a) of block 1
    x[0], x[1] = a * sg[0], b * sg[1]
    x[256], x[257] = b * sg[0], a * sg[1]
    return buf, x, k


W1 = [0, 4, 6, 8, 8, 8, 8, 8]
W2 = [0, 0, 0, 0, 2, 4, 8, 8]
W3 = [0, 0, 0, 0, 0, 0, 0, 8]


def _put(lw, wb, W, k, v):
    pos = W * k
    wi, bb = wb + (pos >> 5), pos & 31
    x = (int(v) & ((1 << W) - 1)) << bb
    lw[wi] |= x & 0xFFFFFFFF
    if bb + W > 32:
        lw[wi + 1] |= x >> 32


def pack_codes(idx, cls, prm):
    """Payload words (tile order) from stage indices idx [rows][K/4][3] by ORIGINAL row, classes cls [ng][nb] per
    sorted tile and prm (sorted -> original). Field layout per lane (CPU.patch:285-309): stage 1 of width W1 < 8 as
    the 32 stored MSBs in word 0 plus (W1 - 1)-bit low fields from word 1, W1 = 8 as 8-bit fields from word 0; stage 2
    from word W1, stage 3 from word W1 + W2; lane j's k-th field is chunk (j + k) & 31; words [i >> 1][j][i & 1]."""
    ng, nb = cls.shape
    words = []
    for g in range(ng):
        for b in range(nb):
            c = int(cls[g, b])
            nw = NW[c]
            if not nw:
                continue
            tile = np.zeros(64 * nw, np.uint32)
            for hs in range(2):
                for j in range(32):
                    r = int(prm[32 * g + j])
                    ch = idx[r, (256 * b + 128 * hs) // 4:(256 * b + 128 * hs) // 4 + 32]
                    lw = [0] * nw
                    for k in range(32):
                        f = ch[(j + k) & 31]
                        if W1[c] == 8:
                            _put(lw, 0, 8, k, f[0])
                        else:
                            lw[0] |= ((int(f[0]) >> (W1[c] - 1)) & 1) << k
                            _put(lw, 1, W1[c] - 1, k, f[0])
                        if W2[c]:
                            _put(lw, W1[c], W2[c], k, f[1])
                        if W3[c]:
                            _put(lw, W1[c] + W2[c], W3[c], k, f[2])
                    for i in range(nw):
                        tile[hs * nw * 32 + ((i >> 1) << 6) + 2 * j + (i & 1)] = lw[i]
            words.append(tile)
    return np.concatenate(words) if words else np.zeros(0, np.uint32)


def _get(w, wb, W, k):
    pos = W * k
    wi, bb = wb + (pos >> 5), pos & 31
    v = int(w[wi]) | ((int(w[wi + 1]) << 32) if wi + 1 < len(w) else 0)
    return (v >> bb) & ((1 << W) - 1)


def slot_codes(slot, rows, K):
    """(cls [ng][nb], idx [rows][K/4][3] by SORTED row, h [rows][K/4] coset bits) read back from a slot's payload;
    the coset bit of chunk t is u_{t-2} of the recursion u_t = z_t ^ u_{t-1} ^ u_{t-3} over the stored stage-1 MSBs
    z in chunk order (CPU.patch:299-304)."""
    ng, nb = rows // 32, K // 256
    nt = ng * nb
    M = slot[2064:2064 + 4 * nt].view(np.uint32)
    offD = a16(2064 + 68 * nt)
    D = slot[offD:offD + 4 * ((slot.size - offD) // 4)].view(np.uint32)
    cls = (M >> 29).astype(np.int64).reshape(ng, nb)
    idx = np.zeros((rows, K // 4, 3), np.int64)
    hb = np.zeros((rows, K // 4), np.int64)
    for g in range(ng):
        for b in range(nb):
            c = int(cls[g, b])
            nw = NW[c]
            if not nw:
                continue
            base = int(M[g * nb + b] & 0x1FFFFFFF)
            for hs in range(2):
                for j in range(32):
                    lw = [int(D[base + hs * nw * 32 + ((i >> 1) << 6) + 2 * j + (i & 1)]) for i in range(nw)]
                    z = [0] * 32
                    for k in range(32):
                        t = (j + k) & 31
                        col = (256 * b + 128 * hs) // 4 + t
                        if W1[c] == 8:
                            f1 = _get(lw, 0, 8, k)
                        else:
                            f1 = _get(lw, 1, W1[c] - 1, k) | (((lw[0] >> k) & 1) << (W1[c] - 1))
                        idx[32 * g + j, col, 0] = f1
                        if W2[c]:
                            idx[32 * g + j, col, 1] = _get(lw, W1[c], W2[c], k)
                        if W3[c]:
                            idx[32 * g + j, col, 2] = _get(lw, W1[c] + W2[c], W3[c], k)
                        z[t] = f1 >> (W1[c] - 1)
                    u = [0] * 32
                    for t in range(32):
                        u[t] = z[t] ^ (u[t - 1] if t >= 1 else 0) ^ (u[t - 3] if t >= 3 else 0)
                        hb[32 * g + j, (256 * b + 128 * hs) // 4 + t] = u[t - 2] if t >= 2 else 0
    return cls, idx, hb
