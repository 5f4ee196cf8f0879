"""Write the golden fixtures of tests/golden/ from the reference's own CPU core.

Run in the build container (needs /root/reference and oracle/_ref built by `make -C oracle`):
    python3 tests/golden/gen_golden.py
Nothing here runs on the GPU host; the committed .npz/.bin files are the data the tests read.

tables_vrc.bin : the shipped codebook A (256 x int8x4) and coset vector c (int8x4), copied out of the raw
                 little-endian f32 storages of research/work/r48k3/tables_vrc.pt (data/0 = A [256,4],
                 data/2 = c [4]) with zipfile; nothing is unpickled.
case_*.npz     : random-valid tensor slots (tests/slotgen.py) and what the reference core
                 (vr-native-cpu-core.h, scalar build) computes on them: exact tile ints (vrc_decode_tile_int),
                 original-domain f32 weights (vrc_dequant_f32), q8 activation prep (vrc_prep_block),
                 x16 prep (vrc_prep_block16) and the GEMV outputs of its two-phase driver.
"""
import os
import sys
import zipfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

PT = "/root/reference/research/work/r48k3/tables_vrc.pt"


def write_tables():
    z = zipfile.ZipFile(PT)
    A = np.frombuffer(z.read("tables_vrc/data/0"), "<f4")
    c = np.frombuffer(z.read("tables_vrc/data/2"), "<f4")
    assert A.size == 1024 and c.size == 4
    assert np.all(A == np.round(A)) and np.all(c == np.round(c))
    out = np.concatenate([A.astype(np.int8), c.astype(np.int8)])
    out.tofile(os.path.join(HERE, "tables_vrc.bin"))
    return out


CASES = [
    # name, rows, K, classes, tables, nd, seed
    ("c1", 32, 512, (1,), "shipped", 0, 101),
    ("c2", 32, 512, (2,), "shipped", 0, 102),
    ("c3", 32, 512, (3,), "shipped", 3, 103),
    ("c4", 32, 512, (4,), "shipped", 0, 104),
    ("c5", 32, 512, (5,), "shipped", 0, 105),
    ("c6", 32, 512, (6,), "shipped", 0, 106),
    ("c7", 32, 512, (7,), "shipped", 0, 107),
    ("mixed", 64, 768, (0, 1, 2, 3, 4, 5, 6, 7), "shipped", 12, 108),
    ("randtab", 64, 512, (1, 2, 3, 4, 5, 6, 7), "random", 5, 109),
]


def main():
    import slotgen
    from oracle import RefCore, RefPool

    write_tables()
    core = RefCore("scalar")
    others = [RefCore(v) for v in ("avx2", "vnni")]
    pool = RefPool(core, 1)
    for name, rows, K, classes, tables, nd, seed in CASES:
        rng = np.random.default_rng(seed)
        buf = slotgen.random_slot(rng, rows, K, classes=classes, tables=tables, nd=nd, extra=48)
        x = rng.standard_normal(K).astype(np.float32)
        t = core.open(buf, rows, K)
        ints = np.concatenate([np.concatenate([t.decode_tile(g, b) for b in range(K // 256)], axis=1)
                               for g in range(rows // 32)], axis=0)
        W = t.dequant()
        X2, XS, SX = t.prep_q8_128(x)
        assert np.array_equal(X2[:, :128], X2[:, 128:])
        Xh, XSh, SXh, Xl, XSl, SXl = t.prep_x16(x)
        y8 = np.zeros(rows, np.float32)
        y16 = np.zeros(rows, np.float32)
        pool.gemv_seq([t], [x], [y8], planes=1)
        pool.gemv_seq([t], [x], [y16], planes=2)
        for oc in others:  # the SIMD builds must reproduce the scalar build exactly
            o = oc.open(buf, rows, K)
            assert np.array_equal(o.dequant().view(np.uint32), W.view(np.uint32)), oc.variant
            a, b_, c_ = o.prep_q8_128(x)
            assert np.array_equal(a, X2) and np.array_equal(b_, XS) and np.array_equal(c_, SX), oc.variant
            o.close()
        np.savez_compressed(
            os.path.join(HERE, f"case_{name}.npz"),
            slot=buf, rows=rows, K=K, x=x, ints=ints, dequant=W,
            q8=X2[:, :128].reshape(-1), q8_d=XS, q8_sum=SX,
            x16_hi=Xh[:, :128].reshape(-1), x16_hi_d=XSh, x16_hi_sum=SXh,
            x16_lo=Xl[:, :128].reshape(-1), x16_lo_d=XSl, x16_lo_sum=SXl,
            y_q8=y8, y_x16=y16)
        t.close()
        print(f"case {name}: rows {rows} K {K} slot {buf.size} B nd {nd}")
    pool.close()


if __name__ == "__main__":
    main()
