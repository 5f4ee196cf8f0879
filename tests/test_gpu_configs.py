"""GPU parity on the configurations the benchmark times, at their real shapes and launch plans.

* Llama-3.1-8B stack as one grouped launch: 32 layers x (q, k, v, o, gate, up, down) + the lm_head as 4 x 32064-row
  shards, 228 jobs; the plan is the benchmark's (whole-K units of 16 and 56 blocks, K-split tail jobs, no
  small-launch fallback).
* Qwen3-4B layer: the 7 shapes as single calls and as one grouped launch.
* Qwen3-14B shapes at 1, 2, 4 and 8 columns: single calls, and the 40-layer grouped launch.
* Llama FFN shapes (14336 x 4096, 4096 x 14336) as single calls.
* The K-split fix-up paths called 50 times in a row, bitwise equal each time.

The plan depends on shapes and tile classes only, so the grouped launches reuse a few tensors for many jobs, each
job with its own activations. Every job is compared with a single p8x_mul_mat_vec call on the same x (itself checked
against the fp64 oracle), and one job per tensor kind directly with the fp64 oracle. Bar: 1e-3 relative L2 of fp64
(the fixture-free oracle consumes the same 8-bit activations); measured values sit near 1e-7, asserted at 1e-5.
"""
import numpy as np
import pytest

import oracle as O
import p8x

pytestmark = pytest.mark.gpu
TOL = 1e-5

LLAMA = [("attn_q", 4096, 4096), ("attn_k", 1024, 4096), ("attn_v", 1024, 4096), ("attn_output", 4096, 4096),
         ("ffn_gate", 14336, 4096), ("ffn_up", 14336, 4096), ("ffn_down", 4096, 14336)]
LLAMA_HEAD = ("lm_head", 32064, 4096)
QWEN4B = [("attn_q", 4096, 2560), ("attn_k", 1024, 2560), ("attn_v", 1024, 2560), ("attn_output", 2560, 4096),
          ("ffn_gate", 9728, 2560), ("ffn_up", 9728, 2560), ("ffn_down", 2560, 9728)]
QWEN14B = [("attn_q", 5120, 5120), ("attn_k", 1024, 5120), ("attn_v", 1024, 5120), ("attn_output", 5120, 5120),
           ("ffn_gate", 17408, 5120), ("ffn_up", 17408, 5120), ("ffn_down", 5120, 17408)]


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


class Kind:
    """one tensor of a layer kind, with its oracle"""

    def __init__(self, name, rows, K, seed, nd=3):
        self.name, self.rows, self.K = name, rows, K
        self.slot = p8x.synth_random(seed, rows, K, nd=nd)
        self.t = p8x.Tensor(self.slot, rows, K)
        self._orc = None

    @property
    def orc(self):
        if self._orc is None:
            self._orc = O.Oracle(self.slot, self.rows, self.K)
        return self._orc


def grouped_check(kinds, plan, ncols, seed, oracle_jobs):
    """one grouped launch over `plan` (indices into kinds), each job with its own activations; every job against a
    single call on the same x, jobs in oracle_jobs against the fp64 oracle. Returns the batch's plan."""
    rng = np.random.default_rng(seed)
    hx = [rng.standard_normal((ncols, kinds[k].K)).astype(np.float32) for k in plan]
    xs = [p8x.DeviceBuffer.from_numpy(x) for x in hx]
    ys = [p8x.DeviceBuffer(4 * ncols * kinds[k].rows) for k in plan]
    batch = p8x.GemvBatch([kinds[k].t for k in plan], xs, ys, ncols=ncols)
    info = batch.info()
    batch.run()
    p8x.synchronize()
    for i, k in enumerate(plan):
        kd = kinds[k]
        Y = ys[i].to_numpy(np.float32, (ncols, kd.rows))
        S = kd.t.mul_mat_vec(hx[i])
        for n in range(ncols):
            assert rel_l2(Y[n], S[n]) < TOL, (i, kd.name, n)
        if i in oracle_jobs:
            R = kd.orc.gemv_f64_cols(hx[i])
            for n in range(ncols):
                assert rel_l2(Y[n], R[n]) < TOL, (i, kd.name, n)
    batch.release()
    for b in xs + ys:
        b.free()
    return info


@pytest.fixture(scope="module")
def llama():
    kinds = [Kind(n, r, K, 300 + i) for i, (n, r, K) in enumerate(LLAMA + [LLAMA_HEAD])]
    yield kinds
    for k in kinds:
        k.t.release()


def test_llama_stack_grouped_plan(llama):
    """the benchmark's grouped launch: 32 layers + 4 head shards (228 jobs, 47016 row groups)"""
    plan = [k for _ in range(32) for k in range(7)] + [7] * 4
    # one job per kind checked against the oracle (a job from the middle of the list, the last layer's down, and the
    # last head shard: the jobs the tail split cuts along K come last)
    first = {k: 7 * 16 + k for k in range(7)}
    oracle_jobs = set(first.values()) | {len(plan) - 5, len(plan) - 1}
    info = grouped_check(llama, plan, 1, 11, oracle_jobs)
    row_groups = sum(llama[k].rows // 32 for k in plan)
    assert info["small_launch"] == 0, info
    assert 0 < info["split_jobs"] < len(plan), info           # only the tail jobs are cut along K
    assert row_groups < info["units"] < 2 * row_groups, info  # whole-K units plus the tail splits
    assert info["class_set"] == 1 << 3


@pytest.mark.parametrize("kind", [4, 5, 6])
def test_llama_ffn_single_calls(llama, kind):
    """ffn_gate / ffn_up (14336 x 4096) and ffn_down (4096 x 14336, the K-split row-group kernel) against fp64"""
    kd = llama[kind]
    X = np.random.default_rng(kind).standard_normal((2, kd.K)).astype(np.float32)
    R = kd.orc.gemv_f64_cols(X)
    assert rel_l2(kd.t.mul_mat_vec(X[0])[0], R[0]) < TOL
    Y = kd.t.mul_mat_vec(X)
    for n in range(2):
        assert rel_l2(Y[n], R[n]) < TOL, n


def test_llama_head_shard_single_call(llama):
    kd = llama[7]
    x = np.random.default_rng(77).standard_normal(kd.K).astype(np.float32)
    assert rel_l2(kd.t.mul_mat_vec(x)[0], kd.orc.gemv_f64(x)) < TOL


def test_split_paths_repeat_bitwise(llama):
    """the K-chunk fix-ups (ffn_down single calls: two workgroups per row group; 8 columns: the task kernel with
    K-chunks) 50 times in one process, every result bitwise equal to the first; stops at the first mismatch"""
    kd = llama[6]
    rng = np.random.default_rng(50)
    for ncols in (1, 8):
        X = rng.standard_normal((ncols, kd.K)).astype(np.float32)
        xd = p8x.DeviceBuffer.from_numpy(X)
        yd = p8x.DeviceBuffer(4 * ncols * kd.rows)
        kd.t.mul_mat_vec_dev(xd, yd, ncols=ncols)
        p8x.synchronize()
        first = yd.to_numpy(np.uint32, (ncols, kd.rows))
        assert rel_l2(first.view(np.float32)[0], kd.orc.gemv_f64(X[0])) < TOL
        for rep in range(50):
            yd.fill(0)
            kd.t.mul_mat_vec_dev(xd, yd, ncols=ncols)
            p8x.synchronize()
            assert np.array_equal(yd.to_numpy(np.uint32, (ncols, kd.rows)), first), (ncols, rep)
        xd.free(); yd.free()


def test_qwen3_4b_layer():
    kinds = [Kind(n, r, K, 400 + i) for i, (n, r, K) in enumerate(QWEN4B)]
    rng = np.random.default_rng(4)
    for kd in kinds:   # single calls, one and two columns
        X = rng.standard_normal((2, kd.K)).astype(np.float32)
        R = kd.orc.gemv_f64_cols(X)
        assert rel_l2(kd.t.mul_mat_vec(X[0])[0], R[0]) < TOL, kd.name
        Y = kd.t.mul_mat_vec(X)
        for n in range(2):
            assert rel_l2(Y[n], R[n]) < TOL, (kd.name, n)
    # the benchmark's grouped launch of one layer (a small launch: units of two or more blocks)
    info = grouped_check(kinds, list(range(7)), 1, 5, set(range(7)))
    assert info["small_launch"] == 1
    for k in kinds:
        k.t.release()


@pytest.fixture(scope="module")
def qwen14b():
    kinds = [Kind(n, r, K, 500 + i) for i, (n, r, K) in enumerate(QWEN14B)]
    yield kinds
    for k in kinds:
        k.t.release()


@pytest.mark.parametrize("ncols", [1, 2, 4, 8])
def test_qwen3_14b_single_calls(qwen14b, ncols):
    rng = np.random.default_rng(ncols)
    for kd in qwen14b:
        if kd.name in ("attn_v", "attn_output", "ffn_up"):   # same shapes as attn_k, attn_q, ffn_gate
            continue
        X = rng.standard_normal((ncols, kd.K)).astype(np.float32)
        R = kd.orc.gemv_f64_cols(X)
        Y = kd.t.mul_mat_vec(X)
        for n in range(ncols):
            assert rel_l2(Y[n], R[n]) < TOL, (kd.name, ncols, n)


@pytest.mark.parametrize("ncols", [1, 2, 4, 8])
def test_qwen3_14b_stack_grouped(qwen14b, ncols):
    """the benchmark's 40-layer grouped launch (280 jobs) at 1, 2, 4, 8 columns"""
    plan = [k for _ in range(40) for k in range(7)]
    oracle_jobs = {7 * 20 + k for k in (0, 1, 4, 6)} | {len(plan) - 1}
    info = grouped_check(qwen14b, plan, ncols, 100 + ncols, oracle_jobs)
    assert info["small_launch"] == 0 and info["ncols"] == ncols, info
