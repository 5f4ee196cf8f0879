"""GPU parity of the prompt GEMM (p8x_mul_mat) against fp64 products of the oracle's dequantized weights.

The reference is independent of the kernel's algebra: y = W x with W the oracle's bit-exact dequant (original
rows, Hadamard applied, clamp delta included) in fp64. Bar: relative L2 below 1e-3 (the kernel rounds x' and
v S to fp16 once each, about 3e-4 combined).
"""
import numpy as np
import pytest

import oracle as O
import p8x

pytestmark = pytest.mark.gpu
REL_L2 = 1e-3
ALL = (1, 1, 1, 1, 1, 1, 1, 1)
C3 = (0, 0, 0, 1, 0, 0, 0, 0)


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def to_bf16(X):
    u = np.ascontiguousarray(X, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(B):
    return (B.astype(np.uint32) << 16).view(np.float32)


def reference(orc, X, tokens=None):
    W = orc.dequant()
    Xs = X if tokens is None else X[tokens]
    return O.dense_f64(W, np.ascontiguousarray(Xs, np.float32))


@pytest.mark.parametrize("rows,K,cp,N,nd", [
    (256, 1024, C3, 128, 0), (256, 1024, C3, 1, 3), (512, 2048, C3, 130, 5), (96, 512, ALL, 37, 4),
    (1024, 2560, ALL, 300, 9), (2048, 4096, (0, 0, 1, 6, 1, 0, 0, 0), 256, 2)])
def test_gemm_f32(rows, K, cp, N, nd):
    slot = p8x.synth_random(rows * 7 + N, rows, K, class_p=cp, nd=nd)
    t = p8x.Tensor(slot, rows, K)
    orc = O.Oracle(slot, rows, K)
    X = np.random.default_rng(N).standard_normal((N, K)).astype(np.float32)
    Y = t.mul_mat(X, p8x.F32)
    assert rel_l2(Y, reference(orc, X)) < REL_L2


@pytest.mark.parametrize("rows,K,N", [(512, 1536, 200), (64, 256, 9)])
def test_gemm_bf16(rows, K, N):
    slot = p8x.synth_random(rows + K, rows, K, class_p=ALL, nd=6)
    t = p8x.Tensor(slot, rows, K)
    orc = O.Oracle(slot, rows, K)
    Xb = to_bf16(np.random.default_rng(K).standard_normal((N, K)))
    Y = t.mul_mat(Xb, p8x.BF16)
    assert rel_l2(Y, reference(orc, bf16_to_f32(Xb))) < REL_L2


def test_gemm_matches_gemv_columns():
    """the GEMM and the multi-column GEMV agree on the same weights (different activation quantization, so the
    comparison goes through fp64: both within tolerance of the same reference)"""
    rows, K, N = 768, 3072, 8
    slot = p8x.synth_random(11, rows, K, class_p=ALL, nd=3)
    t = p8x.Tensor(slot, rows, K)
    orc = O.Oracle(slot, rows, K)
    X = np.random.default_rng(11).standard_normal((N, K)).astype(np.float32)
    ref = reference(orc, X)
    assert rel_l2(t.mul_mat(X), ref) < REL_L2
    assert rel_l2(t.mul_mat_vec(X), ref) < 2e-2   # 8-bit activations


def test_gemm_deterministic_and_split():
    """a deep-K shape takes the K-split path; two runs are bitwise equal"""
    rows, K, N = 512, 14336, 64
    slot = p8x.synth_random(5, rows, K, nd=4)
    t = p8x.Tensor(slot, rows, K)
    X = np.random.default_rng(5).standard_normal((N, K)).astype(np.float32)
    a = t.mul_mat(X)
    b = t.mul_mat(X)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    orc = O.Oracle(slot, rows, K)
    assert rel_l2(a, reference(orc, X)) < REL_L2


@pytest.mark.parametrize("rows,K", [(14336, 4096), (4096, 14336)])
def test_gemm_ffn_512(rows, K):
    """the Llama-3.1-8B FFN shapes at 512 bf16 tokens; fp64 check on a sample of 12 tokens"""
    N = 512
    slot = p8x.synth_random(rows ^ K, rows, K, nd=8)
    t = p8x.Tensor(slot, rows, K)
    orc = O.Oracle(slot, rows, K)
    Xb = to_bf16(np.random.default_rng(rows).standard_normal((N, K)))
    Y = t.mul_mat(Xb, p8x.BF16)
    tok = np.array([0, 1, 31, 32, 127, 128, 200, 255, 256, 383, 500, 511])
    assert rel_l2(Y[tok], reference(orc, bf16_to_f32(Xb), tok)) < REL_L2
    assert np.isfinite(Y).all()


def test_gemm_wide_tile_2000_tokens():
    """2000 tokens of the 14336 x 4096 shape: the plan takes the 256-token workgroup tile (8 MFMA token tiles per
    wave), whose last tile runs past N; fp64 check on tokens of the first, a middle and the last tile"""
    rows, K, N = 14336, 4096, 2000
    slot = p8x.synth_random(2000, rows, K, nd=5)
    t = p8x.Tensor(slot, rows, K)
    orc = O.Oracle(slot, rows, K)
    Xb = to_bf16(np.random.default_rng(2000).standard_normal((N, K)))
    Y = t.mul_mat(Xb, p8x.BF16)
    tok = np.array([0, 1, 255, 256, 1000, 1791, 1792, 1900, 1998, 1999])
    assert rel_l2(Y[tok], reference(orc, bf16_to_f32(Xb), tok)) < REL_L2
    assert np.isfinite(Y).all()


def test_gemm_identity_rows_direct_output():
    """identity row order and one K range: k_mm writes y itself (no planes) and a separate launch adds the clamp
    delta; 250 tokens, so the last token tile runs past N"""
    rows, K, N = 14336, 1024, 250
    slot = p8x.synth_random(77, rows, K, nd=6, permute=False)
    t = p8x.Tensor(slot, rows, K)
    orc = O.Oracle(slot, rows, K)
    X = np.random.default_rng(77).standard_normal((N, K)).astype(np.float32)
    Y = t.mul_mat(X, p8x.F32)
    tok = np.array([0, 1, 127, 128, 200, 248, 249])
    assert rel_l2(Y[tok], reference(orc, X, tok)) < REL_L2
    assert np.isfinite(Y).all()


def test_gemm_reserve_then_smaller_calls():
    """workspace reserved for 300 tokens serves calls with 300 and fewer tokens, results unchanged"""
    rows, K = 512, 4096
    slot = p8x.synth_random(21, rows, K, nd=2)
    t = p8x.Tensor(slot, rows, K)
    t.mul_mat_reserve(300)
    orc = O.Oracle(slot, rows, K)
    for N in (300, 17, 128):
        X = np.random.default_rng(N).standard_normal((N, K)).astype(np.float32)
        assert rel_l2(t.mul_mat(X), reference(orc, X)) < REL_L2
