"""Oracle pinning for the decode step's layer ops: matmul over F32 / BF16 / I8 weights,
int8 quantization, the embedding row lookup, rmsnorm and silu.

Each oracle function is checked bit-exactly against the reference's own CPU code compiled
from its sources into oracle/_ref (src/matrix.cpp scalar kernel, src/ops.cpp rmsnorm and
silu), and against what the mathematics fixes: identity and one-hot weight matrices,
constant rows, float64 dot products. The reference's default matmul kernel is AVX2, whose
summation order differs; it is checked here to the same float64 tolerance."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
SHAPES = [(1, 7, 16), (5, 37, 96), (64, 128, 896), (3, 896, 896), (2, 130, 4864)]


def bf16(x):
    return O.round_to_kv(np.asarray(x, np.float32), 2)


def widen(bits):
    return O.widen_kv(bits, 2).reshape(bits.shape)


def weights(rng, rows, cols):
    wb = bf16(rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05))
    return wb, widen(wb)


@needs_ref
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", [O.W_F32, O.W_BF16, O.W_I8])
def test_matmul_bitexact_vs_reference_scalar(shape, dtype):
    T, rows, cols = shape
    rng = np.random.default_rng(rows * 7 + cols + dtype)
    x = rng.standard_normal((T, cols), dtype=np.float32)
    wb, wf = weights(rng, rows, cols)
    bias = rng.standard_normal(rows, dtype=np.float32) if dtype != O.W_I8 else None
    want, sc, q = O.ref_matmul_bf16(x, wb, dtype, bias, kernel=0)
    if dtype == O.W_F32:
        got = O.matmul(x, wf, O.W_F32, None, bias)
    elif dtype == O.W_BF16:
        got = O.matmul(x, wb, O.W_BF16, None, bias)
    else:
        q2, s2 = O.quantize_i8(wf)
        assert np.array_equal(q2, q) and np.array_equal(s2.view(np.uint32), sc.view(np.uint32))
        got = O.matmul(x, q2, O.W_I8, s2, bias)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("dtype", [O.W_F32, O.W_BF16, O.W_I8])
def test_matmul_reference_avx2_within_fp64_tolerance(dtype):
    """The reference's default (AVX2) kernel sums in another order: both it and the oracle
    sit within float32 rounding of the float64 product."""
    rng = np.random.default_rng(11 + dtype)
    T, rows, cols = 8, 256, 896
    x = rng.standard_normal((T, cols), dtype=np.float32)
    wb, wf = weights(rng, rows, cols)
    avx, sc, q = O.ref_matmul_bf16(x, wb, dtype, None, kernel=1)
    w64 = (q.astype(np.float64) * sc[:, None].astype(np.float64)) if dtype == O.W_I8 else wf.astype(np.float64)
    exact = x.astype(np.float64) @ w64.T
    got = (O.matmul(x, q, O.W_I8, sc) if dtype == O.W_I8 else
           O.matmul(x, wb if dtype == O.W_BF16 else wf, dtype))
    scale = np.abs(exact).max()
    assert np.abs(got - exact).max() / scale < 1e-6
    assert np.abs(avx - exact).max() / scale < 1e-6


@pytest.mark.parametrize("dtype", [O.W_F32, O.W_BF16])
def test_matmul_identity_and_one_hot(dtype):
    """Identity weights give x + bias exactly; a one-hot row picks one input column."""
    rng = np.random.default_rng(3)
    n = 64
    x = rng.standard_normal((4, n), dtype=np.float32)
    b = rng.standard_normal(n, dtype=np.float32)
    eye = np.eye(n, dtype=np.float32)
    w = bf16(eye) if dtype == O.W_BF16 else eye
    y = O.matmul(x, w, dtype, None, b)
    assert np.array_equal(y, x + b)
    perm = rng.permutation(n)
    hot = np.zeros((n, n), np.float32)
    hot[np.arange(n), perm] = 1.0
    w = bf16(hot) if dtype == O.W_BF16 else hot
    assert np.array_equal(O.matmul(x, w, dtype), x[:, perm])


def test_matmul_i8_scale_applied_after_the_sum():
    """I8: y = (sum q x) * scale + bias, with q the rounded weight / scale."""
    rng = np.random.default_rng(4)
    w = rng.standard_normal((32, 48), dtype=np.float32)
    q, s = O.quantize_i8(w)
    assert np.all(np.abs(q) <= 127) and np.all(np.abs(q).max(axis=1) == 127)
    assert np.allclose(q * s[:, None], w, atol=np.max(s) / 2 + 1e-7)
    x = rng.standard_normal((3, 48), dtype=np.float32)
    exact = (x.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)
    assert np.abs(O.matmul(x, q, O.W_I8, s) - exact).max() < 1e-5
    zero_q, zero_s = O.quantize_i8(np.zeros((2, 8), np.float32))
    assert np.all(zero_q == 0) and np.all(zero_s == 1.0)


@needs_ref
@pytest.mark.parametrize("dtype", [O.W_F32, O.W_BF16, O.W_I8])
def test_row_to_f32_vs_reference(dtype):
    rng = np.random.default_rng(6)
    wb, wf = weights(rng, 20, 896)
    q, s = O.quantize_i8(wf)
    for r in (0, 7, 19):
        want = O.ref_row_to_f32(wb, dtype, r)
        got = (O.row_to_f32(q, O.W_I8, r, s) if dtype == O.W_I8 else
               O.row_to_f32(wb if dtype == O.W_BF16 else wf, dtype, r))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("dim", [64, 96, 896, 4864])
def test_rmsnorm_bitexact_vs_reference(dim):
    rng = np.random.default_rng(dim)
    x = rng.standard_normal((6, dim), dtype=np.float32) * np.float32(3.0)
    w = rng.standard_normal(dim, dtype=np.float32)
    got = O.rmsnorm(x, w, 1e-6)
    want = O.ref_rmsnorm(x, w, 1e-6)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_rmsnorm_closed_forms():
    """A constant row c gives w * c / sqrt(c^2 + eps); float64 agreement elsewhere."""
    w = np.linspace(-2, 2, 896).astype(np.float32)
    for c in (1.0, -3.5, 0.25):
        y = O.rmsnorm(np.full((1, 896), c, np.float32), w, 1e-6)[0]
        want = w.astype(np.float64) * c / np.sqrt(c * c + 1e-6)
        assert np.abs(y - want).max() < 1e-6 * np.abs(want).max()
    rng = np.random.default_rng(9)
    x = rng.standard_normal((5, 896), dtype=np.float32)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-6) * w
    assert np.abs(O.rmsnorm(x, w, 1e-6) - want).max() < 1e-5


@needs_ref
def test_silu_bitexact_vs_reference_and_closed_forms():
    rng = np.random.default_rng(10)
    g = np.concatenate([rng.standard_normal(4000, dtype=np.float32) * np.float32(6.0),
                        np.array([0.0, -0.0, 30.0, -30.0, 88.0, -88.0], np.float32)])
    u = rng.standard_normal(g.size, dtype=np.float32)
    got = O.silu_mul(g, np.ones_like(g))
    want = np.array([O.ref_silu(float(v)) for v in g], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert got[-6] == 0.0 and abs(got[-4] - 30.0) < 1e-5 and abs(got[-3]) < 1e-10
    g64 = g.astype(np.float64)
    assert np.abs(O.silu_mul(g, u) - g64 / (1 + np.exp(-g64)) * u).max() < 1e-5
