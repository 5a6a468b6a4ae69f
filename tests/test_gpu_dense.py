"""The decode step's dense ops on the GPU vs the CPU oracle (itself bit-exact with the
reference's src/matrix.cpp and src/ops.cpp): embedding (exact), rmsnorm, matmul with BF16
and INT8 weights (bias, residual accumulation, ragged shapes), the fused gate/up + SiLU.

Tolerance: the fp32 bar of the north star, max |d| / max |ref| <= 1e-5 (the reference's
metric, src/npy.cpp:98-110). Only summation order differs: the MFMA kernel multiplies the
weights (exact in bf16) by each activation split into three bf16 parts, which is the exact
f32 product."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
REL = 1e-5


def rel_err(got, want):
    return O.compare(got, want)[0]


def bf16_bits(x):
    return O.round_to_kv(np.asarray(x, np.float32), 2)


def widen(bits):
    return O.widen_kv(bits, 2).reshape(bits.shape)


def dev_weights(ie, dev, w32, int8):
    """(ie_matrix, keep-alive tensors, oracle args) for f32 master weights."""
    if int8:
        q, s = O.quantize_i8(w32)
        dq = torch.from_numpy(q).to(dev)
        ds = torch.from_numpy(s).to(dev)
        return ie.matrix(dq, ds), (dq, ds), (q, O.W_I8, s)
    b = bf16_bits(w32)
    db = torch.from_numpy(b.view(np.int16)).to(dev)
    return ie.matrix(db), (db,), (b, O.W_BF16, None)


@pytest.mark.parametrize("int8", [False, True])
def test_embedding_exact(ie, dev, int8):
    rng = np.random.default_rng(1)
    vocab, dim = 1000, 896
    table = rng.standard_normal((vocab, dim), dtype=np.float32)
    m, keep, (w, fmt, s) = dev_weights(ie, dev, table, int8)
    ids = np.array([0, vocab - 1, 5, 5, 731, 2], np.int32)
    x = torch.full((ids.size, dim), float("nan"), device=dev)
    ie.embedding(x, torch.from_numpy(ids).to(dev), m)
    torch.cuda.synchronize()
    got = x.cpu().numpy()
    want = np.stack([O.row_to_f32(w, fmt, int(i), s) for i in ids])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dim", [64, 896, 4864])
@pytest.mark.parametrize("in_place", [False, True])
def test_rmsnorm(ie, dev, dim, in_place):
    rng = np.random.default_rng(dim)
    x = rng.standard_normal((33, dim), dtype=np.float32) * np.float32(4.0)
    w = rng.standard_normal(dim, dtype=np.float32)
    dx = torch.from_numpy(x).to(dev)
    y = dx if in_place else torch.empty_like(dx)
    ie.rmsnorm(y, dx, torch.from_numpy(w).to(dev), 1e-6)
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), O.rmsnorm(x, w, 1e-6)) <= REL


MATMULS = [
    # T, rows, cols, bias, accumulate
    (1, 896, 896, True, False),      # q_proj, one token
    (64, 128, 896, True, False),     # k/v_proj at decode batch 64
    (64, 896, 896, False, True),     # o_proj into the residual
    (64, 896, 4864, False, True),    # down_proj into the residual
    (37, 130, 104, True, True),      # ragged: rows % 16, cols % 32, T % 16 all nonzero
    (300, 896, 896, True, False),    # a prompt chunk
    (64, 9000, 128, False, True),    # 2 row tiles per workgroup (>= 4 tiles per compute unit)
    (40, 120000, 32, True, False),   # 4 x 4 tiles (>= 64 per unit), 3 token tiles rounded to 4
    (64, 70000, 64, False, True),    # 4 x 4 tiles, every token in one workgroup
    (20, 210000, 16, True, False),   # 4 x 2 tiles
]


@pytest.mark.parametrize("case", range(len(MATMULS)))
@pytest.mark.parametrize("int8", [False, True])
def test_matmul(ie, dev, case, int8):
    T, rows, cols, with_bias, acc = MATMULS[case]
    rng = np.random.default_rng(100 + case)
    x = rng.standard_normal((T, cols), dtype=np.float32)
    w32 = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05)
    bias = rng.standard_normal(rows, dtype=np.float32) if with_bias else None
    y0 = rng.standard_normal((T, rows), dtype=np.float32)
    m, keep, (w, fmt, s) = dev_weights(ie, dev, w32, int8)
    y = torch.from_numpy(y0).to(dev)
    ie.matmul(y, torch.from_numpy(x).to(dev), m,
              None if bias is None else torch.from_numpy(bias).to(dev), accumulate=acc)
    torch.cuda.synchronize()
    want = O.matmul(x, w, fmt, s, bias)
    if acc:
        want = want + y0  # the CPU adds the projection into x afterwards (src/model.cpp:80)
    assert rel_err(y.cpu().numpy(), want) <= REL


@pytest.mark.parametrize("int8", [False, True])
@pytest.mark.parametrize("T", [1, 64, 1024])
def test_gate_up_silu(ie, dev, int8, T):
    """T = 1,024 at 4,864 rows has more than 64 output tiles per compute unit: the launch
    must still size its grid for the 2-row-tile gate kernel it runs."""
    rng = np.random.default_rng(7 + T)
    rows, cols = 4864, 896
    x = rng.standard_normal((T, cols), dtype=np.float32)
    wg32 = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05)
    wu32 = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05)
    mg, kg, (wg, fmt, sg) = dev_weights(ie, dev, wg32, int8)
    mu, ku, (wu, _, su) = dev_weights(ie, dev, wu32, int8)
    out = torch.full((T, rows), float("nan"), device=dev)
    ie.gate_up_silu(out, torch.from_numpy(x).to(dev), mg, mu)
    torch.cuda.synchronize()
    want = O.silu_mul(O.matmul(x, wg, fmt, sg), O.matmul(x, wu, fmt, su))
    assert rel_err(out.cpu().numpy(), want) <= REL


@pytest.mark.parametrize("int8", [False, True])
@pytest.mark.parametrize("T", [1, 64, 300])
def test_qkv_proj_matches_three_matmuls(ie, dev, int8, T):
    """The one-launch q/k/v projection: Wq, Wk, Wv stacked, each output to its own buffer."""
    rng = np.random.default_rng(20 + T)
    H, QD, KVD = 896, 896, 128
    x = rng.standard_normal((T, H), dtype=np.float32)
    w32 = rng.standard_normal((QD + 2 * KVD, H), dtype=np.float32) * np.float32(0.05)
    b = rng.standard_normal(QD + 2 * KVD, dtype=np.float32)
    m, keep, (w, fmt, s) = dev_weights(ie, dev, w32, int8)
    q = torch.full((T, QD), float("nan"), device=dev)
    k = torch.full((T, KVD), float("nan"), device=dev)
    v = torch.full((T, KVD), float("nan"), device=dev)
    ie.qkv_proj(q, k, v, torch.from_numpy(x).to(dev), m, torch.from_numpy(b).to(dev))
    torch.cuda.synchronize()
    want = O.matmul(x, w, fmt, s, b)
    assert rel_err(q.cpu().numpy(), want[:, :QD]) <= REL
    assert rel_err(k.cpu().numpy(), want[:, QD:QD + KVD]) <= REL
    assert rel_err(v.cpu().numpy(), want[:, QD + KVD:]) <= REL


EPS = 1e-6


@pytest.mark.parametrize("int8", [False, True])
@pytest.mark.parametrize("T", [1, 64, 300])
def test_rmsnorm_qkv_proj(ie, dev, int8, T):
    """The input norm folded into the q/k/v projection: against the oracle's rmsnorm
    followed by the projection (the reference's two launches)."""
    rng = np.random.default_rng(40 + T)
    H, QD, KVD = 896, 896, 128
    x = rng.standard_normal((T, H), dtype=np.float32) * np.float32(4.0)
    wn = rng.standard_normal(H, dtype=np.float32)
    w32 = rng.standard_normal((QD + 2 * KVD, H), dtype=np.float32) * np.float32(0.05)
    b = rng.standard_normal(QD + 2 * KVD, dtype=np.float32)
    m, keep, (w, fmt, s) = dev_weights(ie, dev, w32, int8)
    q = torch.full((T, QD), float("nan"), device=dev)
    k = torch.full((T, KVD), float("nan"), device=dev)
    v = torch.full((T, KVD), float("nan"), device=dev)
    ie.rmsnorm_qkv_proj(q, k, v, torch.from_numpy(x).to(dev), torch.from_numpy(wn).to(dev), EPS,
                        m, torch.from_numpy(b).to(dev))
    torch.cuda.synchronize()
    want = O.matmul(O.rmsnorm(x, wn, EPS), w, fmt, s, b)
    assert rel_err(q.cpu().numpy(), want[:, :QD]) <= REL
    assert rel_err(k.cpu().numpy(), want[:, QD:QD + KVD]) <= REL
    assert rel_err(v.cpu().numpy(), want[:, QD + KVD:]) <= REL


@pytest.mark.parametrize("int8", [False, True])
@pytest.mark.parametrize("T", [1, 64, 1024])
def test_rmsnorm_gate_up_silu(ie, dev, int8, T):
    """The post-attention norm folded into gate/up + SiLU, against the oracle's rmsnorm
    followed by the two projections and silu(g) * u."""
    rng = np.random.default_rng(50 + T)
    rows, cols = 4864, 896
    x = rng.standard_normal((T, cols), dtype=np.float32) * np.float32(4.0)
    wn = rng.standard_normal(cols, dtype=np.float32)
    wg32 = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05)
    wu32 = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05)
    mg, kg, (wg, fmt, sg) = dev_weights(ie, dev, wg32, int8)
    mu, ku, (wu, _, su) = dev_weights(ie, dev, wu32, int8)
    out = torch.full((T, rows), float("nan"), device=dev)
    ie.rmsnorm_gate_up_silu(out, torch.from_numpy(x).to(dev), torch.from_numpy(wn).to(dev), EPS,
                            mg, mu)
    torch.cuda.synchronize()
    xn = O.rmsnorm(x, wn, EPS)
    want = O.silu_mul(O.matmul(xn, wg, fmt, sg), O.matmul(xn, wu, fmt, su))
    assert rel_err(out.cpu().numpy(), want) <= REL


@pytest.mark.parametrize("int8", [False, True])
@pytest.mark.parametrize("cols", [32, 96, 2080, 4864])
def test_rmsnorm_folds_widths(ie, dev, int8, cols):
    """Both folds at hidden widths other than 896: the norm weight reaches LDS in
    16-byte pieces, 64 to a wave and 512 to a pass of the 8 waves, so 32 and 96 leave
    most lanes idle, 2,080 (520 pieces) takes a second pass and 4,864 three."""
    rng = np.random.default_rng(60 + cols)
    T, rows = 17, 96
    x = rng.standard_normal((T, cols), dtype=np.float32) * np.float32(4.0)
    wn = rng.standard_normal(cols, dtype=np.float32)
    wg32 = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05)
    wu32 = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05)
    mg, kg, (wg, fmt, sg) = dev_weights(ie, dev, wg32, int8)
    mu, ku, (wu, _, su) = dev_weights(ie, dev, wu32, int8)
    dx, dwn = torch.from_numpy(x).to(dev), torch.from_numpy(wn).to(dev)
    out = torch.full((T, rows), float("nan"), device=dev)
    ie.rmsnorm_gate_up_silu(out, dx, dwn, EPS, mg, mu)
    QD, KVD = 64, 16
    b = rng.standard_normal(QD + 2 * KVD, dtype=np.float32)
    wq32 = rng.standard_normal((QD + 2 * KVD, cols), dtype=np.float32) * np.float32(0.05)
    mq, kq, (wq, fmtq, sq) = dev_weights(ie, dev, wq32, int8)
    q = torch.full((T, QD), float("nan"), device=dev)
    k = torch.full((T, KVD), float("nan"), device=dev)
    v = torch.full((T, KVD), float("nan"), device=dev)
    ie.rmsnorm_qkv_proj(q, k, v, dx, dwn, EPS, mq, torch.from_numpy(b).to(dev))
    torch.cuda.synchronize()
    xn = O.rmsnorm(x, wn, EPS)
    want = O.silu_mul(O.matmul(xn, wg, fmt, sg), O.matmul(xn, wu, fmt, su))
    assert rel_err(out.cpu().numpy(), want) <= REL
    wq_ = O.matmul(xn, wq, fmtq, sq, b)
    assert rel_err(q.cpu().numpy(), wq_[:, :QD]) <= REL
    assert rel_err(k.cpu().numpy(), wq_[:, QD:QD + KVD]) <= REL
    assert rel_err(v.cpu().numpy(), wq_[:, QD + KVD:]) <= REL


def test_rmsnorm_folds_batch_invariant(ie, dev):
    """A row's output is the same bits in a batch of 64 as alone (the sum of squares is
    reduced in an order fixed by the matrix shape)."""
    rng = np.random.default_rng(60)
    H, QD, KVD, rows = 896, 896, 128, 4864
    x = rng.standard_normal((64, H), dtype=np.float32) * np.float32(4.0)
    wn = torch.from_numpy(rng.standard_normal(H, dtype=np.float32)).to(dev)
    m, keep, _ = dev_weights(ie, dev, rng.standard_normal((QD + 2 * KVD, H), dtype=np.float32) *
                            np.float32(0.05), False)
    mg, kg, _ = dev_weights(ie, dev, rng.standard_normal((rows, H), dtype=np.float32) *
                            np.float32(0.05), False)
    mu, ku, _ = dev_weights(ie, dev, rng.standard_normal((rows, H), dtype=np.float32) *
                            np.float32(0.05), False)

    def run(xs):
        T = xs.shape[0]
        q, k, v = (torch.empty((T, n), device=dev) for n in (QD, KVD, KVD))
        g = torch.empty((T, rows), device=dev)
        dx = torch.from_numpy(np.ascontiguousarray(xs)).to(dev)
        ie.rmsnorm_qkv_proj(q, k, v, dx, wn, EPS, m)
        ie.rmsnorm_gate_up_silu(g, dx, wn, EPS, mg, mu)
        torch.cuda.synchronize()
        return [t.cpu().numpy() for t in (q, k, v, g)]

    batch = run(x)
    for t in (0, 17, 63):
        alone = run(x[t:t + 1])
        for b_, a_ in zip(batch, alone):
            assert np.array_equal(b_[t:t + 1].view(np.uint32), a_.view(np.uint32)), t


def test_rmsnorm_fold_errors(ie, dev):
    x = torch.zeros((4, 896), device=dev)
    w = torch.zeros((16, 896), dtype=torch.int16, device=dev)
    q, k, v = (torch.zeros((4, n), device=dev) for n in (8, 4, 4))
    with pytest.raises(ie.IeHipError, match="null pointer"):
        ie.rmsnorm_qkv_proj(q, k, v, x, None, EPS, ie.matrix(w))
    wn = torch.zeros(897, device=dev)[1:]  # 4-byte aligned only
    with pytest.raises(ie.IeHipError, match="aligned"):
        ie.rmsnorm_gate_up_silu(torch.zeros((4, 16), device=dev), x, wn, EPS, ie.matrix(w),
                                ie.matrix(w))


def test_dense_argument_errors(ie, dev):
    x = torch.zeros((4, 12), device=dev)
    y = torch.zeros((4, 16), device=dev)
    w = torch.zeros((16, 12), dtype=torch.int16, device=dev)
    with pytest.raises(ie.IeHipError, match="multiple of 8"):
        ie.matmul(y, x, ie.matrix(w))
    q = torch.zeros((16, 16), dtype=torch.int8, device=dev)
    bad = ie.Matrix(q.data_ptr(), None, 1, 16, 16)
    with pytest.raises(ie.IeHipError, match="scales"):
        ie.matmul(y, torch.zeros((4, 16), device=dev), bad)
    w1 = torch.zeros((16, 16), dtype=torch.int16, device=dev)
    w2 = torch.zeros((8, 16), dtype=torch.int16, device=dev)
    with pytest.raises(ie.IeHipError, match="shapes differ"):
        ie.gate_up_silu(y, torch.zeros((4, 16), device=dev), ie.matrix(w1), ie.matrix(w2))
