"""Batch invariance on the GPU: a row computed in a batch equals the same row computed
alone, bit for bit. The reference engine's self-test demands this of its matmul kernels
("batch of N == N single tokens, bit for bit", src/cuda/cuda_runner.cu:798-829) and
serve-bench --check relies on it end to end (src/main.cpp:845-888): every request served
in a batch must produce the tokens it produces alone. Here it is checked for every dense
op of the decode step (all tilings, BF16 and INT8 weights), for decode attention (every
KV type; the chunk partition fixed, the batch, its chunk count and the launch shape
varied) and for the fused RoPE + append + attention launch."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import NH, NKV, HD, QD, KVD, PAGE, kv_pool, make_tables, normal, to_dev

pytestmark = pytest.mark.gpu


def dev_matrix(ie, dev, w32, int8):
    if int8:
        q, s = O.quantize_i8(w32)
        dq, ds = torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev)
        return ie.matrix(dq, ds), (dq, ds)
    b = O.round_to_kv(np.asarray(w32, np.float32), 2)
    db = torch.from_numpy(b.view(np.int16)).to(dev)
    return ie.matrix(db), (db,)


def same_bits(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.contiguous().view(torch.int32), b.contiguous().view(torch.int32))


# rows, cols: q/k/v stacked, o_proj, gate/up, down, and an LM-head-wide matrix
SHAPES = [(1152, 896), (896, 896), (4864, 896), (896, 4864), (70000, 64)]


@pytest.mark.parametrize("shape", range(len(SHAPES)))
@pytest.mark.parametrize("int8", [False, True])
def test_matmul_batch_of_n_equals_singles(ie, dev, shape, int8):
    rows, cols = SHAPES[shape]
    rng = np.random.default_rng(300 + shape)
    w32 = normal(rng, (rows, cols), 0.05)
    m, keep = dev_matrix(ie, dev, w32, int8)
    bias = torch.from_numpy(normal(rng, rows)).to(dev)
    for T in (2, 13, 31, 64, 100, 300):
        x = torch.from_numpy(normal(rng, (T, cols))).to(dev)
        yb = torch.empty((T, rows), device=dev)
        ie.matmul(yb, x, m, bias)
        y1 = torch.empty((1, rows), device=dev)
        for t in sorted({0, 1, T // 2, T - 1}):
            ie.matmul(y1, x[t:t + 1], m, bias)
            torch.cuda.synchronize()
            assert same_bits(yb[t:t + 1], y1), f"T={T} row {t}"


@pytest.mark.parametrize("int8", [False, True])
def test_gate_up_and_qkv_batch_of_n_equals_singles(ie, dev, int8):
    rng = np.random.default_rng(17)
    H, I = 896, 4864
    mg, kg = dev_matrix(ie, dev, normal(rng, (I, H), 0.05), int8)
    mu, ku = dev_matrix(ie, dev, normal(rng, (I, H), 0.05), int8)
    mq, kq = dev_matrix(ie, dev, normal(rng, (QD + 2 * KVD, H), 0.05), int8)
    bq = torch.from_numpy(normal(rng, QD + 2 * KVD)).to(dev)
    for T in (2, 31, 64, 1024):
        x = torch.from_numpy(normal(rng, (T, H))).to(dev)
        gb = torch.empty((T, I), device=dev)
        ie.gate_up_silu(gb, x, mg, mu)
        qb, kb, vb = (torch.empty((T, n), device=dev) for n in (QD, KVD, KVD))
        ie.qkv_proj(qb, kb, vb, x, mq, bq)
        g1 = torch.empty((1, I), device=dev)
        q1, k1, v1 = (torch.empty((1, n), device=dev) for n in (QD, KVD, KVD))
        for t in sorted({0, T // 3, T - 1}):
            ie.gate_up_silu(g1, x[t:t + 1], mg, mu)
            ie.qkv_proj(q1, k1, v1, x[t:t + 1], mq, bq)
            torch.cuda.synchronize()
            assert same_bits(gb[t:t + 1], g1), f"gate/up T={T} row {t}"
            for a, b in ((qb, q1), (kb, k1), (vb, v1)):
                assert same_bits(a[t:t + 1], b), f"qkv T={T} row {t}"


def test_rmsnorm_batch_of_n_equals_singles(ie, dev):
    rng = np.random.default_rng(5)
    x = torch.from_numpy(normal(rng, (64, 896), 3.0)).to(dev)
    w = torch.from_numpy(normal(rng, 896)).to(dev)
    yb = torch.empty_like(x)
    ie.rmsnorm(yb, x, w, 1e-6)
    y1 = torch.empty((1, 896), device=dev)
    for t in (0, 17, 63):
        ie.rmsnorm(y1, x[t:t + 1], w, 1e-6)
        torch.cuda.synchronize()
        assert same_bits(yb[t:t + 1], y1)


def _paged_batch(rng, lens, kv_dtype, seed_pages=3):
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=seed_pages)
    kp = kv_pool(rng, num_pages, kv_dtype, O)
    vp = kv_pool(rng, num_pages, kv_dtype, O)
    q = normal(rng, (len(lens), QD))
    return tables, max_pages, kp, vp, q


@pytest.mark.parametrize("kv", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("chunk_tokens", [64, 128, 256])
def test_attention_row_alone_equals_row_in_batch(ie, dev, kv, chunk_tokens):
    """64 ragged rows (contexts 1 .. 4,096) in one launch, then rows alone: the launch
    grid, the workspace's chunk count and the merge's launch shape all change; the
    outputs must not."""
    kvd = {"f32": 0, "f16": 1, "bf16": 2}[kv]
    rng = np.random.default_rng(41 + kvd)
    lens = [int(x) for x in rng.integers(1, 4097, 64)]
    lens[:4] = [1, chunk_tokens, chunk_tokens + 1, 4096]
    tables, max_pages, kp, vp, q = _paged_batch(rng, lens, kvd)
    dkp, dvp = to_dev(kp, dev, kvd), to_dev(vp, dev, kvd)
    dtab = to_dev(tables, dev)
    T = len(lens)
    pos = np.array([n - 1 for n in lens], np.int32)
    seq = np.arange(T, dtype=np.int32)
    nc = ie.attention_chunks(4096, chunk_tokens)
    ws = ie.attention_workspace(T, NH, HD, nc)
    out_b = torch.empty((T, QD), device=dev)
    ie.attention(out_b, to_dev(q, dev), dkp, dvp, to_dev(pos, dev), to_dev(seq, dev), dtab,
                 max_pages, nc, chunk_tokens, ws, NH, NKV, HD)
    out_1 = torch.empty((1, QD), device=dev)
    for t in [0, 1, 2, 3, 10, 33, 63]:
        own = ie.attention_chunks(lens[t], chunk_tokens)
        for n_chunks in sorted({own, nc + 5}):  # just enough, and more than the batch's
            ws1 = ie.attention_workspace(1, NH, HD, n_chunks)
            ie.attention(out_1, to_dev(q[t:t + 1], dev), dkp, dvp, to_dev(pos[t:t + 1], dev),
                         to_dev(seq[t:t + 1], dev), dtab, max_pages, n_chunks, chunk_tokens, ws1,
                         NH, NKV, HD)
            torch.cuda.synchronize()
            assert same_bits(out_b[t:t + 1], out_1), f"row {t} (len {lens[t]}), {n_chunks} chunks"


@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_fused_step_row_alone_equals_row_in_batch(ie, dev, kv):
    """The decode step's fused RoPE + append + attention: each row's pages and output
    are the same in a batch of 64 as in a batch of one."""
    kvd = {"f16": 1, "bf16": 2}[kv]
    rng = np.random.default_rng(77 + kvd)
    lens = [int(x) for x in rng.integers(2, 4097, 64)]
    tables, max_pages, kp, vp, q = _paged_batch(rng, lens, kvd)
    T = len(lens)
    k = normal(rng, (T, KVD))
    v = normal(rng, (T, KVD))
    pos = np.array([n - 1 for n in lens], np.int32)
    seq = np.arange(T, dtype=np.int32)
    ct = 128
    assert ie.rope_cache_attention_supported(kvd, NH, NKV, HD, ct)
    table = ie.rope_table(4096, HD, 1e6).to(dev)
    dtab = to_dev(tables, dev)
    nc = ie.attention_chunks(4096, ct)
    dkp, dvp = to_dev(kp, dev, kvd), to_dev(vp, dev, kvd)
    out_b = torch.empty((T, QD), device=dev)
    ie.rope_cache_attention(out_b, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), dkp, dvp,
                            table, to_dev(pos, dev), to_dev(seq, dev), dtab, max_pages, nc, ct,
                            ie.attention_workspace(T, NH, HD, nc), NH, NKV, HD)
    torch.cuda.synchronize()
    kb, vb = dkp.clone(), dvp.clone()
    dkp, dvp = to_dev(kp, dev, kvd), to_dev(vp, dev, kvd)  # fresh pools, rows one at a time
    out_1 = torch.empty((T, QD), device=dev)
    for t in range(T):
        n1 = ie.attention_chunks(lens[t], ct)
        ie.rope_cache_attention(out_1[t:t + 1], to_dev(q[t:t + 1], dev), to_dev(k[t:t + 1], dev),
                                to_dev(v[t:t + 1], dev), dkp, dvp, table, to_dev(pos[t:t + 1], dev),
                                to_dev(seq[t:t + 1], dev), dtab, max_pages, n1, ct,
                                ie.attention_workspace(1, NH, HD, n1), NH, NKV, HD)
    torch.cuda.synchronize()
    assert torch.equal(kb.view(torch.int16), dkp.view(torch.int16))
    assert torch.equal(vb.view(torch.int16), dvp.view(torch.int16))
    assert same_bits(out_b, out_1)
