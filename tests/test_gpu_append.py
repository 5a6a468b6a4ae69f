"""Fused RoPE + paged KV append on the GPU vs the CPU oracle: bit-exact.

Compares every byte of both page pools (untouched rows must stay as they
were) and the rotated queries, for f32, f16 and bf16 caches, on the reference
self-test's rows (src/cuda/cuda_runner.cu:849-903), random batches, page and
position edges, and BASELINE config 2 at full size (64 rows, 65,536-page pool).
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from helpers import HD, KVD, NH, NKV, QD, THETA, from_dev, kv_pool, make_tables, normal, to_dev

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KVS = {"f32": 0, "f16": 1, "bf16": 2}


def run_case(ie, O, dev, kvt, tables, max_pages, num_pages, row_seq, row_pos, q, k, v, rng,
             with_q=True, table_positions=None):
    kp = kv_pool(rng, num_pages, kvt, O)
    vp = kv_pool(rng, num_pages, kvt, O)
    q_ref, kp_ref, vp_ref = O.rope_append_paged(q, k, v, kp, vp, kvt, row_pos, row_seq, tables,
                                                max_pages, NH, NKV, HD, THETA)
    n_pos = table_positions or int(np.max(row_pos)) + 1
    table = ie.rope_table(n_pos, HD, THETA).to(dev)
    dq = to_dev(q, dev) if with_q else None
    dkp, dvp = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt)
    ie.rope_and_cache(dq, to_dev(k, dev), to_dev(v, dev), dkp, dvp, table, to_dev(row_pos, dev),
                      to_dev(row_seq, dev), to_dev(tables, dev), max_pages, NH, NKV, HD)
    torch.cuda.synchronize()
    if with_q:
        assert np.array_equal(from_dev(dq).view(np.uint32), q_ref.view(np.uint32))
    got_k, got_v = from_dev(dkp), from_dev(dvp)
    if kvt == 0:
        got_k, got_v, kp_ref, vp_ref = (a.view(np.uint32) for a in (got_k, got_v, kp_ref, vp_ref))
    bad_k = np.argwhere(got_k != kp_ref)
    assert bad_k.size == 0, f"K pages differ at {bad_k[:5].tolist()}"
    assert np.array_equal(got_v, vp_ref)


@pytest.mark.parametrize("kv", list(KVS))
def test_selftest_rows(ie, O, dev, kv):
    """Rows (0,20) (0,21) (1,3) (0,39) of sequences of length 40 and 20."""
    g = np.load(os.path.join(GOLDEN, "rope_cache.npz"))
    rng = np.random.default_rng(1)
    tables = g["tables"]
    run_case(ie, O, dev, KVS[kv], tables, tables.shape[1], int(g["num_pages"]) + 3, g["row_seq"],
             g["row_pos"], g["q"], g["k"], g["v"], rng)


@pytest.mark.parametrize("kv", list(KVS))
@pytest.mark.parametrize("with_q", [True, False])
def test_random_batch(ie, O, dev, kv, with_q):
    rng = np.random.default_rng(2 + KVS[kv])
    lens = [int(x) for x in rng.integers(1, 700, 37)]
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=9)
    row_seq = np.arange(len(lens), dtype=np.int32)
    row_pos = np.array([n - 1 for n in lens], np.int32)
    T = len(lens)
    run_case(ie, O, dev, KVS[kv], tables, max_pages, num_pages, row_seq, row_pos,
             normal(rng, (T, QD), 3.0), normal(rng, (T, KVD), 3.0), normal(rng, (T, KVD), 3.0), rng,
             with_q=with_q)


@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_edges_and_subnormals(ie, O, dev, kv):
    """Position 0 (identity), page edges 15/16, last slot of a page; tiny values that round
    to binary16 subnormals or to zero; large values (bf16 carry, f16 overflow to inf)."""
    rng = np.random.default_rng(4)
    lens = [17, 16, 33, 1, 32]
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=2)
    row_seq = np.array([0, 0, 1, 2, 3, 4], np.int32)
    row_pos = np.array([0, 16, 15, 32, 0, 31], np.int32)
    T = len(row_pos)
    scale = np.logspace(-9, 5, QD).astype(np.float32)
    q = normal(rng, (T, QD)) * scale
    k = normal(rng, (T, KVD)) * scale[:KVD][::-1]
    v = normal(rng, (T, KVD)) * scale[-KVD:]
    run_case(ie, O, dev, KVS[kv], tables, max_pages, num_pages, row_seq, row_pos,
             q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), rng)


def test_out_of_table_positions_are_skipped(ie, O, dev):
    """A row whose position lies beyond the RoPE table writes nothing (no fault)."""
    rng = np.random.default_rng(5)
    tables, max_pages, num_pages = make_tables([64], rng)
    kvt = 1
    kp = kv_pool(rng, num_pages, kvt, O)
    vp = kv_pool(rng, num_pages, kvt, O)
    dkp, dvp = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt)
    table = ie.rope_table(10, HD, THETA).to(dev)
    pos = np.array([40], np.int32)
    ie.rope_and_cache(None, to_dev(normal(rng, (1, KVD)), dev), to_dev(normal(rng, (1, KVD)), dev),
                      dkp, dvp, table, to_dev(pos, dev), to_dev(np.zeros(1, np.int32), dev),
                      to_dev(tables, dev), max_pages, NH, NKV, HD)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(dkp), kp) and np.array_equal(from_dev(dvp), vp)


def test_config2_full_size(ie, O, dev):
    """64 rows, pos ~ U[1, 4096), 65,536-page f16 pool, tables a seeded
    permutation of the free list; every byte of both pools checked."""
    rng = np.random.default_rng(20262)
    num_pages, kvt = 65536, 1
    max_pages = 4096 // 16
    perm = rng.permutation(num_pages).astype(np.int32)
    tables = perm[:64 * max_pages].reshape(64, max_pages)
    row_seq = np.arange(64, dtype=np.int32)
    row_pos = rng.integers(1, 4096, 64).astype(np.int32)
    run_case(ie, O, dev, kvt, tables, max_pages, num_pages, row_seq, row_pos,
             normal(rng, (64, QD)), normal(rng, (64, KVD)), normal(rng, (64, KVD)), rng,
             table_positions=4096)


@pytest.mark.parametrize("kv", list(KVS))
@pytest.mark.parametrize("with_q", [False, True])
def test_large_launch(ie, O, dev, kv, with_q):
    """A launch of over a million threads: 22,003 rows of 128 sequences, every slot
    distinct, rows in shuffled order (so neighbouring threads write scattered pages);
    every byte of both pools and q checked."""
    rng = np.random.default_rng(9 + KVS[kv] + 3 * with_q)
    n_seq, per_seq, T = 128, 172, 22003
    lens = [per_seq] * n_seq
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=5)
    slots = np.array([(s, p) for s in range(n_seq) for p in range(per_seq)], np.int32)
    slots = slots[rng.permutation(len(slots))[:T]]
    row_seq = np.ascontiguousarray(slots[:, 0])
    row_pos = np.ascontiguousarray(slots[:, 1])
    run_case(ie, O, dev, KVS[kv], tables, max_pages, num_pages, row_seq, row_pos,
             normal(rng, (T, QD)), normal(rng, (T, KVD)), normal(rng, (T, KVD)), rng,
             with_q=with_q)
