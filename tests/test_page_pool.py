"""The page allocator behind BatchRunner (host only, no GPU).

Compared step by step with the reference's allocation order restated in
oracle/allocator.py (src/cuda/cuda_runner.cu:191-313): page ids handed out,
page tables, free counts and every error path (pool exhaustion, over-length
sequences, closed ids, double close) under seeded churn.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle.allocator import AllocError, RefAllocator, pages_for


def snapshot(pool, ref):
    assert pool.free_pages == ref.free_pages
    assert pool.host_tables() == ref.tables
    for s in range(ref.max_batch):
        if ref.open[s]:
            assert pool.pages(s) == ref.pages[s]


def test_first_pages_in_order(ie):
    pool = ie.PagePool(10, 2, 64)
    s = pool.open_sequence()
    pool.ensure(s, 33)
    assert pool.pages(s) == [0, 1, 2]
    assert pool.free_pages == 7 and pool.max_pages_per_seq == 4


def test_close_returns_pages_lifo(ie):
    pool, ref = ie.PagePool(8, 3, 128), RefAllocator(8, 3, 128)
    for p in (pool, ref):
        a, b = p.open_sequence(), p.open_sequence()
        p.ensure(a, 40)
        p.ensure(b, 20)
        p.close_sequence(a)
        c = p.open_sequence()
        p.ensure(c, 48)
    snapshot(pool, ref)
    # the closed sequence's last page is reused first
    assert pool.pages(0)[:3] == [2, 1, 0]


def test_errors(ie):
    pool = ie.PagePool(3, 2, 40)
    with pytest.raises(ie.IeHipError) as e:
        pool.ensure(0, 1)  # not open
    assert e.value.code == ie.ESEQ and "invalid or closed sequence id 0" in str(e.value)
    s = pool.open_sequence()
    with pytest.raises(ie.IeHipError) as e:
        pool.ensure(s, 41)
    assert e.value.code == ie.ERANGE and "longer than the maximum (40 tokens)" in str(e.value)
    pool.ensure(s, 40)  # 3 pages, all of the pool
    t = pool.open_sequence()
    with pytest.raises(ie.IeHipError) as e:
        pool.ensure(t, 1)
    assert e.value.code == ie.EFULL and "KV cache full" in str(e.value)
    assert pool.open_sequence() == -1  # both slots busy
    pool.close_sequence(s)
    with pytest.raises(ie.IeHipError) as e:
        pool.close_sequence(s)  # double close
    assert e.value.code == ie.ESEQ
    with pytest.raises(ie.IeHipError):
        pool.close_sequence(7)  # out of range
    assert pool.free_pages == 3


def test_bad_construction(ie):
    with pytest.raises(ie.IeHipError):
        ie.PagePool(0, 1, 16)
    with pytest.raises(ie.IeHipError):
        ie.PagePool(4, 0, 16)


def test_pages_for(ie):
    for n in (0, 1, 15, 16, 17, 4000, 32768):
        assert ie.pages_for(n) == pages_for(n)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_seeded_churn_matches_reference_order(ie, seed):
    """Random open / grow / close traffic, with a 25% free-and-reallocate phase."""
    rng = np.random.default_rng(seed)
    num_pages, max_batch, max_seq = 300, 24, 400
    pool, ref = ie.PagePool(num_pages, max_batch, max_seq), RefAllocator(num_pages, max_batch, max_seq)
    live = []
    for step in range(600):
        op = rng.random()
        if op < 0.25 or not live:
            a, b = pool.open_sequence(), ref.open_sequence()
            assert a == b
            if a >= 0:
                live.append(a)
        elif op < 0.8:
            s = live[rng.integers(len(live))]
            n = int(rng.integers(0, max_seq + 40))
            try:
                ref.ensure(s, n)
                kind = None
            except AllocError as e:
                kind = e.kind
            if kind is None:
                pool.ensure(s, n)
            else:
                with pytest.raises(ie.IeHipError) as e:
                    pool.ensure(s, n)
                assert e.value.code == {"full": ie.EFULL, "range": ie.ERANGE, "seq": ie.ESEQ}[kind]
        else:
            s = live.pop(rng.integers(len(live)))
            pool.close_sequence(s)
            ref.close_sequence(s)
        if step % 50 == 0:
            snapshot(pool, ref)
        # conservation: every page is free or owned by exactly one open sequence
        owned = [p for s in live for p in pool.pages(s)]
        assert len(owned) == len(set(owned))
        assert len(owned) + pool.free_pages == num_pages
    snapshot(pool, ref)
