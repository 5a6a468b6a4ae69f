"""The host-built decode work list (ie_hip_attention_plan), on the CPU.

The planner is host code in libie_hip.so: it runs without a GPU. Its output is
checked against a plain restatement of the layout include/ie_hip.h documents --
header [items, chunk_tokens, num_chunks, rows]; one item per (row, chunk),
min(p / chunk + 1, num_chunks) chunks per row, none for p < 0, longer chunks first
(row and chunk order among chunks of one length); an item is
[row, chunk, position, sequence, the chunk's page ids], ids -1 for pages past the
row's position or its table row, padded to a multiple of 4 ints -- and on its
errors. Whether the kernels read it right is tests/test_gpu_plan.py's part (bit
equality with the unplanned calls)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import PAGE


def restated_plan(row_pos, row_seq, tables, num_chunks, chunk_tokens):
    pages = chunk_tokens // PAGE
    stride = 4 + ((pages + 3) & ~3)
    max_pages = tables.shape[1]
    items = []
    for t, (p, s) in enumerate(zip(row_pos, row_seq)):
        if p < 0:
            continue
        for c in range(min(p // chunk_tokens + 1, num_chunks)):
            it = [t, c, p, s]
            for j in range(stride - 4):
                pi = c * pages + j
                ok = j < pages and pi * PAGE <= p and pi < max_pages
                it.append(int(tables[s, pi]) if ok else -1)
            items.append((min(chunk_tokens, p + 1 - c * chunk_tokens), it))
    # dispatch order: longer chunks first, row and chunk order within a length (stable)
    items = [it for _, it in sorted(items, key=lambda e: -e[0])]
    return [len(items), chunk_tokens, num_chunks, len(row_pos)], items, stride


@pytest.mark.parametrize("chunk_tokens", [64, 128, 256, 1024, 48])
def test_plan_matches_restatement(ie, chunk_tokens):
    rng = np.random.default_rng(40 + chunk_tokens)
    T, max_pages, seqs = 37, 300, 50
    tables = rng.integers(-2, 70000, (seqs, max_pages)).astype(np.int32)  # ids outside a pool too
    row_seq = rng.permutation(seqs)[:T].astype(np.int32)
    row_pos = rng.integers(-1, max_pages * PAGE + 100, T).astype(np.int32)  # -1 rows, past the table
    row_pos[:3] = [0, chunk_tokens - 1, chunk_tokens]                          # chunk edges
    num_chunks = ie.attention_chunks(int(row_pos.max()) + 1, chunk_tokens) - 1  # one row capped
    plan = ie.attention_plan(row_pos, row_seq, tables, num_chunks, chunk_tokens)
    head, items, stride = restated_plan(row_pos, row_seq, tables, num_chunks, chunk_tokens)
    assert plan.size == ie.attention_plan_ints(T, num_chunks, chunk_tokens)
    assert plan.size == 4 + T * num_chunks * stride
    assert list(plan[:4]) == head
    got = plan[4:4 + len(items) * stride].reshape(len(items), stride)
    assert np.array_equal(got, np.array(items, np.int32))


def test_plan_empty_batch_and_all_idle_rows(ie):
    tables = np.zeros((4, 8), np.int32)
    plan = ie.attention_plan(np.full(3, -1, np.int32), np.arange(3, dtype=np.int32), tables, 2, 64)
    assert list(plan[:4]) == [0, 64, 2, 3]


def test_plan_errors(ie):
    tables = np.zeros((4, 8), np.int32)
    with pytest.raises(ie.IeHipError, match="outside the table"):
        ie.attention_plan(np.array([5], np.int32), np.array([4], np.int32), tables, 2, 64)
    with pytest.raises(ie.IeHipError, match="chunk"):
        ie.attention_plan(np.array([5], np.int32), np.array([0], np.int32), tables, 2, 40)
    assert ie.attention_plan_ints(4, 2, 40) == 0 and ie.attention_plan_ints(0, 2, 64) == 0
    plan = np.zeros(8, np.int32)  # too small for 1 row x 2 chunks
    rc = ie.lib().ie_hip_attention_plan(plan.ctypes.data, plan.size, 1,
                                        np.array([5], np.int32).ctypes.data,
                                        np.array([0], np.int32).ctypes.data, tables.ctypes.data,
                                        4, 8, 2, 64)
    assert rc == ie.EINVAL and "ie_hip_attention_plan_ints" in ie.last_error()
