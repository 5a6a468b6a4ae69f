"""Row gather and block-table gather on the GPU vs the oracle: bit-exact."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import KVD, from_dev, kv_pool, make_tables, normal, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dim", [896, 151, 4])
def test_gather_rows(ie, O, dev, dim):
    """The reference self-test's case (9 x 896, rows {8, 0, 3}, src/cuda/cuda_runner.cu:1010-1018)
    plus an odd width and repeats."""
    rng = np.random.default_rng(dim)
    x = normal(rng, (9, dim))
    for rows in ([8, 0, 3], [5, 5, 1, 8, 0, 2, 7]):
        r = np.array(rows, np.int32)
        dst = torch.empty((len(rows), dim), dtype=torch.float32, device=dev)
        ie.gather_rows(dst, to_dev(x, dev), to_dev(r, dev))
        torch.cuda.synchronize()
        assert np.array_equal(from_dev(dst).view(np.uint32), O.gather_rows(x, r).view(np.uint32))


@pytest.mark.parametrize("kvt", [0, 1, 2])
def test_gather_kv(ie, O, dev, kvt):
    rng = np.random.default_rng(10 + kvt)
    lens = [1, 16, 17, 300, 1000]
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=5)
    pool = kv_pool(rng, num_pages, kvt, O)
    dpool, dtab = to_dev(pool, dev, kvt), to_dev(tables, dev)
    for s, n in enumerate(lens):
        dst = torch.full((n, KVD), float("nan"), dtype=torch.float32, device=dev)
        ie.gather_kv(dst, dpool, dtab, max_pages, s, n, KVD)
        torch.cuda.synchronize()
        want = O.gather_kv(pool, kvt, tables, max_pages, s, n, KVD)
        assert np.array_equal(from_dev(dst).view(np.uint32), want.view(np.uint32))
