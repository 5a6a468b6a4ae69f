"""ie_hip_attention_noalloc (the entry point that allocates nothing: its split-K partials
live in the library's fixed device scratch) against ie_hip_attention with a workspace of
its own, through the C ABI: bit for bit, on two calls in a row, the second with a smaller
input (fewer rows, shorter contexts, fewer chunks) so that it runs over what the first
left in the scratch; and the size limit refused with a clear error."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import HD, NH, NKV, QD, kv_pool, make_tables, normal, to_dev

pytestmark = pytest.mark.gpu


def _case(ie, dev, rng, lens, kvt, ct):
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=2)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    T = len(lens)
    pos = to_dev(np.array([n - 1 for n in lens], np.int32), dev)
    seq = to_dev(np.arange(T, dtype=np.int32), dev)
    q = to_dev(normal(rng, (T, QD)), dev)
    nc = ie.attention_chunks(max(lens), ct)
    args = (to_dev(kp, dev, kvt), to_dev(vp, dev, kvt), pos, seq, to_dev(tables, dev), max_pages,
            nc)
    want = torch.full((T, QD), float("nan"), device=dev)
    ie.attention(want, q, *args, ct, ie.attention_workspace(T, NH, HD, nc), NH, NKV, HD)
    got = torch.full((T, QD), float("nan"), device=dev)
    ie.attention_noalloc(got, q, *args, ct, NH, NKV, HD)
    torch.cuda.synchronize()
    return got, want


@pytest.mark.parametrize("kv", [0, 1, 2])
def test_noalloc_matches_workspace_entry_point(ie, dev, kv):
    print(f"attention_noalloc kv={kv}", flush=True)
    rng = np.random.default_rng(900 + kv)
    ct = 128 if kv else 64
    big = [int(x) for x in rng.integers(128, 4097, 64)]     # config 3's shape
    small = [int(x) for x in rng.integers(1, 700, 5)]
    for lens in (big, small):
        got, want = _case(ie, dev, rng, lens, kv, ct)
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), f"{len(lens)} rows"


def test_noalloc_refuses_more_than_its_scratch(ie, dev):
    T, nc = 64, 72  # 64 x 14 x 72 slots of 264 bytes > 16 MiB
    need = int(ie.lib().ie_hip_attention_workspace_bytes(T, NH, HD, nc))
    assert need > ie.NOALLOC_SCRATCH_BYTES
    rng = np.random.default_rng(1)
    tables, max_pages, num_pages = make_tables([16] * T, rng)
    pool = torch.zeros((num_pages * 16, NKV * HD), dtype=torch.float16, device=dev)
    z = torch.zeros((T, QD), device=dev)
    pos = torch.full((T,), 15, dtype=torch.int32, device=dev)
    seq = torch.arange(T, dtype=torch.int32, device=dev)
    with pytest.raises(ie.IeHipError, match="fixed scratch"):
        ie.attention_noalloc(z, z, pool, pool, pos, seq, to_dev(tables, dev), max_pages, nc, 64,
                             NH, NKV, HD)
