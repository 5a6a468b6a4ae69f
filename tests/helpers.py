"""Shared test utilities: seeded paged-cache fixtures and host/device copies."""
from __future__ import annotations

import numpy as np

NH, NKV, HD, THETA = 14, 2, 64, 1e6
QD, KVD = NH * HD, NKV * HD
PAGE = 16
DTYPES = {"f32": 0, "f16": 1, "bf16": 2}


def make_tables(lens, rng, extra_pages: int = 0):
    """Pages handed out as a shuffled permutation, so no sequence is contiguous.

    Restates the reference self-test's TestPages (src/cuda/cuda_runner.cu:691-711);
    `extra_pages` adds unused pages to the pool (they must stay untouched).
    Returns (tables [n_seq, max_pages] int32, max_pages, num_pages).
    """
    max_pages = max(1, max((n + PAGE - 1) // PAGE for n in lens))
    need = sum((n + PAGE - 1) // PAGE for n in lens)
    num_pages = need + extra_pages
    order = rng.permutation(num_pages).astype(np.int32)
    tables = np.zeros((len(lens), max_pages), np.int32)
    nxt = 0
    for s, n in enumerate(lens):
        for i in range((n + PAGE - 1) // PAGE):
            tables[s, i] = order[nxt]
            nxt += 1
    return tables, max_pages, num_pages


def normal(rng, shape, scale: float = 1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32)


def kv_pool(rng, num_pages, kv_dtype, O, scale: float = 1.0):
    """Pool [num_pages*16, KVD] of N(0,1)*scale values in kv_dtype (uint16 bits for 16-bit)."""
    x = normal(rng, (num_pages * PAGE, KVD), scale)
    return O.round_to_kv(x, kv_dtype)


def to_dev(a, dev, kv_dtype=None):
    """numpy -> torch on dev; uint16 pools become float16/bfloat16 tensors (same bits)."""
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16)).to(dev)
        return t.view(torch.bfloat16 if kv_dtype == 2 else torch.float16)
    return torch.from_numpy(a).to(dev)


def from_dev(t):
    """torch -> numpy; 16-bit float tensors come back as uint16 bit patterns."""
    import torch
    t = t.detach().cpu()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a
