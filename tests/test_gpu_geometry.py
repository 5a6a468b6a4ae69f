"""Head geometries other than Qwen2.5's 14/2 on the GPU vs the CPU oracle.

The kernels are written for the reference's limits (head_dim 64 for attention,
at most 8 query heads per KV head; head_dim 64 or 128 for RoPE + append), with
the matrix-core decode kernel taking rows of 128 KV elements and up to 16 query
heads, and the matrix-core prefill kernel instantiated per group size and with
one or two teams of waves. These cases run every such variant against the
oracle at the same tolerances as the Qwen tests (f32: the reference's compare()
<= 1e-5; f16/bf16: 2e-3 absolute), through both implementations.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import PAGE, THETA, from_dev, make_tables, normal, to_dev
from test_gpu_decode import check

pytestmark = pytest.mark.gpu
KVS = {"f32": 0, "f16": 1, "bf16": 2}
HD = 64

# (query heads, KV heads): group sizes 8, 4, 3, 1 on 128-element KV rows (the
# matrix-core decode kernel's shape), then KV rows of 64, 256 and 512 elements.
GEOMETRIES = [(16, 2), (8, 2), (6, 2), (2, 2), (7, 1), (4, 4), (16, 8)]


@pytest.fixture(params=["auto", "valu"])
def impl(request, ie):
    prev = ie.set_attention_impl({"auto": ie.IMPL_AUTO, "valu": ie.IMPL_VALU}[request.param])
    yield request.param
    ie.set_attention_impl(prev)


def pools(rng, O, num_pages, kvd, kvt):
    k = O.round_to_kv(normal(rng, (num_pages * PAGE, kvd)), kvt)
    v = O.round_to_kv(normal(rng, (num_pages * PAGE, kvd)), kvt)
    return k, v


@pytest.mark.parametrize("geom", GEOMETRIES, ids=[f"{h}q{k}kv" for h, k in GEOMETRIES])
@pytest.mark.parametrize("kv", list(KVS))
def test_decode(ie, O, dev, geom, kv, impl):
    nh, nkv = geom
    kvt = KVS[kv]
    rng = np.random.default_rng(1000 + 10 * nh + nkv)
    lens = [700, 1, 64, 65, 333]
    tables, max_pages, num_pages = make_tables(lens, rng)
    kp, vp = pools(rng, O, num_pages, nkv * HD, kvt)
    row_pos = np.array([n - 1 for n in lens], np.int32)
    row_seq = np.arange(len(lens), dtype=np.int32)
    q = normal(rng, (len(lens), nh * HD))
    want = O.paged_attention(q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, nh, nkv, HD,
                             threads=8)
    for ct in (64, 128):
        nc = ie.attention_chunks(int(row_pos.max()) + 1, ct)
        ws = ie.attention_workspace(len(lens), nh, HD, nc)
        out = torch.full((len(lens), nh * HD), float("nan"), dtype=torch.float32, device=dev)
        ie.attention(out, to_dev(q, dev), to_dev(kp, dev, kvt), to_dev(vp, dev, kvt),
                     to_dev(row_pos, dev), to_dev(row_seq, dev), to_dev(tables, dev), max_pages,
                     nc, ct, ws, nh, nkv, HD)
        torch.cuda.synchronize()
        check(O, from_dev(out), want, kvt, f"{nh}/{nkv} chunk {ct}")


@pytest.mark.parametrize("geom", GEOMETRIES, ids=[f"{h}q{k}kv" for h, k in GEOMETRIES])
@pytest.mark.parametrize("kv", list(KVS))
def test_prefill(ie, O, dev, geom, kv, impl):
    """A 300-token prompt continuing a 40-token context, and (with 8 KV heads) a
    1,100-token prompt whose grid exceeds the compute units: the one-team kernel."""
    nh, nkv = geom
    kvt = KVS[kv]
    rng = np.random.default_rng(2000 + 10 * nh + nkv)
    start, T = (0, 1100) if nkv == 8 else (40, 300)
    L = start + T
    tables, max_pages, num_pages = make_tables([L], rng)
    kp, vp = pools(rng, O, num_pages, nkv * HD, kvt)
    row_pos = np.arange(start, L, dtype=np.int32)
    row_seq = np.zeros(T, np.int32)
    q = normal(rng, (T, nh * HD))
    want = O.paged_attention(q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, nh, nkv, HD,
                             threads=8)
    out = torch.full((T, nh * HD), float("nan"), dtype=torch.float32, device=dev)
    ie.attention_prefill(out, to_dev(q, dev), to_dev(kp, dev, kvt), to_dev(vp, dev, kvt),
                         to_dev(row_pos, dev), to_dev(row_seq, dev), to_dev(tables, dev),
                         max_pages, nh, nkv, HD)
    torch.cuda.synchronize()
    check(O, from_dev(out), want, kvt, f"{nh}/{nkv} prefill T={T}")


@pytest.mark.parametrize("geom", [(16, 2, 64), (7, 1, 64), (8, 2, 128), (4, 4, 128)],
                         ids=["16q2kv_hd64", "7q1kv_hd64", "8q2kv_hd128", "4q4kv_hd128"])
@pytest.mark.parametrize("kv", list(KVS))
def test_append(ie, O, dev, geom, kv):
    """RoPE + paged append, bit-exact: rotated q, and every byte of both pools."""
    nh, nkv, hd = geom
    kvt = KVS[kv]
    rng = np.random.default_rng(3000 + 10 * nh + nkv + hd)
    lens = [90, 17, 300]
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=5)
    kvd = nkv * hd
    kp = O.round_to_kv(normal(rng, (num_pages * PAGE, kvd)), kvt)
    vp = O.round_to_kv(normal(rng, (num_pages * PAGE, kvd)), kvt)
    row_seq = np.array([0, 1, 2, 2, 0], np.int32)
    row_pos = np.array([89, 0, 299, 150, 16], np.int32)
    q = normal(rng, (len(row_pos), nh * hd))
    k = normal(rng, (len(row_pos), kvd))
    v = normal(rng, (len(row_pos), kvd))
    q_ref, kp_ref, vp_ref = O.rope_append_paged(q, k, v, kp, vp, kvt, row_pos, row_seq, tables,
                                                max_pages, nh, nkv, hd, THETA)
    table = ie.rope_table(int(row_pos.max()) + 1, hd, THETA).to(dev)
    dq = to_dev(q, dev)
    dkp, dvp = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt)
    ie.rope_and_cache(dq, to_dev(k, dev), to_dev(v, dev), dkp, dvp, table, to_dev(row_pos, dev),
                      to_dev(row_seq, dev), to_dev(tables, dev), max_pages, nh, nkv, hd)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(dq).view(np.uint32), q_ref.view(np.uint32))
    got_k, got_v = from_dev(dkp), from_dev(dvp)
    if kvt == 0:
        got_k, got_v, kp_ref, vp_ref = (a.view(np.uint32) for a in (got_k, got_v, kp_ref, vp_ref))
    assert np.array_equal(got_k, kp_ref)
    assert np.array_equal(got_v, vp_ref)
