"""ie_hip_rope_cache_attention (RoPE + paged append + attention in one launch) on the GPU.

The contract: pages and `out` bit-identical to ie_hip_rope_and_cache followed by
ie_hip_attention on the same inputs (run here on copies), q left unmodified, and the
oracle's append + attention within the 16-bit tolerance (2e-3 absolute). Rows are
distinct sequences, as in a decode step. Cases: positions on page, pair and chunk
edges; a row whose position lies past the RoPE table (not appended, query unrotated,
as rope_and_cache skips it); a row whose target page lies outside the pool (not
written, masked); one long row (the small-grid layout: one wave per page pair).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import HD, KVD, NH, NKV, QD, THETA, from_dev, kv_pool, make_tables, normal, to_dev
from test_gpu_decode import check

pytestmark = pytest.mark.gpu
KVS = {"f16": 1, "bf16": 2}


def run_both(ie, dev, kvt, q, k, v, kp, vp, row_pos, row_seq, tables, max_pages, ct,
             table_positions):
    """(fused out, fused pools, q after), (two-call out, two-call pools)."""
    T = len(row_pos)
    nc = ie.attention_chunks(int(row_pos.max()) + 1, ct)
    table = ie.rope_table(table_positions, HD, THETA).to(dev)
    d_pos, d_seq, d_tab = to_dev(row_pos, dev), to_dev(row_seq, dev), to_dev(tables, dev)
    dk, dv = to_dev(k, dev), to_dev(v, dev)

    fq = to_dev(q, dev)
    fkp, fvp = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt)
    fout = torch.full((T, QD), float("nan"), dtype=torch.float32, device=dev)
    ws = ie.attention_workspace(T, NH, HD, nc)
    ie.rope_cache_attention(fout, fq, dk, dv, fkp, fvp, table, d_pos, d_seq, d_tab, max_pages, nc,
                            ct, ws, NH, NKV, HD)

    tq = to_dev(q, dev)
    tkp, tvp = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt)
    tout = torch.full((T, QD), float("nan"), dtype=torch.float32, device=dev)
    ws2 = ie.attention_workspace(T, NH, HD, nc)
    ie.rope_and_cache(tq, dk, dv, tkp, tvp, table, d_pos, d_seq, d_tab, max_pages, NH, NKV, HD)
    ie.attention(tout, tq, tkp, tvp, d_pos, d_seq, d_tab, max_pages, nc, ct, ws2, NH, NKV, HD)
    torch.cuda.synchronize()
    return ((from_dev(fout), from_dev(fkp), from_dev(fvp), from_dev(fq)),
            (from_dev(tout), from_dev(tkp), from_dev(tvp)))


@pytest.mark.parametrize("ct", [64, 128, 256])
@pytest.mark.parametrize("kv", list(KVS))
def test_matches_two_calls_and_oracle(ie, O, dev, kv, ct):
    kvt = KVS[kv]
    rng = np.random.default_rng(700 + ct + kvt)
    pos = [0, 1, 15, 16, 31, 32, 63, 64, 127, 128, 500, 2047, 2100, 700]
    lens = [p + 1 for p in pos]
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=3)
    # row 12: position past the RoPE table (2048 positions); row 13: its target page
    # lies outside the pool.
    table_positions = 2048
    tables[13, 700 // 16] = num_pages + 3
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_pos = np.array(pos, np.int32)
    row_seq = np.arange(len(pos), dtype=np.int32)
    q = normal(rng, (len(pos), QD))
    k = normal(rng, (len(pos), KVD))
    v = normal(rng, (len(pos), KVD))
    (fout, fkp, fvp, fq), (tout, tkp, tvp) = run_both(ie, dev, kvt, q, k, v, kp, vp, row_pos,
                                                      row_seq, tables, max_pages, ct,
                                                      table_positions)
    assert np.array_equal(fq.view(np.uint32), q.view(np.uint32)), "q was modified"
    assert np.array_equal(fkp, tkp) and np.array_equal(fvp, tvp), "pages differ from two calls"
    assert np.array_equal(fout.view(np.uint32), tout.view(np.uint32)), "out differs from two calls"
    # The oracle (like the reference, it has no pool bounds check, so row 13 -- covered
    # bit for bit by the two-call comparison above -- stays out): append the rows inside
    # the table, then attention with their rotated queries.
    keep = np.arange(len(pos)) != 13
    inside = keep & (row_pos < table_positions)
    q_ref, kp_ref, vp_ref = O.rope_append_paged(q[inside], k[inside], v[inside], kp, vp, kvt,
                                                row_pos[inside], row_seq[inside], tables,
                                                max_pages, NH, NKV, HD, THETA)
    q_all = q.copy()
    q_all[inside] = q_ref
    assert np.array_equal(fkp, kp_ref) and np.array_equal(fvp, vp_ref), "pages differ from oracle"
    want = O.paged_attention(q_all[keep], kp_ref, vp_ref, kvt, row_pos[keep], row_seq[keep],
                             tables, max_pages, NH, NKV, HD, threads=8)
    check(O, fout[keep], want, kvt, f"fused, chunk {ct}")


@pytest.mark.parametrize("kv", list(KVS))
def test_long_single_row(ie, O, dev, kv):
    """One row at position 8,191 in 512-token chunks: four waves per workgroup (128
    positions each), and the appended position sits in the last wave's last pair."""
    kvt = KVS[kv]
    rng = np.random.default_rng(800 + kvt)
    L = 8192
    tables, max_pages, num_pages = make_tables([L], rng)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_pos, row_seq = np.array([L - 1], np.int32), np.zeros(1, np.int32)
    q, k, v = normal(rng, (1, QD)), normal(rng, (1, KVD)), normal(rng, (1, KVD))
    (fout, fkp, fvp, fq), (tout, tkp, tvp) = run_both(ie, dev, kvt, q, k, v, kp, vp, row_pos,
                                                      row_seq, tables, max_pages, 512, L)
    assert np.array_equal(fq.view(np.uint32), q.view(np.uint32))
    assert np.array_equal(fkp, tkp) and np.array_equal(fvp, tvp)
    assert np.array_equal(fout.view(np.uint32), tout.view(np.uint32))


def test_unsupported_shapes_fail_loudly(ie, dev):
    """f32 caches (and other shapes) are refused with EINVAL: the caller uses the two calls."""
    assert not ie.rope_cache_attention_supported(ie.KV_F32, NH, NKV, HD, 128)
    assert ie.rope_cache_attention_supported(ie.KV_F16, NH, NKV, HD, 128)
    assert not ie.rope_cache_attention_supported(ie.KV_F16, NH, NKV, HD, 48)
    rng = np.random.default_rng(5)
    tables, max_pages, num_pages = make_tables([40], rng)
    kp = torch.zeros((num_pages * 16, KVD), dtype=torch.float32, device=dev)
    out = torch.zeros((1, QD), device=dev)
    q = torch.zeros((1, QD), device=dev)
    kv_rows = torch.zeros((1, KVD), device=dev)
    table = ie.rope_table(64, HD, THETA).to(dev)
    ws = ie.attention_workspace(1, NH, HD, 1)
    with pytest.raises(ie.IeHipError):
        ie.rope_cache_attention(out, q, kv_rows, kv_rows, kp, kp, table,
                                torch.tensor([39], dtype=torch.int32, device=dev),
                                torch.zeros(1, dtype=torch.int32, device=dev),
                                to_dev(tables, dev), max_pages, 1, 64, ws, NH, NKV, HD)
