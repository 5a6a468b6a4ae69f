"""ie_hip_rope_cache_attention_prefill (RoPE + paged append of a prompt chunk, then
prefill attention with q rotated inside the prefill kernel) on the GPU.

The contract: pages and `out` bit-identical to ie_hip_rope_and_cache (q rotated in
place) followed by ie_hip_attention_prefill on the same inputs (run here on copies), q
left unmodified, and the oracle's append + attention within the 16-bit caches'
tolerance (2e-3 absolute); f32 caches are refused (the caller uses the two calls).
Cases: the reference self-test's prompt lengths (src/cuda/cuda_runner.cu:920-934), a
continuation, a prompt starting mid-tile, a prompt whose keys run past 32,768 (page ids
staged in two segments), rows whose positions lie past the RoPE table (not appended,
queries unrotated, as rope_and_cache skips them), a page outside the pool (not written,
its keys masked), and BASELINE config 5's 4,000-token prompt into a churned pool.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import HD, KVD, NH, NKV, QD, THETA, from_dev, kv_pool, make_tables, normal, to_dev
from test_gpu_decode import check

pytestmark = pytest.mark.gpu
KVS = {"f16": 1, "bf16": 2}


def run_both(ie, dev, kvt, q, k, v, kp, vp, row_pos, row_seq, tables, max_pages,
             table_positions):
    """(fused out, fused pools, q after), (two-call out, two-call pools, rotated q)."""
    T = len(row_pos)
    table = ie.rope_table(table_positions, HD, THETA).to(dev)
    d_pos, d_seq, d_tab = to_dev(row_pos, dev), to_dev(row_seq, dev), to_dev(tables, dev)
    dk, dv = to_dev(k, dev), to_dev(v, dev)

    fq = to_dev(q, dev)
    fkp, fvp = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt)
    fout = torch.full((T, QD), float("nan"), dtype=torch.float32, device=dev)
    ie.rope_cache_attention_prefill(fout, fq, dk, dv, fkp, fvp, table, d_pos, d_seq, d_tab,
                                    max_pages, NH, NKV, HD)

    tq = to_dev(q, dev)
    tkp, tvp = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt)
    tout = torch.full((T, QD), float("nan"), dtype=torch.float32, device=dev)
    ie.rope_and_cache(tq, dk, dv, tkp, tvp, table, d_pos, d_seq, d_tab, max_pages, NH, NKV, HD)
    ie.attention_prefill(tout, tq, tkp, tvp, d_pos, d_seq, d_tab, max_pages, NH, NKV, HD)
    torch.cuda.synchronize()
    return ((from_dev(fout), from_dev(fkp), from_dev(fvp), from_dev(fq)),
            (from_dev(tout), from_dev(tkp), from_dev(tvp), from_dev(tq)))


def same_bits(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


# (sequence lengths, the prompt's sequence, its first position, rows)
PROMPTS = [
    ([1], 0, 0, 1),
    ([17], 0, 0, 17),
    ([300], 0, 0, 300),
    ([1000], 0, 0, 1000),
    ([540], 0, 500, 40),          # a prompt continuing at 500
    ([100, 300], 1, 0, 300),     # the 2nd of 2 sequences
    ([129], 0, 63, 66),          # starts mid-tile, crosses tile edges
    ([32830], 0, 32750, 80),     # keys past 32,768: the page ids are staged in two segments
]


@pytest.mark.parametrize("case", range(len(PROMPTS)))
@pytest.mark.parametrize("kv", list(KVS))
def test_matches_two_calls_and_oracle(ie, O, dev, kv, case):
    lens, seq, start, T = PROMPTS[case]
    kvt = KVS[kv]
    rng = np.random.default_rng(1300 + 10 * case + kvt)
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=2)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_pos = np.arange(start, start + T, dtype=np.int32)
    row_seq = np.full(T, seq, np.int32)
    q, k, v = normal(rng, (T, QD)), normal(rng, (T, KVD)), normal(rng, (T, KVD))
    (fout, fkp, fvp, fq), (tout, tkp, tvp, tq) = run_both(ie, dev, kvt, q, k, v, kp, vp, row_pos,
                                                          row_seq, tables, max_pages,
                                                          max(2048, start + T))
    assert same_bits(fq, q), "q was modified"
    assert same_bits(fkp, tkp) and same_bits(fvp, tvp), "pages differ from the two calls"
    assert same_bits(fout, tout), "out differs from the two calls"
    q_ref, kp_ref, vp_ref = O.rope_append_paged(q, k, v, kp, vp, kvt, row_pos, row_seq, tables,
                                                max_pages, NH, NKV, HD, THETA)
    assert same_bits(tq, q_ref), "the two calls' rotated q differs from the oracle"
    assert same_bits(fkp, kp_ref) and same_bits(fvp, vp_ref), "pages differ from the oracle"
    want = O.paged_attention(q_ref, kp_ref, vp_ref, kvt, row_pos, row_seq, tables, max_pages, NH,
                             NKV, HD, threads=8)
    check(O, fout, want, kvt, f"fused prefill, case {case}")


@pytest.mark.parametrize("kv", list(KVS))
def test_rows_past_the_table_and_a_page_outside_the_pool(ie, O, dev, kv):
    """A prompt at positions 1,990 .. 2,059 with a 2,048-position RoPE table: its last 12
    rows are neither appended nor rotated (both paths); one page of the sequence lies
    outside the pool (its rows are not written and its keys are not attended)."""
    kvt = KVS[kv]
    rng = np.random.default_rng(1400 + kvt)
    start, T = 1990, 70
    tables, max_pages, num_pages = make_tables([start + T], rng, extra_pages=2)
    tables[0, 2000 // 16] = num_pages + 5
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_pos = np.arange(start, start + T, dtype=np.int32)
    row_seq = np.zeros(T, np.int32)
    q, k, v = normal(rng, (T, QD)), normal(rng, (T, KVD)), normal(rng, (T, KVD))
    (fout, fkp, fvp, fq), (tout, tkp, tvp, tq) = run_both(ie, dev, kvt, q, k, v, kp, vp, row_pos,
                                                          row_seq, tables, max_pages, 2048)
    assert same_bits(fq, q)
    assert same_bits(fkp, tkp) and same_bits(fvp, tvp)
    assert same_bits(fout, tout)
    past = row_pos >= 2048
    assert same_bits(tq[past], q[past]), "rows past the table must keep their query"
    assert np.isfinite(fout).all()


@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_config5_prompt_into_churned_pool(ie, O, dev, kv):
    """BASELINE config 5's prompt: 4,000 rows appended into pages scattered over a pool
    (a seeded permutation of 8,192 pages), both paths bit for bit, every row against the
    oracle."""
    kvt = KVS[kv]
    rng = np.random.default_rng(1500 + kvt)
    T, num_pages = 4000, 8192
    pages = (T + 15) // 16
    max_pages = pages
    tables = rng.permutation(num_pages)[:pages].astype(np.int32)[None, :]
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_pos = np.arange(T, dtype=np.int32)
    row_seq = np.zeros(T, np.int32)
    q, k, v = normal(rng, (T, QD)), normal(rng, (T, KVD)), normal(rng, (T, KVD))
    (fout, fkp, fvp, fq), (tout, tkp, tvp, tq) = run_both(ie, dev, kvt, q, k, v, kp, vp, row_pos,
                                                          row_seq, tables, max_pages, T)
    assert same_bits(fq, q)
    assert same_bits(fkp, tkp) and same_bits(fvp, tvp)
    assert same_bits(fout, tout)
    # The oracle over the prompt's own pages (gathered; the pool's other pages are not read).
    ids = tables[0]
    rows = (ids[:, None].astype(np.int64) * 16 + np.arange(16)).reshape(-1)
    small_k = fkp.reshape(num_pages * 16, KVD)[rows]
    small_v = fvp.reshape(num_pages * 16, KVD)[rows]
    small_tab = np.arange(pages, dtype=np.int32)[None, :]
    want = O.paged_attention(tq, small_k, small_v, kvt, row_pos, row_seq, small_tab, pages, NH,
                             NKV, HD, threads=8)
    check(O, fout, want, kvt, "fused prefill, config 5")


def test_unsupported_fails_loudly(ie, dev):
    """f32 caches, the VALU kernels and shapes the matrix-core prefill does not take are
    refused with EINVAL: the caller uses the two calls."""
    assert ie.rope_cache_attention_prefill_supported(ie.KV_F16, NH, NKV, HD)
    assert ie.rope_cache_attention_prefill_supported(ie.KV_BF16, NH, NKV, HD)
    assert not ie.rope_cache_attention_prefill_supported(ie.KV_F32, NH, NKV, HD)
    assert not ie.rope_cache_attention_prefill_supported(ie.KV_F16, NH, NKV, 128)
    prev = ie.set_attention_impl(ie.IMPL_VALU)
    try:
        assert not ie.rope_cache_attention_prefill_supported(ie.KV_F16, NH, NKV, HD)
        rng = np.random.default_rng(6)
        tables, max_pages, num_pages = make_tables([40], rng)
        kp = torch.zeros((num_pages * 16, KVD), dtype=torch.float16, device=dev)
        vp = torch.zeros_like(kp)
        out = torch.zeros((20, QD), device=dev)
        q = torch.zeros((20, QD), device=dev)
        kv_rows = torch.zeros((20, KVD), device=dev)
        table = ie.rope_table(64, HD, THETA).to(dev)
        pos = torch.arange(20, dtype=torch.int32, device=dev)
        seq = torch.zeros(20, dtype=torch.int32, device=dev)
        with pytest.raises(ie.IeHipError, match="rope_cache_attention_prefill"):
            ie.rope_cache_attention_prefill(out, q, kv_rows, kv_rows, kp, vp, table, pos, seq,
                                            to_dev(tables, dev), max_pages, NH, NKV, HD)
    finally:
        ie.set_attention_impl(prev)
    kp32 = torch.zeros((num_pages * 16, KVD), device=dev)
    vp32 = torch.zeros_like(kp32)
    with pytest.raises(ie.IeHipError, match="rope_cache_attention_prefill"):
        ie.rope_cache_attention_prefill(out, q, kv_rows, kv_rows, kp32, vp32, table, pos, seq,
                                        to_dev(tables, dev), max_pages, NH, NKV, HD)
    assert int(kp32.count_nonzero()) == 0
