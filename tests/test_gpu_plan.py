"""The host-planned decode path on the GPU: ie_hip_attention_planned and
ie_hip_rope_cache_attention_planned give the same bits as ie_hip_attention and
ie_hip_rope_cache_attention (outputs, and pages for the fused call), for every KV
type, one-wave and one-pair-per-wave workgroups, rows at position -1, a row past
the chunks' capacity, and BASELINE config 3 at full size. The unplanned calls are
checked against the oracle elsewhere (test_gpu_decode.py, test_gpu_fused.py), so
equality carries that parity over. Item slots past the plan's item count hold
in-bounds but wrong items (another row's valid pages), which the kernel must
never read."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import HD, KVD, NH, NKV, PAGE, QD, from_dev, kv_pool, make_tables, normal, to_dev

pytestmark = pytest.mark.gpu
KVS = {"f32": 0, "f16": 1, "bf16": 2}


def planted_plan(ie, row_pos, row_seq, tables, nc, ct):
    """attention_plan()'s list with every unused item slot holding a copy of item 0 whose
    page ids are another row's (valid pages): wrong if read, never out of bounds."""
    plan = ie.attention_plan(row_pos, row_seq, tables, nc, ct)
    items, stride = int(plan[0]), 4 + ((ct // PAGE + 3) & ~3)
    if items > 0:
        decoy = plan[4:4 + stride].copy()
        other = int(row_seq[-1])
        decoy[4:4 + ct // PAGE] = tables[other, :ct // PAGE]
        slots = (plan.size - 4) // stride
        for i in range(items, slots):
            plan[4 + i * stride:4 + (i + 1) * stride] = decoy
    return plan


def run_pair(ie, dev, kvt, q, kp, vp, row_pos, row_seq, tables, max_pages, nc, ct):
    T = len(row_pos)
    ws = ie.attention_workspace(T, NH, HD, nc)
    d = dict(q=to_dev(q, dev), kp=to_dev(kp, dev, kvt), vp=to_dev(vp, dev, kvt),
             pos=to_dev(row_pos, dev), seq=to_dev(row_seq, dev), tab=to_dev(tables, dev))
    plan = torch.from_numpy(planted_plan(ie, row_pos, row_seq, tables, nc, ct)).to(dev)
    a = torch.full((T, QD), 7.0, device=dev)
    b = torch.full((T, QD), 7.0, device=dev)
    ie.attention(a, d["q"], d["kp"], d["vp"], d["pos"], d["seq"], d["tab"], max_pages, nc, ct, ws,
                 NH, NKV, HD)
    ie.attention_planned(b, d["q"], d["kp"], d["vp"], d["pos"], d["seq"], d["tab"], max_pages, nc,
                         ct, ws, plan, NH, NKV, HD)
    torch.cuda.synchronize()
    return from_dev(a), from_dev(b)


# (rows, context range, chunk tokens): small grids split chunks one pair per wave
CASES = [(1, (3000, 3001), 128), (3, (100, 2100), 256), (64, (128, 4097), 128),
         (200, (1, 900), 64), (5, (500, 5000), 512)]


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("kv", list(KVS))
def test_planned_equals_unplanned(ie, O, dev, kv, case):
    T, (lo, hi), ct = CASES[case]
    kvt = KVS[kv]
    rng = np.random.default_rng(1300 + case)
    lens = rng.integers(lo, hi, T)
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=3)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_seq = np.arange(T, dtype=np.int32)
    pos = (lens - 1).astype(np.int32)
    if T > 4:
        pos[rng.random(T) < 0.1] = -1
    nc = ie.attention_chunks(int(lens.max()), ct)
    if T >= 64:  # one row past the capacity of nc - 1 chunks
        nc = max(1, nc - 1)
    q = normal(rng, (T, QD))
    a, b = run_pair(ie, dev, kvt, q, kp, vp, pos, row_seq, tables, int(max_pages), nc, ct)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), \
        f"planned differs ({T} rows, chunk {ct}, {nc} chunks)"


@pytest.mark.parametrize("ct", [128, 192, 256])
def test_config3_planned_full_size(ie, O, dev, ct):
    """64 rows, L ~ U[128, 4096], 65,536-page f16 pools, shuffled
    tables; 192-token chunks (the library's choice for this grid), 128 and 256."""
    rng = np.random.default_rng(20263)
    T, num_pages = 64, 65536
    lens = rng.integers(128, 4097, T)
    max_pages = 4096 // PAGE
    perm = rng.permutation(num_pages).astype(np.int32)
    tables = np.zeros((T, max_pages), np.int32)
    nxt = 0
    for t in range(T):
        n = (int(lens[t]) + PAGE - 1) // PAGE
        tables[t, :n] = perm[nxt:nxt + n]
        nxt += n
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    kp = torch.randn(num_pages * PAGE, KVD, device=dev, generator=gen).to(torch.float16)
    vp = torch.randn(num_pages * PAGE, KVD, device=dev, generator=gen).to(torch.float16)
    q = torch.randn(T, QD, device=dev, generator=gen)
    pos, seq = (lens - 1).astype(np.int32), np.arange(T, dtype=np.int32)
    nc = ie.attention_chunks(4096, ct)
    ws = ie.attention_workspace(T, NH, HD, nc)
    d_pos, d_seq, d_tab = to_dev(pos, dev), to_dev(seq, dev), to_dev(tables, dev)
    plan = torch.from_numpy(planted_plan(ie, pos, seq, tables, nc, ct)).to(dev)
    a = torch.empty(T, QD, device=dev)
    b = torch.empty(T, QD, device=dev)
    ie.attention(a, q, kp, vp, d_pos, d_seq, d_tab, max_pages, nc, ct, ws, NH, NKV, HD)
    ie.attention_planned(b, q, kp, vp, d_pos, d_seq, d_tab, max_pages, nc, ct, ws, plan, NH, NKV,
                         HD)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


@pytest.mark.parametrize("kv", ["f16", "bf16"])
@pytest.mark.parametrize("ct", [128, 256])
def test_fused_planned_equals_unplanned(ie, O, dev, kv, ct):
    kvt = KVS[kv]
    rng = np.random.default_rng(1400 + ct + kvt)
    pos = np.array([0, 1, 15, 16, 31, 127, 128, 500, 2047, 2100, 700, 3000], np.int32)
    T = len(pos)
    tables, max_pages, num_pages = make_tables(pos + 1, rng, extra_pages=3)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    seq = np.arange(T, dtype=np.int32)
    q, k, v = normal(rng, (T, QD)), normal(rng, (T, KVD)), normal(rng, (T, KVD))
    table = ie.rope_table(2048, HD, 1e6).to(dev)  # row 9 (2100) and 11 (3000) lie past it
    nc = ie.attention_chunks(3001, ct)
    ws = ie.attention_workspace(T, NH, HD, nc)
    plan = torch.from_numpy(planted_plan(ie, pos, seq, tables, nc, ct)).to(dev)
    outs, pools = [], []
    for planned in (False, True):
        dkp, dvp = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt)
        out = torch.full((T, QD), 7.0, device=dev)
        args = (out, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), dkp, dvp, table,
                to_dev(pos, dev), to_dev(seq, dev), to_dev(tables, dev), int(max_pages), nc, ct, ws)
        if planned:
            ie.rope_cache_attention_planned(*args, plan, NH, NKV, HD)
        else:
            ie.rope_cache_attention(*args, NH, NKV, HD)
        torch.cuda.synchronize()
        outs.append(from_dev(out))
        pools.append((from_dev(dkp), from_dev(dvp)))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.array_equal(pools[0][0], pools[1][0]) and np.array_equal(pools[0][1], pools[1][1])


def test_planned_refuses_a_short_plan(ie, dev):
    T, nc, ct = 4, 3, 128
    small = torch.zeros(int(ie.attention_plan_ints(T, nc, ct)) - 4, dtype=torch.int32, device=dev)
    z = torch.zeros(T, QD, device=dev)
    pool = torch.zeros(16, KVD, dtype=torch.float16, device=dev)
    idx = torch.zeros(T, dtype=torch.int32, device=dev)
    tab = torch.zeros(T, 1, dtype=torch.int32, device=dev)
    ws = ie.attention_workspace(T, NH, HD, nc)
    with pytest.raises(ie.IeHipError, match="plan holds"):
        ie.attention_planned(z, z, pool, pool, idx, idx, tab, 1, nc, ct, ws, small, NH, NKV, HD)


def test_config4_fused_planned_full_size(ie, O, dev):
    """BASELINE config 4's benched call at full size: one row at position 32,767, bf16
    pages in a shuffled table, the library's chunk size for that grid,
    rope_cache_attention_planned. Pages bit-exact against the oracle's RoPE + append,
    attention within 2e-3 of the oracle over all 32,768 positions, and the same bits as
    ie_hip_rope_and_cache followed by ie_hip_attention."""
    kvt = KVS["bf16"]
    rng = np.random.default_rng(20264)
    L = 32768
    tables, max_pages, num_pages = make_tables([L], rng, extra_pages=64)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    pos, seq = np.array([L - 1], np.int32), np.zeros(1, np.int32)
    q, k, v = normal(rng, (1, QD)), normal(rng, (1, KVD)), normal(rng, (1, KVD))
    ct = ie.attention_chunk_tokens(1, L, kvt)
    nc = ie.attention_chunks(L, ct)
    table = ie.rope_table(L, HD, 1e6).to(dev)
    plan = torch.from_numpy(ie.attention_plan(pos, seq, tables, nc, ct)).to(dev)
    d_pos, d_seq, d_tab = to_dev(pos, dev), to_dev(seq, dev), to_dev(tables, dev)
    dk, dv = to_dev(k, dev), to_dev(v, dev)
    ws = ie.attention_workspace(1, NH, HD, nc)

    fkp, fvp = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt)
    fout = torch.full((1, QD), float("nan"), device=dev)
    ie.rope_cache_attention_planned(fout, to_dev(q, dev), dk, dv, fkp, fvp, table, d_pos, d_seq,
                                    d_tab, int(max_pages), nc, ct, ws, plan, NH, NKV, HD)
    tkp, tvp = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt)
    tq = to_dev(q, dev)
    tout = torch.full((1, QD), float("nan"), device=dev)
    ws2 = ie.attention_workspace(1, NH, HD, nc)
    ie.rope_and_cache(tq, dk, dv, tkp, tvp, table, d_pos, d_seq, d_tab, int(max_pages), NH, NKV,
                      HD)
    ie.attention(tout, tq, tkp, tvp, d_pos, d_seq, d_tab, int(max_pages), nc, ct, ws2, NH, NKV,
                 HD)
    torch.cuda.synchronize()

    q_ref, kp_ref, vp_ref = O.rope_append_paged(q, k, v, kp, vp, kvt, pos, seq, tables,
                                                int(max_pages), NH, NKV, HD, 1e6)
    assert np.array_equal(from_dev(fkp), kp_ref) and np.array_equal(from_dev(fvp), vp_ref)
    want = O.paged_attention(q_ref, kp_ref, vp_ref, kvt, pos, seq, tables, int(max_pages), NH,
                             NKV, HD, threads=8)
    got = from_dev(fout)
    assert np.all(np.isfinite(got))
    err = float(np.abs(got - want).max())
    assert err <= 2e-3, f"config 4: abs err {err:.3e} (chunk {ct}, {nc} chunks)"
    assert np.array_equal(got.view(np.uint32), from_dev(tout).view(np.uint32))


@pytest.mark.parametrize("fused,kv", [(False, "f16"), (True, "f16"), (False, "f32")])
def test_mismatched_plan_writes_nothing(ie, O, dev, fused, kv):
    """A plan built for another launch -- another chunk size, or another row count --
    passes the host's capacity check but would address other slots: the kernel
    compares the plan's header with its own arguments and writes nothing, neither
    partials, nor a single-chunk row's output, nor (fused) the appended rows. The
    merge kernel still runs over the untouched workspace, inside its bounds; the
    guard words past `out` and the workspace stay as they were."""
    kvt = KVS[kv]
    rng = np.random.default_rng(1500 + fused)
    lens = np.array([100, 700, 1500])
    T = len(lens)
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=3)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    pos, seq = (lens - 1).astype(np.int32), np.arange(T, dtype=np.int32)
    ct, nc = 256, ie.attention_chunks(1500, 256)
    plans = [ie.attention_plan(pos, seq, tables, ie.attention_chunks(1500, 128), 128),
             ie.attention_plan(pos[:2], seq[:2], tables, 2 * nc, ct)]
    q, k, v = normal(rng, (T, QD)), normal(rng, (T, KVD)), normal(rng, (T, KVD))
    table = ie.rope_table(2048, HD, 1e6).to(dev)
    for plan_h in plans:
        assert plan_h.size >= ie.attention_plan_ints(T, nc, ct)
        plan = torch.from_numpy(plan_h).to(dev)
        ws_n = ie.lib().ie_hip_attention_workspace_bytes(T, NH, HD, nc) // 4
        wsbuf = torch.full((ws_n + 256,), 5.0, device=dev)
        outbuf = torch.full((T * QD + 256,), 7.0, device=dev)
        out = outbuf[:T * QD].view(T, QD)
        ws = wsbuf[:ws_n]
        dkp, dvp = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt)
        args = (to_dev(pos, dev), to_dev(seq, dev), to_dev(tables, dev), int(max_pages), nc, ct,
                ws, plan, NH, NKV, HD)
        if fused:
            ie.rope_cache_attention_planned(out, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev),
                                            dkp, dvp, table, *args)
        else:
            ie.attention_planned(out, to_dev(q, dev), dkp, dvp, *args)
        torch.cuda.synchronize()
        assert torch.all(outbuf[T * QD:] == 7.0), "wrote past out"
        assert torch.all(wsbuf == 5.0), "the partial kernel wrote into the workspace"
        assert torch.all(out[0] == 7.0), "a single-chunk row was written"
        assert np.array_equal(from_dev(dkp), kp) and np.array_equal(from_dev(dvp), vp)
