"""Prefill (prompt-chunk) attention into pages on the GPU vs the CPU oracle.

Same tolerances as decode (f32: rel 1e-5; f16/bf16: 2e-3 abs). Cases: the
reference self-test's prompts (src/cuda/cuda_runner.cu:920-934: 1, 17, 300,
1000 rows; a prompt continuing at 500; the 2nd of 2 sequences), a prompt whose
keys run past 32,768 (the kernels stage page ids 512 tiles at a time), and the
4,000-token prefill of BASELINE config 5, appended into fresh pages of a
churned pool with the fused RoPE+append kernel first (all 4,000 rows checked
against the oracle). Decode and prefill kernels must agree on the same rows. The
f16 prefill's single rounding of P is checked at its worst: rows with few keys
whose V rows lie far apart.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import HD, KVD, NH, NKV, QD, THETA, from_dev, kv_pool, make_tables, normal, to_dev
from test_gpu_decode import check, gpu_attention

pytestmark = pytest.mark.gpu
KVS = {"f32": 0, "f16": 1, "bf16": 2}


@pytest.fixture(params=["auto", "valu"])
def impl(request, ie):
    """Runs a test with the default kernels (MFMA for 16-bit caches) and with the VALU ones."""
    prev = ie.set_attention_impl({"auto": ie.IMPL_AUTO, "valu": ie.IMPL_VALU}[request.param])
    yield request.param
    ie.set_attention_impl(prev)


def gpu_prefill(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages):
    out = torch.full((len(row_pos), QD), float("nan"), dtype=torch.float32, device=dev)
    ie.attention_prefill(out, to_dev(q, dev), to_dev(kp, dev, kvt), to_dev(vp, dev, kvt),
                         to_dev(row_pos, dev), to_dev(row_seq, dev), to_dev(tables, dev), max_pages,
                         NH, NKV, HD)
    torch.cuda.synchronize()
    return from_dev(out)


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
def test_prompts(ie, O, dev, case, kv, impl):
    lens, seq, start, T = PROMPTS[case]
    kvt = KVS[kv]
    rng = np.random.default_rng(200 + case)
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=2)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_pos = np.arange(start, start + T, dtype=np.int32)
    row_seq = np.full(T, seq, np.int32)
    q = normal(rng, (T, QD))
    want = O.paged_attention(q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, NH, NKV, HD,
                             threads=8)
    got = gpu_prefill(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages)
    check(O, got, want, kvt, f"prompt case {case}")
    dec = gpu_attention(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, 256)
    check(O, dec, want, kvt, f"decode kernel on prompt case {case}")


@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_config5_mixed_step_into_churned_pool(ie, O, dev, kv, impl):
    """BASELINE config 5, both halves of the step: 48 decode sequences (contexts
    U[256, 2048]) hold pages; 12 of them (25%) finish and 12 new ones take their pages
    back from the free list; then a 4,000-token prompt is appended into fresh pages
    (RoPE+append kernel) and attended causally, and the 48 decode rows append their new
    token and attend. Pages are checked bit-exactly; attention on every decode row and
    on 256 sampled prompt rows plus the page and tile edges."""
    kvt = KVS[kv]
    rng = np.random.default_rng(20265)
    num_pages, T = 8192, 4000
    pool = ie.PagePool(num_pages, 64, 8192)
    seqs = [pool.open_sequence() for _ in range(48)]
    lens = {}
    for s in seqs:
        lens[s] = int(rng.integers(256, 2049))
        pool.ensure(s, lens[s])
    done = [int(s) for s in rng.permutation(seqs)[:12]]  # 25% of the decode sequences finish
    for s in done:
        pool.close_sequence(s)
        del lens[s]
    for _ in done:  # ... and new ones re-allocate their pages from the free list
        s = pool.open_sequence()
        lens[s] = int(rng.integers(256, 2049))
        pool.ensure(s, lens[s])
    dec = sorted(lens)
    assert len(dec) == 48
    p = pool.open_sequence()
    pool.ensure(p, T)
    max_pages = pool.max_pages_per_seq
    tables = np.array(pool.host_tables(), np.int32).reshape(pool.max_batch, max_pages)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    q = normal(rng, (T, QD))
    k = normal(rng, (T, KVD))
    v = normal(rng, (T, KVD))
    row_pos = np.arange(T, dtype=np.int32)
    row_seq = np.full(T, p, np.int32)
    q_rot, kp_ref, vp_ref = O.rope_append_paged(q, k, v, kp, vp, kvt, row_pos, row_seq, tables,
                                                max_pages, NH, NKV, HD, THETA)
    dq = to_dev(q, dev)
    dkp, dvp = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt)
    dtab = torch.zeros(tables.size, dtype=torch.int32, device=dev)
    assert pool.upload_tables(dtab)
    table = ie.rope_table(8192, HD, THETA).to(dev)
    dpos, dseq = to_dev(row_pos, dev), to_dev(row_seq, dev)
    ie.rope_and_cache(dq, to_dev(k, dev), to_dev(v, dev), dkp, dvp, table, dpos, dseq, dtab,
                      max_pages, NH, NKV, HD)
    out = torch.full((T, QD), float("nan"), dtype=torch.float32, device=dev)
    ie.attention_prefill(out, dq, dkp, dvp, dpos, dseq, dtab, max_pages, NH, NKV, HD)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(dq).view(np.uint32), q_rot.view(np.uint32))
    assert np.array_equal(from_dev(dkp), kp_ref) and np.array_equal(from_dev(dvp), vp_ref)
    # Every one of the 4,000 rows, against the oracle's causal attention over the
    # prompt gathered out of the churned pool (one contiguous copy, as the reference
    # self-test gathers, src/cuda/cuda_runner.cu:959-965).
    kc = O.gather_kv(kp_ref, kvt, tables, max_pages, p, T, KVD)
    vc = O.gather_kv(vp_ref, kvt, tables, max_pages, p, T, KVD)
    want = O.attention(q_rot, kc, vc, 0, NH, NKV, HD, threads=8)
    check(O, from_dev(out), want, kvt, "config 5 prefill, all 4,000 rows")

    # The decode half: each sequence's new token at its current length, appended and
    # attended in one decode launch over the same (churned) pool.
    for s in dec:
        pool.ensure(s, lens[s] + 1)
    tables = np.array(pool.host_tables(), np.int32).reshape(pool.max_batch, max_pages)
    pool.upload_tables(dtab)
    n = len(dec)
    dpos_h = np.array([lens[s] for s in dec], np.int32)
    dseq_h = np.array(dec, np.int32)
    qd, kd, vd = normal(rng, (n, QD)), normal(rng, (n, KVD)), normal(rng, (n, KVD))
    qd_rot, kp_ref, vp_ref = O.rope_append_paged(qd, kd, vd, kp_ref, vp_ref, kvt, dpos_h, dseq_h,
                                                 tables, max_pages, NH, NKV, HD, THETA)
    dqd = to_dev(qd, dev)
    ddpos, ddseq = to_dev(dpos_h, dev), to_dev(dseq_h, dev)
    ie.rope_and_cache(dqd, to_dev(kd, dev), to_dev(vd, dev), dkp, dvp, table, ddpos, ddseq, dtab,
                      max_pages, NH, NKV, HD)
    ct = ie.attention_chunk_tokens(n, 2049, kvt)
    nc = ie.attention_chunks(2049, ct)
    ws = ie.attention_workspace(n, NH, HD, nc)
    dout = torch.full((n, QD), float("nan"), dtype=torch.float32, device=dev)
    ie.attention(dout, dqd, dkp, dvp, ddpos, ddseq, dtab, max_pages, nc, ct, ws, NH, NKV, HD)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(dqd).view(np.uint32), qd_rot.view(np.uint32))
    assert np.array_equal(from_dev(dkp), kp_ref) and np.array_equal(from_dev(dvp), vp_ref)
    want = O.paged_attention(qd_rot, kp_ref, vp_ref, kvt, dpos_h, dseq_h, tables, max_pages, NH,
                             NKV, HD, threads=8)
    check(O, from_dev(dout), want, kvt, "config 5 decode rows")


@pytest.mark.parametrize("kv", list(KVS))
def test_mfma_forced(ie, O, dev, kv):
    """IMPL_MFMA runs the matrix-core prefill kernels for every KV type: 16-bit caches
    in their own type (f16: q and P rounded once; bf16: hi + lo operands), f32 caches on
    the f32 matrix instructions."""
    kvt = KVS[kv]
    rng = np.random.default_rng(41)
    tables, max_pages, num_pages = make_tables([333], rng)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_pos = np.arange(100, 333, dtype=np.int32)
    row_seq = np.zeros(len(row_pos), np.int32)
    q = normal(rng, (len(row_pos), QD))
    want = O.paged_attention(q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, NH, NKV, HD,
                             threads=8)
    prev = ie.set_attention_impl(ie.IMPL_MFMA)
    try:
        check(O, gpu_prefill(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages), want,
              kvt)
    finally:
        ie.set_attention_impl(prev)


@pytest.mark.parametrize("kv", list(KVS))
def test_stale_nonfinite_pool_rows_do_not_leak(ie, O, dev, kv, impl):
    """Prefill over a pool whose rows past the prompt (and all unused pages) hold inf/NaN."""
    kvt = KVS[kv]
    rng = np.random.default_rng(44)
    L = 150  # the sequence's pages cover 160 positions; 150..159 are stale
    tables, max_pages, num_pages = make_tables([L + 10], rng, extra_pages=2)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    used = np.zeros(num_pages * 16, bool)
    for p_ in range(L):
        used[tables[0, p_ // 16] * 16 + p_ % 16] = True
    poison = O.round_to_kv(np.resize(np.array([np.inf, np.nan], np.float32),
                                     (int((~used).sum()), KVD)).astype(np.float32), kvt)
    kp[~used] = poison
    vp[~used] = poison
    row_pos = np.arange(40, L, dtype=np.int32)
    row_seq = np.zeros(len(row_pos), np.int32)
    q = normal(rng, (len(row_pos), QD))
    want = O.paged_attention(q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, NH, NKV, HD)
    check(O, gpu_prefill(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages), want, kvt,
          "stale rows")


@pytest.mark.parametrize("kv", list(KVS))
def test_out_of_pool_pages_are_skipped(ie, O, dev, kv, impl):
    """Table entries outside the pool (one past it, one negative) inside a prompt's
    context: the kernels never dereference them and their 32 keys are invisible
    (scores masked, V elements zeroed), while every other byte of the pool holds
    inf/NaN. Expected: the oracle's attention over the sequence with those 32
    positions removed -- rows at positions p >= 48 then see the first p + 1 - 32
    keys of the compacted copy, i.e. position p - 32 of it."""
    kvt = KVS[kv]
    rng = np.random.default_rng(46)
    L, start = 300, 100
    tables, max_pages, num_pages = make_tables([L], rng, extra_pages=2)
    good = tables.copy()
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    used = np.zeros(num_pages * 16, bool)
    for p_ in range(L):
        used[good[0, p_ // 16] * 16 + p_ % 16] = True
    poison = O.round_to_kv(np.resize(np.array([np.inf, np.nan], np.float32),
                                     (int((~used).sum()), KVD)).astype(np.float32), kvt)
    kp[~used] = poison
    vp[~used] = poison
    tables[0, 1] = num_pages + 7  # positions 16..31
    tables[0, 2] = -3             # positions 32..47
    row_pos = np.arange(start, L, dtype=np.int32)
    row_seq = np.zeros(len(row_pos), np.int32)
    q = normal(rng, (len(row_pos), QD))
    keep = np.r_[0:16, 48:L]
    kc = O.gather_kv(kp, kvt, good, max_pages, 0, L, KVD)[keep]
    vc = O.gather_kv(vp, kvt, good, max_pages, 0, L, KVD)[keep]
    want = O.attention(q, kc, vc, start - 32, NH, NKV, HD, threads=8)
    check(O, gpu_prefill(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages), want, kvt,
          "out-of-pool pages")


@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_few_keys_far_apart_values(ie, O, dev, kv):
    """The f16 prefill rounds each weight once (to nearest, as the reference's tensor-core
    kernel does, src/cuda/kernels.cu:741), which moves a row's output by at most
    2^-11 * sum_i w_i |v_i - o|. That is largest where a row has few keys, of nearly
    equal weight, whose V rows lie far apart: here the first 16 rows of a prompt over
    keys whose V rows alternate between +3 and -3 in every dim (exact in both 16-bit
    types), with small queries (near-uniform weights). Worst case 2^-11 * 3 = 1.5e-3,
    inside the 2e-3 bound; rounding toward zero would allow twice that bias."""
    kvt = KVS[kv]
    rng = np.random.default_rng(47)
    T = 64
    tables, max_pages, num_pages = make_tables([T], rng, extra_pages=1)
    kp = kv_pool(rng, num_pages, kvt, O)
    vp = kv_pool(rng, num_pages, kvt, O)
    sign = np.where(np.arange(T) % 2 == 0, 3.0, -3.0).astype(np.float32)
    for p_ in range(T):
        vp[tables[0, p_ // 16] * 16 + p_ % 16] = O.round_to_kv(
            np.full(KVD, sign[p_] * (1.0 + 0.01 * (p_ % 5)), np.float32), kvt)
    row_pos = np.arange(T, dtype=np.int32)
    row_seq = np.zeros(T, np.int32)
    q = normal(rng, (T, QD), scale=0.05)
    want = O.paged_attention(q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, NH, NKV, HD)
    got = gpu_prefill(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages)
    err = float(np.abs(got[:16] - want[:16]).max())
    assert err <= 2e-3, f"rows 0-15: max abs error {err:.3e}"
    check(O, got, want, kvt, "few keys, far-apart values")


def test_f16_split_rounding_mode(ie, O, dev):
    """ie_hip_set_prefill_rounding (the counterpart of the reference's set_tc_fp16):
    PREFILL_SPLIT gives an f16 cache's prefill hi + lo operands, float32-level
    results (the bf16 path's ~1e-6); PREFILL_SINGLE (the default) rounds q and P once
    (~1e-4). Both within the 2e-3 bound; the switch restores."""
    kvt = KVS["f16"]
    rng = np.random.default_rng(48)
    tables, max_pages, num_pages = make_tables([1000], rng)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_pos = np.arange(1000, dtype=np.int32)
    row_seq = np.zeros(1000, np.int32)
    q = normal(rng, (1000, QD))
    want = O.paged_attention(q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, NH, NKV, HD,
                             threads=8)
    errs = {}
    for mode in (ie.PREFILL_SPLIT, ie.PREFILL_SINGLE):
        prev = ie.set_prefill_rounding(mode)
        try:
            got = gpu_prefill(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages)
        finally:
            ie.set_prefill_rounding(prev)
        errs[mode] = float(np.abs(got - want).max())
    assert errs[ie.PREFILL_SPLIT] <= 2e-5, errs
    assert errs[ie.PREFILL_SINGLE] <= 2e-3, errs
    assert errs[ie.PREFILL_SPLIT] < errs[ie.PREFILL_SINGLE], errs
    assert ie.set_prefill_rounding(ie.PREFILL_SINGLE) == ie.PREFILL_SINGLE
