"""Flash-decoding attention over pages on the GPU vs the CPU oracle.

Tolerances (north star): f32 KV -- the reference's metric max|d| / max|ref|
(src/npy.cpp:98-110) <= 1e-5; f16 / bf16 KV -- max |d| <= 2e-3 absolute. The
oracle attends over the same 16-bit values widened to f32. Outputs must also
be finite (the reference metric lets a NaN through unless it is last).
Cases: the golden fixtures (made from the reference's own CPU code), the
reference self-test's cases (src/cuda/cuda_runner.cu:914-941) including extra
empty chunks, several chunk sizes, and BASELINE config 3 at full size.
"""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

from helpers import HD, KVD, NH, NKV, QD, from_dev, kv_pool, make_tables, normal, to_dev

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KVS = {"f32": 0, "f16": 1, "bf16": 2}
F32_REL, HALF_ABS = 1e-5, 2e-3


def check(O, got, want, kvt, what=""):
    assert np.all(np.isfinite(got)), f"non-finite output {what}"
    if kvt == 0:
        rel = O.compare(got, want)[0]
        assert rel <= F32_REL, f"rel err {rel:.3e} {what}"
    else:
        err = float(np.abs(got - want).max())
        assert err <= HALF_ABS, f"abs err {err:.3e} {what}"


@pytest.fixture(params=["auto", "valu"])
def impl(request, ie):
    """Runs a test with the default kernels (MFMA for 16-bit caches) and with the VALU ones."""
    prev = ie.set_attention_impl({"auto": ie.IMPL_AUTO, "valu": ie.IMPL_VALU}[request.param])
    yield request.param
    ie.set_attention_impl(prev)


def gpu_attention(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, chunk_tokens,
                  num_chunks=None):
    T = len(row_pos)
    if num_chunks is None:
        num_chunks = ie.attention_chunks(int(np.max(row_pos)) + 1, chunk_tokens)
    ws = ie.attention_workspace(T, NH, HD, num_chunks)
    out = torch.full((T, QD), float("nan"), dtype=torch.float32, device=dev)
    ie.attention(out, to_dev(q, dev), to_dev(kp, dev, kvt), to_dev(vp, dev, kvt),
                 to_dev(row_pos, dev), to_dev(row_seq, dev), to_dev(tables, dev), max_pages,
                 num_chunks, chunk_tokens, ws, NH, NKV, HD)
    torch.cuda.synchronize()
    return from_dev(out)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "attn_*.npz"))),
                         ids=lambda p: os.path.basename(p)[5:-4])
@pytest.mark.parametrize("kv", list(KVS))
def test_golden(ie, O, dev, path, kv, impl):
    g = np.load(path)
    kvt = KVS[kv]
    tables, max_pages = g["tables"], g["tables"].shape[1]
    kf, vf = O.widen_kv(g["k_pool_f16"], 1), O.widen_kv(g["v_pool_f16"], 1)
    kp, vp = O.round_to_kv(kf, kvt), O.round_to_kv(vf, kvt)
    if kvt == 2:  # bf16 pools hold different values: the oracle recomputes the expectation
        want = O.paged_attention(g["q"], kp, vp, kvt, g["row_pos"], g["row_seq"], tables, max_pages,
                                 NH, NKV, HD)
    else:
        want = g["out"]
    for ct in (16, 64, 512):
        got = gpu_attention(ie, dev, g["q"], kp, vp, kvt, g["row_pos"], g["row_seq"], tables,
                            max_pages, ct)
        check(O, got, want, kvt, f"chunk {ct}")


SELFTEST = [
    # lens, rows, capacity (the launch covers `capacity` positions: extra chunks are empty)
    ([1], [(0, 0)], 1),
    ([64], [(0, 63)], 64),
    ([65], [(0, 64)], 1000),
    ([256], [(0, 255)], 256),
    ([257], [(0, 256)], 4096),
    ([3000], [(0, 2999)], 3000),
    ([540], [(0, p) for p in range(500, 540)], 540),
    ([6, 17, 256, 257, 3000], [(0, 5), (1, 16), (2, 255), (3, 256), (4, 2999)], 4096),
    ([101, 30, 1001], [(0, 100), (2, 1000)] + [(1, p) for p in range(30)], 1024),
]


@pytest.mark.parametrize("case", range(len(SELFTEST)))
@pytest.mark.parametrize("kv", list(KVS))
@pytest.mark.parametrize("chunk_tokens", [64, 256, 512])
def test_selftest_cases(ie, O, dev, case, kv, chunk_tokens, impl):
    lens, rows, capacity = SELFTEST[case]
    kvt = KVS[kv]
    rng = np.random.default_rng(100 + case)
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=3)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_seq = np.array([r[0] for r in rows], np.int32)
    row_pos = np.array([r[1] for r in rows], np.int32)
    q = normal(rng, (len(rows), QD))
    want = O.paged_attention(q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, NH, NKV, HD,
                             threads=8)
    nc = ie.attention_chunks(capacity, chunk_tokens)
    got = gpu_attention(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, chunk_tokens,
                        num_chunks=nc)
    check(O, got, want, kvt, f"case {case}")


def test_page_permutation_invariance(ie, O, dev, impl):
    """The same logical K/V under two page permutations gives the same output (bit-exact:
    the kernel's arithmetic depends only on positions, not on where pages live)."""
    rng = np.random.default_rng(7)
    L, kvt = 1500, 1
    logical_k = kv_pool(rng, (L + 15) // 16, kvt, O)
    logical_v = kv_pool(rng, (L + 15) // 16, kvt, O)
    q = normal(rng, (1, QD))
    outs = []
    for seed in (1, 2):
        tables, max_pages, num_pages = make_tables([L], np.random.default_rng(seed), extra_pages=4)
        kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
        for p in range(L):
            kp[tables[0, p // 16] * 16 + p % 16] = logical_k[p]
            vp[tables[0, p // 16] * 16 + p % 16] = logical_v[p]
        outs.append(gpu_attention(ie, dev, q, kp, vp, kvt, np.array([L - 1], np.int32),
                                  np.zeros(1, np.int32), tables, max_pages, 256))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


def test_chunk_size_invariance(ie, O, dev, impl):
    """Split-K partition size changes only rounding (log-sum-exp merge is exact)."""
    rng = np.random.default_rng(8)
    lens = [4096, 129, 2000]
    tables, max_pages, num_pages = make_tables(lens, rng)
    kvt = 1
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_pos = np.array([n - 1 for n in lens], np.int32)
    row_seq = np.arange(len(lens), dtype=np.int32)
    q = normal(rng, (len(lens), QD))
    outs = [gpu_attention(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, ct)
            for ct in (64, 128, 512)]
    assert np.abs(outs[0] - outs[1]).max() < 2e-6 and np.abs(outs[0] - outs[2]).max() < 2e-6


@pytest.mark.parametrize("kv", ["f16", "f32"])
@pytest.mark.parametrize("partition", ["512", "bench"])
def test_config3_full_size(ie, O, dev, kv, impl, partition):
    """batch 64, L ~ U[128, 4096], 16-token pages, tables a seeded
    permutation of a 65,536-page pool; 512-token partitions (BASELINE's), and the
    partition bench.py times (the library's own choice for 64 rows of up to 4,096
    tokens, over the chunk count of the full 4,096)."""
    rng = np.random.default_rng(20263)
    kvt = KVS[kv]
    num_pages = 65536
    lens = rng.integers(128, 4097, 64)
    max_pages = 4096 // 16
    perm = rng.permutation(num_pages).astype(np.int32)
    tables = np.zeros((64, max_pages), np.int32)
    nxt = 0
    for s, n in enumerate(lens):
        k = (int(n) + 15) // 16
        tables[s, :k] = perm[nxt:nxt + k]
        nxt += k
    kp = kv_pool(rng, num_pages, kvt, O)
    vp = kv_pool(rng, num_pages, kvt, O)
    row_pos = (lens - 1).astype(np.int32)
    row_seq = np.arange(64, dtype=np.int32)
    q = normal(rng, (64, QD))
    want = O.paged_attention(q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, NH, NKV, HD,
                             threads=8)
    if partition == "512":
        ct, nc = 512, 8
    else:
        ct = ie.attention_chunk_tokens(64, 4096, kvt)
        nc = ie.attention_chunks(4096, ct)
    got = gpu_attention(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, ct,
                        num_chunks=nc)
    check(O, got, want, kvt, f"config 3, {ct}-token chunks")


@pytest.mark.parametrize("rows", [1, 12, 24])
@pytest.mark.parametrize("kv", list(KVS))
def test_merge_layouts(ie, O, dev, rows, kv, impl):
    """Split-K merge layouts: rows x heads below and above the compute-unit count (4 dim
    slices of one wave per (head, row) for 1 and 12 rows; 1 slice of four waves, with the
    LDS stage, for 24) with 64-token chunks over contexts up to 8,192 (128 chunks), mixed
    with rows that fit one chunk."""
    rng = np.random.default_rng(100 + rows)
    lens = [8192] + [int(x) for x in rng.integers(1, 8193, rows - 1)]
    if rows > 2:
        lens[1], lens[2] = 64, 65  # one chunk exactly; one position into a second chunk
    kvt = KVS[kv]
    tables, max_pages, num_pages = make_tables(lens, rng)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_pos = np.array([n - 1 for n in lens], np.int32)
    row_seq = np.arange(rows, dtype=np.int32)
    q = normal(rng, (rows, QD))
    want = O.paged_attention(q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, NH, NKV, HD,
                             threads=8)
    got = gpu_attention(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, 64)
    check(O, got, want, kvt, f"rows {rows}")


def test_config4_full_size(ie, O, dev):
    """BASELINE config 4's attention: batch 1, context 32,768, bf16 KV, shuffled 16-token
    pages, with the library's own chunk choice (256 chunks of 128 tokens: a merge of 8 dim
    slices, its lane tree on DPP moves and v_permlane16_swap)."""
    rng = np.random.default_rng(20263)
    kvt = KVS["bf16"]
    L = 32768
    tables, max_pages, num_pages = make_tables([L], rng)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_pos, row_seq = np.array([L - 1], np.int32), np.zeros(1, np.int32)
    q = normal(rng, (1, QD))
    ct = ie.attention_chunk_tokens(1, L, ie.KV_BF16)
    want = O.paged_attention(q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, NH, NKV, HD,
                             threads=8)
    got = gpu_attention(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, ct)
    check(O, got, want, kvt, f"config 4, chunk {ct}")


@pytest.mark.parametrize("rows,L", [(1, 32768), (2, 65536)])
def test_merge_lane_tree_widths(ie, O, dev, rows, L):
    """The widest merge lane trees: 64-token chunks over 32,768 positions (512 chunks: 16
    dim slices of one wave, the lane tree's last level on v_permlane32_swap) and over
    65,536 (1,024 chunks: 16 slices of two waves, then the LDS stage)."""
    rng = np.random.default_rng(300 + rows)
    kvt = KVS["f16"]
    lens = [L] + [int(x) for x in rng.integers(1, L + 1, rows - 1)]
    tables, max_pages, num_pages = make_tables(lens, rng)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_pos = np.array([n - 1 for n in lens], np.int32)
    row_seq = np.arange(rows, dtype=np.int32)
    q = normal(rng, (rows, QD))
    want = O.paged_attention(q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, NH, NKV, HD,
                             threads=8)
    got = gpu_attention(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, 64)
    check(O, got, want, kvt, f"rows {rows}, L {L}")


@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_mfma_forced_and_shape_limits(ie, O, dev, kv):
    """IMPL_MFMA runs the matrix-core kernel; shapes it cannot take fail loudly (no silent fallback)."""
    kvt = KVS[kv]
    rng = np.random.default_rng(9)
    tables, max_pages, num_pages = make_tables([700], rng)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    q = normal(rng, (1, QD))
    pos, seq = np.array([699], np.int32), np.zeros(1, np.int32)
    want = O.paged_attention(q, kp, vp, kvt, pos, seq, tables, max_pages, NH, NKV, HD)
    prev = ie.set_attention_impl(ie.IMPL_MFMA)
    try:
        check(O, gpu_attention(ie, dev, q, kp, vp, kvt, pos, seq, tables, max_pages, 128), want, kvt)
        with pytest.raises(ie.IeHipError):
            gpu_attention(ie, dev, q, kp, vp, kvt, pos, seq, tables, max_pages, 48)
    finally:
        ie.set_attention_impl(prev)


@pytest.mark.parametrize("kv", ["f16", "f32"])
def test_graph_replay_matches_eager(ie, O, dev, kv):
    """A decode step (append + attention) recorded into a HIP graph replays to the eager
    result every time, with eager work and synchronisations between the replays (the
    library records no memset nodes: every node is one of its kernels)."""
    kvt = KVS[kv]
    rng = np.random.default_rng(31)
    lens = [700, 1300, 90, 2049]
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=2)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_pos = np.array([n - 1 for n in lens], np.int32)
    row_seq = np.arange(len(lens), dtype=np.int32)
    q, k, v = normal(rng, (4, QD)), normal(rng, (4, KVD)), normal(rng, (4, KVD))
    table = ie.rope_table(4096, HD, 1e6).to(dev)
    dkp, dvp = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt)
    dtab, dpos, dseq = to_dev(tables, dev), to_dev(row_pos, dev), to_dev(row_seq, dev)
    dk, dv = to_dev(k, dev), to_dev(v, dev)
    ct = ie.attention_chunk_tokens(4, 4096, kvt)
    nc = ie.attention_chunks(4096, ct)
    ws = ie.attention_workspace(4, NH, HD, nc)
    q0 = to_dev(q, dev)
    dq = q0.clone()
    out = torch.empty((4, QD), dtype=torch.float32, device=dev)

    def step():
        dq.copy_(q0)
        ie.rope_and_cache(dq, dk, dv, dkp, dvp, table, dpos, dseq, dtab, max_pages, NH, NKV, HD)
        ie.attention(out, dq, dkp, dvp, dpos, dseq, dtab, max_pages, nc, ct, ws, NH, NKV, HD)

    step()
    torch.cuda.synchronize()
    eager = from_dev(out).copy()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for i in range(4):
        out.fill_(float("nan"))
        scratch = torch.randn(1 << 20, device=dev).sum()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = from_dev(out)
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {i}"
    del scratch


@pytest.mark.parametrize("kv", list(KVS))
def test_stale_nonfinite_pool_rows_do_not_leak(ie, O, dev, kv, impl):
    """Pool rows the attention must not see -- the tail of each row's last page, every
    other page of the pool -- hold inf and NaN; outputs stay finite and match the oracle
    (which only ever reads positions 0..p)."""
    kvt = KVS[kv]
    rng = np.random.default_rng(43)
    lens = [37, 200, 1, 130]
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=3)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    used = np.zeros(num_pages * 16, bool)
    for s_, n in enumerate(lens):
        for p_ in range(n):
            used[tables[s_, p_ // 16] * 16 + p_ % 16] = True
    poison = O.round_to_kv(np.resize(np.array([np.nan, np.inf], np.float32),
                                     (int((~used).sum()), KVD)).astype(np.float32), kvt)
    kp[~used] = poison
    vp[~used] = poison
    row_pos = np.array([n - 1 for n in lens], np.int32)
    row_seq = np.arange(len(lens), dtype=np.int32)
    q = normal(rng, (len(lens), QD))
    want = O.paged_attention(q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, NH, NKV, HD)
    for ct in (64, 128, 256):
        got = gpu_attention(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, ct)
        check(O, got, want, kvt, f"chunk {ct}")


@pytest.mark.parametrize("kv", list(KVS))
def test_out_of_pool_pages_are_skipped(ie, O, dev, kv, impl):
    """Table entries outside the pool (past it or negative) inside rows' contexts: the
    kernels never dereference them and their positions are not attended, while every
    pool row the attention may not see holds inf/NaN. Cases: two pages in the middle
    of a row; the row's first page; its last page (its own position among the
    skipped ones); a whole 128-position chunk (an all-skipped partial in the merge).
    Expected: per row, the oracle's attention over the sequence with the skipped
    positions removed, where the row's query sits at the last kept position <= p."""
    kvt = KVS[kv]
    rng = np.random.default_rng(47)
    lens = [700, 100, 300, 700]
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=3)
    good = tables.copy()
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    used = np.zeros(num_pages * 16, bool)
    for s_, n in enumerate(lens):
        for p_ in range(n):
            used[good[s_, p_ // 16] * 16 + p_ % 16] = True
    poison = O.round_to_kv(np.resize(np.array([np.nan, np.inf], np.float32),
                                     (int((~used).sum()), KVD)).astype(np.float32), kvt)
    kp[~used] = poison
    vp[~used] = poison
    skipped = {0: [5, 6], 1: [0], 2: [18], 3: list(range(8, 16))}
    for s_, pages in skipped.items():
        for i, pg in enumerate(pages):
            tables[s_, pg] = num_pages + 5 if i % 2 == 0 else -2
    row_pos = np.array([n - 1 for n in lens], np.int32)
    row_seq = np.arange(len(lens), dtype=np.int32)
    q = normal(rng, (len(lens), QD))
    want = np.empty_like(q)
    for s_, n in enumerate(lens):
        keep = np.array([p_ for p_ in range(n) if p_ // 16 not in skipped[s_]])
        kc = O.gather_kv(kp, kvt, good, max_pages, s_, n, KVD)[keep]
        vc = O.gather_kv(vp, kvt, good, max_pages, s_, n, KVD)[keep]
        want[s_] = O.attention(q[s_:s_ + 1], kc, vc, len(keep) - 1, NH, NKV, HD)[0]
    for ct in (64, 128, 256):
        got = gpu_attention(ie, dev, q, kp, vp, kvt, row_pos, row_seq, tables, max_pages, ct)
        check(O, got, want, kvt, f"chunk {ct}")


BATCH_SHAPES = [
    # rows, context length range [lo, hi), chunk tokens (None: the library's choice)
    (64, (128, 4097), None),  # BASELINE config 3's shape (the library's 192-token chunks)
    (64, (1, 300), 64),
    (200, (1, 2000), 128),
    (256, (1, 700), 64),
    (257, (1, 700), 64),
    (3, (1, 5000), 64),
    (1, (2000, 2001), 64),
    (40, (1, 40), 64),        # every row inside its first chunk
]


@pytest.mark.parametrize("case", range(len(BATCH_SHAPES)))
@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_batch_shapes(ie, O, dev, case, kv):
    """Batches of 1 to 257 rows of random lengths with one-wave and four-wave chunk
    workgroups. Rows with position -1 take no work and their output is left as it was; a
    row past the chunks' capacity (num_chunks * chunk_tokens positions) attends to that
    many (expected: the oracle at the last covered position). A second call on the same
    workspace, with other lengths, must not read the first call's partials."""
    T, (lo, hi), ct = BATCH_SHAPES[case]
    kvt = KVS[kv]
    rng = np.random.default_rng(900 + case)
    lens = rng.integers(lo, hi, T)
    tables, max_pages, num_pages = make_tables(lens, rng, extra_pages=3)
    max_pages = int(max_pages)
    kp, vp = kv_pool(rng, num_pages, kvt, O), kv_pool(rng, num_pages, kvt, O)
    row_seq = np.arange(T, dtype=np.int32)
    if ct is None:
        ct = ie.attention_chunk_tokens(T, int(lens.max()), kvt)
    nc = ie.attention_chunks(int(lens.max()), ct)
    ws = ie.attention_workspace(T, NH, HD, nc)
    d_kp, d_vp, d_tab = to_dev(kp, dev, kvt), to_dev(vp, dev, kvt), to_dev(tables, dev)
    d_seq = to_dev(row_seq, dev)
    for call in range(2):
        pos = (lens - 1).astype(np.int32)
        if call == 1:  # shorter contexts: other chunk counts per row
            pos = (rng.integers(1, lens + 1) - 1).astype(np.int32)
        empty = rng.random(T) < (0.1 if T > 4 else 0.0)
        pos[empty] = -1
        capped = None
        if T >= 40 and call == 0:  # one row past the capacity of nc - 1 chunks
            capped = int(np.argmax(np.where(empty, -1, pos)))
        ncall = nc - 1 if capped is not None and nc > 1 and pos[capped] >= (nc - 1) * ct else nc
        q = normal(rng, (T, QD))
        eff = np.minimum(pos, ncall * ct - 1).astype(np.int32)
        live = pos >= 0
        want = O.paged_attention(q[live], kp, vp, kvt, eff[live], row_seq[live], tables,
                                 max_pages, NH, NKV, HD, threads=8)
        out = torch.full((T, QD), 7.0, dtype=torch.float32, device=dev)
        ie.attention(out, to_dev(q, dev), d_kp, d_vp, to_dev(pos, dev), d_seq, d_tab, max_pages,
                     ncall, ct, ws, NH, NKV, HD)
        torch.cuda.synchronize()
        got = from_dev(out)
        check(O, got[live], want, kvt, f"call {call}, chunk {ct}, {ncall} chunks")
        assert np.all(got[~live] == 7.0), "rows with position -1 must be left untouched"
