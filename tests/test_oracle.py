"""Pins the CPU oracle (oracle/) before anything is compared against it.

Checks, per oracle function:
  * bit-exact agreement with the reference's own CPU code (oracle/_ref, built
    from src/ops.cpp + src/threadpool.cpp) -- when that build is present;
  * the committed golden fixtures (tests/golden, made from oracle/_ref);
  * closed forms and invariants chosen so a dropped term, a wrong sign, a
    transposed index or a changed rounding fails.
"""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

from helpers import HD, KVD, NH, NKV, QD, THETA, normal, make_tables

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
needs_ref = pytest.mark.skipif(
    not __import__("oracle").ref_available(), reason="oracle/_ref not built (no reference checkout)")


def u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------------ RoPE ----
@needs_ref
@pytest.mark.parametrize("pos", [0, 1, 2, 17, 511, 4095, 8191, 32767, 99991])
def test_rope_matches_reference_build(O, pos):
    rng = np.random.default_rng(pos)
    x = normal(rng, (3, QD), 2.0)
    assert np.array_equal(u32(O.rope(x, NH, HD, pos, THETA)), u32(O.ref_rope(x, NH, HD, pos, THETA)))


@needs_ref
def test_rope_many_positions_and_geometries(O):
    rng = np.random.default_rng(3)
    for hd, nh, theta in [(64, 2, 1e6), (128, 4, 1e4), (32, 3, 5e5)]:
        x = normal(rng, (257, nh * hd))
        assert np.array_equal(u32(O.rope(x, nh, hd, 1000, theta)),
                              u32(O.ref_rope(x, nh, hd, 1000, theta)))


def test_rope_position_zero_is_identity(O):
    x = normal(np.random.default_rng(1), (1, QD), 3.0)
    assert np.array_equal(u32(O.rope(x, NH, HD, 0, THETA)), u32(x))


def test_rope_matches_fp64_rotation(O):
    """The rotation pairs element i with i + 32, angle pos * theta^(-2i/64)."""
    rng = np.random.default_rng(2)
    x = normal(rng, (1, NKV * HD))
    pos = 1234
    got = O.rope(x, NKV, HD, pos, THETA).reshape(NKV, HD)
    xh = x.astype(np.float64).reshape(NKV, HD)
    i = np.arange(HD // 2)
    ang = pos * THETA ** (-2.0 * i / HD)
    c, s = np.cos(ang), np.sin(ang)
    want = np.concatenate([xh[:, :32] * c - xh[:, 32:] * s, xh[:, 32:] * c + xh[:, :32] * s], 1)
    # float32 angle (pos * inv_freq rounded) limits agreement to ~pos * 2^-24 rad
    assert np.abs(got - want).max() < 5e-4
    # swapping the sign of the sin term (a plausible slip) is far outside that
    wrong = np.concatenate([xh[:, :32] * c + xh[:, 32:] * s, xh[:, 32:] * c - xh[:, :32] * s], 1)
    assert np.abs(got - wrong).max() > 1e-2


def test_rope_table_matches_rope(O):
    """Rotating with the oracle's cos/sin table reproduces orc_rope exactly."""
    tab = O.rope_table(600, HD, THETA)
    rng = np.random.default_rng(4)
    x = normal(rng, (1, KVD))
    for pos in (0, 5, 599):
        c, s = tab[pos, :32], tab[pos, 32:]
        y = x.reshape(NKV, HD).copy()
        x0, x1 = y[:, :32].copy(), y[:, 32:].copy()
        # fma(x0, c, -(x1*s)) via float64 on exact float32 products is exact here
        r0 = (x0.astype(np.float64) * c - (x1 * s).astype(np.float32)).astype(np.float32)
        r1 = (x1.astype(np.float64) * c + (x0 * s).astype(np.float32)).astype(np.float32)
        want = np.concatenate([r0, r1], 1).reshape(1, KVD)
        assert np.array_equal(u32(O.rope(x, NKV, HD, pos, THETA)), u32(want))


def test_golden_rope(O):
    g = np.load(os.path.join(GOLDEN, "rope_cache.npz"))
    for t in range(len(g["row_pos"])):
        p = int(g["row_pos"][t])
        assert np.array_equal(u32(O.rope(g["q"][t], NH, HD, p, THETA)), u32(g["q_rot"][t]))
        assert np.array_equal(u32(O.rope(g["k"][t], NKV, HD, p, THETA)), u32(g["k_rot"][t]))


# ------------------------------------------------------ softmax, attention ----
@needs_ref
@pytest.mark.parametrize("n", [1, 2, 7, 512, 4097])
def test_softmax_matches_reference_build(O, n):
    x = normal(np.random.default_rng(n), (n,), 4.0)
    assert np.array_equal(u32(O.softmax(x)), u32(O.ref_softmax(x)))


@needs_ref
@pytest.mark.parametrize("T,pos0,nh,nkv,hd", [
    (1, 0, 14, 2, 64), (1, 511, 14, 2, 64), (7, 100, 14, 2, 64), (40, 500, 14, 2, 64),
    (3, 50, 8, 1, 128), (2, 20, 4, 2, 12), (2, 9, 2, 2, 5)])
def test_attention_matches_reference_build(O, T, pos0, nh, nkv, hd):
    rng = np.random.default_rng(T * 1000 + pos0)
    q = normal(rng, (T, nh * hd))
    k = normal(rng, (pos0 + T, nkv * hd))
    v = normal(rng, (pos0 + T, nkv * hd))
    want = O.ref_attention(q, k, v, pos0, nh, nkv, hd)
    assert np.array_equal(u32(O.attention(q, k, v, pos0, nh, nkv, hd)), u32(want))
    assert np.array_equal(u32(O.attention(q, k, v, pos0, nh, nkv, hd, threads=3)), u32(want))


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "attn_*.npz"))),
                         ids=lambda p: os.path.basename(p)[5:-4])
def test_golden_attention(O, path):
    g = np.load(path)
    tables, max_pages = g["tables"], g["tables"].shape[1]
    got = O.paged_attention(g["q"], g["k_pool_f16"], g["v_pool_f16"], O.KV_F16, g["row_pos"],
                            g["row_seq"], tables, max_pages, NH, NKV, HD)
    assert np.array_equal(u32(got), u32(g["out"]))


def test_attention_single_position_returns_v0(O):
    rng = np.random.default_rng(5)
    q, k, v = normal(rng, (1, QD)), normal(rng, (1, KVD)), normal(rng, (1, KVD))
    out = O.attention(q, k, v, 0, NH, NKV, HD).reshape(NH, HD)
    for h in range(NH):
        assert np.array_equal(u32(out[h]), u32(v.reshape(NKV, HD)[h // 7]))


def test_attention_constant_keys_average_values(O):
    rng = np.random.default_rng(6)
    L = 300
    q = normal(rng, (1, QD))
    k = np.repeat(normal(rng, (1, KVD)), L, 0)
    v = normal(rng, (L, KVD))
    out = O.attention(q, k, v, L - 1, NH, NKV, HD).reshape(NH, HD)
    mean = v.astype(np.float64).mean(0).reshape(NKV, HD)
    for h in range(NH):
        assert np.abs(out[h] - mean[h // 7]).max() < 1e-5


def test_attention_dominant_score_picks_its_value(O):
    rng = np.random.default_rng(7)
    L = 64
    q = normal(rng, (1, QD))
    k = normal(rng, (L, KVD)) * 0.01
    k[37] = np.tile(q.reshape(NH, HD)[[0, 7]].reshape(-1), 1) * 40.0  # huge score at position 37
    v = normal(rng, (L, KVD))
    out = O.attention(q, k, v, L - 1, NH, NKV, HD).reshape(NH, HD)
    assert np.abs(out[0] - v[37, :HD]).max() < 1e-6
    assert np.abs(out[7] - v[37, HD:]).max() < 1e-6


def test_attention_matches_fp64_brute_force(O):
    rng = np.random.default_rng(8)
    T, pos0 = 4, 30
    q = normal(rng, (T, QD))
    k = normal(rng, (pos0 + T, KVD))
    v = normal(rng, (pos0 + T, KVD))
    got = O.attention(q, k, v, pos0, NH, NKV, HD)
    qh = q.astype(np.float64).reshape(T, NH, HD)
    kh = k.astype(np.float64).reshape(-1, NKV, HD)
    vh = v.astype(np.float64).reshape(-1, NKV, HD)
    want = np.zeros((T, NH, HD))
    for t in range(T):
        p = pos0 + t
        for h in range(NH):
            s = kh[:p + 1, h // 7] @ qh[t, h] / 8.0
            w = np.exp(s - s.max())
            w /= w.sum()
            want[t, h] = w @ vh[:p + 1, h // 7]
    assert O.compare(got, want.reshape(T, QD).astype(np.float32))[0] < 2e-6
    # the GQA map h -> h // 7 matters: mapping h -> h % 2 is far off
    wrong = want.copy()
    for t in range(T):
        p = pos0 + t
        for h in range(NH):
            s = kh[:p + 1, h % 2] @ qh[t, h] / 8.0
            w = np.exp(s - s.max())
            wrong[t, h] = (w / w.sum()) @ vh[:p + 1, h % 2]
    assert O.compare(got, wrong.reshape(T, QD).astype(np.float32))[0] > 1e-2


# ------------------------------------------------------------ 16-bit ----
def _f32_sample(rng, n):
    """float32 bit patterns over every exponent, plus f16 ties and edge values."""
    b = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    x = b.view(np.float32)
    x = x[np.isfinite(x)]
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 5.96e-8, 2.98e-8, 2.9802322e-08,
                     6.1035156e-05, 6.097555e-05, 1.0 + 2**-11, 1.0 + 3 * 2**-11, -(1.0 + 2**-11),
                     2**-25, 2**-24 * 1.5, 2**-24 * 2.5, 1e30, -1e30], np.float32)
    # exact binary16 ties: an f16 value plus half an f16 ulp, at many scales
    base = (rng.standard_normal(4000) * 100).astype(np.float16).astype(np.float32)
    ulp = np.abs(np.spacing(base.astype(np.float16)).astype(np.float32))
    ties = (base + ulp / 2).astype(np.float32)
    small = (rng.standard_normal(20000) * 1e-4).astype(np.float32)  # subnormal f16 range
    return np.concatenate([x, edge, ties, small])


def test_f16_rounding_matches_numpy(O):
    x = _f32_sample(np.random.default_rng(9), 400000)
    want = x.astype(np.float16).view(np.uint16)
    got = O.round_to_kv(x, O.KV_F16)
    assert np.array_equal(got, want)
    back = O.widen_kv(got, O.KV_F16)
    assert np.array_equal(u32(back), u32(want.view(np.float16).astype(np.float32)))


def test_f16_widen_all_patterns(O):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.widen_kv(h, O.KV_F16)
    want = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(u32(got[fin]), u32(want[fin]))
    assert np.all(np.isnan(got[np.isnan(want)]))


def test_bf16_rounding_matches_torch(O):
    x = _f32_sample(np.random.default_rng(10), 400000)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.round_to_kv(x, O.KV_BF16), want)


def test_bf16_known_answers(O):
    # ties to even, and inf/NaN truncated (src/matrix.cpp:46-52)
    cases = {0x3F808000: 0x3F80, 0x3F818000: 0x3F82, 0x3F808001: 0x3F81, 0x7F800000: 0x7F80,
             0x7FC00001: 0x7FC0, 0xFF800000: 0xFF80, 0x7F7FFFFF: 0x7F80}
    x = np.array(list(cases), np.uint32).view(np.float32)
    assert list(O.round_to_kv(x, O.KV_BF16)) == list(cases.values())


# ------------------------------------------------------------ paging ----
def test_kv_offset_closed_form(O):
    rng = np.random.default_rng(11)
    tables, max_pages, _ = make_tables([40, 20, 70], rng)
    for s, n in enumerate([40, 20, 70]):
        for p in range(n):
            want = (int(tables[s, p >> 4]) * 16 + (p & 15)) * KVD
            assert O.kv_offset(tables, max_pages, 16, s, p, KVD) == want


def test_gather_invariant_under_page_permutation(O):
    """The same logical sequence stored under two page permutations gathers identically."""
    rng = np.random.default_rng(12)
    L = 77
    logical = normal(rng, (L, KVD))
    pages = (L + 15) // 16
    outs = []
    for seed in (1, 2):
        perm = np.random.default_rng(seed).permutation(pages + 5).astype(np.int32)[:pages]
        pool = normal(rng, ((pages + 5) * 16, KVD))
        for p in range(L):
            pool[perm[p >> 4] * 16 + (p & 15)] = logical[p]
        outs.append(O.gather_kv(pool, O.KV_F32, perm[None, :], pages, 0, L, KVD))
    assert np.array_equal(outs[0], logical) and np.array_equal(outs[1], logical)


def test_rope_append_paged_composition(O):
    """Page writes = per-row rope at the row's position, rounded, at kv_offset; rest untouched."""
    g = np.load(os.path.join(GOLDEN, "rope_cache.npz"))
    tables, max_pages, num_pages = g["tables"], g["tables"].shape[1], int(g["num_pages"])
    rng = np.random.default_rng(13)
    for kvt in (O.KV_F32, O.KV_F16, O.KV_BF16):
        kp = O.round_to_kv(normal(rng, (num_pages * 16, KVD)), kvt)
        vp = O.round_to_kv(normal(rng, (num_pages * 16, KVD)), kvt)
        q2, kp2, vp2 = O.rope_append_paged(g["q"], g["k"], g["v"], kp, vp, kvt, g["row_pos"],
                                           g["row_seq"], tables, max_pages, NH, NKV, HD, THETA)
        assert np.array_equal(u32(q2), u32(g["q_rot"]))
        want_k, want_v = kp.copy(), vp.copy()
        for t in range(len(g["row_pos"])):
            off = O.kv_offset(tables, max_pages, 16, int(g["row_seq"][t]), int(g["row_pos"][t]), KVD)
            want_k[off // KVD] = O.round_to_kv(g["k_rot"][t], kvt)
            want_v[off // KVD] = O.round_to_kv(g["v"][t], kvt)
        assert np.array_equal(kp2, want_k) and np.array_equal(vp2, want_v)


def test_gather_rows(O):
    rng = np.random.default_rng(14)
    x = normal(rng, (9, 896))
    rows = [8, 0, 3]
    assert np.array_equal(O.gather_rows(x, rows), x[rows])


def test_compare_metric(O):
    got = np.array([1.0, 2.5, -3.0], np.float32)
    want = np.array([1.0, 2.0, -4.0], np.float32)
    rel, mae, worst = O.compare(got, want)
    assert (rel, mae, worst) == (0.25, 1.0, 2)
    # The reference's NaN handling (src/npy.cpp:101-105): a NaN error replaces the maximum, but
    # any later element replaces a NaN maximum again, so only a trailing NaN survives. GPU
    # parity tests therefore also assert that outputs are finite.
    rel, _, worst = O.compare(np.array([0, np.nan], np.float32), np.array([0, 1], np.float32))
    assert np.isnan(rel) and worst == 1
    rel, _, worst = O.compare(np.array([np.nan, 0], np.float32), np.array([1, 0], np.float32))
    assert rel == 0.0 and worst == 1


def test_physical_cores(O):
    assert 1 <= O.physical_cores() <= os.cpu_count()
    if O.ref_available():
        assert O.physical_cores() == O.ref().ref_physical_cores()
