"""Writes the golden fixtures of the paged KV-cache path (tests/golden/*.npz).

Inputs are seeded N(0,1) tensors (numpy PCG64); expected outputs come from the
reference's OWN CPU code -- src/ops.cpp ie::rope / ie::attention compiled in
place by oracle/Makefile into oracle/_ref/libieref.so -- so the fixtures pin the
oracle restatement to the reference even where that build is absent.

The cases re-create the reference GPU self-test's paged cases
(src/cuda/cuda_runner.cu:849-1007) at fixture-friendly sizes:
  rope_cache.npz   lens {40, 20}; rows (0,20) (0,21) (1,3) (0,39); theta 1e6 (:849-874)
  attn_*.npz       first token; chunk edge 63; position 64; positions 255/256;
                   a prompt continuing at 40; whole prompts of 1 and 17 rows;
                   a prompt of the 2nd of 2 sequences; a batch of 5 decodes;
                   mixed prefill + decode (:914-941). The long-context case (3000)
                   is covered live, not as a fixture.
Pools are stored as float16 bit patterns (values are rounded to f16 first, so
the same pools serve the f32, f16 and bf16-widened checks exactly); the
expected outputs are float32.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import oracle as O  # noqa: E402
from helpers import HD, KVD, NH, NKV, QD, THETA, normal, make_tables  # noqa: E402

CASES = [
    # name, lens, rows [(seq, pos)]
    ("first_token", [1], [(0, 0)]),
    ("chunk_edge_63", [64], [(0, 63)]),
    ("position_64", [65], [(0, 64)]),
    ("position_255", [256], [(0, 255)]),
    ("position_256", [257], [(0, 256)]),
    ("prompt_continuing_40", [60], [(0, p) for p in range(40, 60)]),
    ("prompt_1", [1], [(0, 0)]),
    ("prompt_17", [17], [(0, p) for p in range(17)]),
    ("prompt_2nd_of_2", [30, 45], [(1, p) for p in range(45)]),
    ("batch_of_5", [6, 17, 64, 65, 300], [(0, 5), (1, 16), (2, 63), (3, 64), (4, 299)]),
    ("mixed_prefill_decode", [101, 30, 200], [(0, 100), (2, 199)] + [(1, p) for p in range(30)]),
]


def rope_case(rng):
    lens = [40, 20]
    rows = [(0, 20), (0, 21), (1, 3), (0, 39)]
    tables, max_pages, num_pages = make_tables(lens, rng)
    T = len(rows)
    q = normal(rng, (T, QD))
    k = normal(rng, (T, KVD))
    v = normal(rng, (T, KVD))
    q_rot = np.empty_like(q)
    k_rot = np.empty_like(k)
    for t, (s, p) in enumerate(rows):
        q_rot[t] = O.ref_rope(q[t], NH, HD, p, THETA)
        k_rot[t] = O.ref_rope(k[t], NKV, HD, p, THETA)
    np.savez(os.path.join(HERE, "rope_cache.npz"), lens=np.array(lens, np.int32),
             row_seq=np.array([r[0] for r in rows], np.int32),
             row_pos=np.array([r[1] for r in rows], np.int32), tables=tables,
             num_pages=np.int32(num_pages), q=q, k=k, v=v, q_rot=q_rot, k_rot=k_rot,
             theta=np.float32(THETA))


def attn_case(rng, name, lens, rows):
    tables, max_pages, num_pages = make_tables(lens, rng)
    kp = O.round_to_kv(normal(rng, (num_pages * 16, KVD)), O.KV_F16)
    vp = O.round_to_kv(normal(rng, (num_pages * 16, KVD)), O.KV_F16)
    T = len(rows)
    q = normal(rng, (T, QD))
    out = np.empty_like(q)
    kf = O.widen_kv(kp, O.KV_F16)
    vf = O.widen_kv(vp, O.KV_F16)
    for t, (s, p) in enumerate(rows):
        idx = [(tables[s, i // 16] * 16 + i % 16) for i in range(p + 1)]
        out[t] = O.ref_attention(q[t], kf[idx], vf[idx], p, NH, NKV, HD)
    np.savez(os.path.join(HERE, f"attn_{name}.npz"), lens=np.array(lens, np.int32),
             row_seq=np.array([r[0] for r in rows], np.int32),
             row_pos=np.array([r[1] for r in rows], np.int32), tables=tables,
             num_pages=np.int32(num_pages), k_pool_f16=kp, v_pool_f16=vp, q=q, out=out)


def main():
    if not O.ref_available():
        O.build()
    rng = np.random.default_rng(20261201)
    rope_case(rng)
    for name, lens, rows in CASES:
        attn_case(rng, name, lens, rows)
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
