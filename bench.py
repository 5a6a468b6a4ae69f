#!/usr/bin/env python3
"""Benchmark of the gfx950 paged KV-cache path on one MI355X.

Default workload (the headline metric): flash-decoding paged
attention, batch 64, ragged contexts L ~ U[128, 4096], GQA 14 query / 2 KV
heads, head_dim 64, f16 KV in 16-token pages, block tables a seeded permutation
of a 65,536-page pool, split-K partitions merged by log-sum-exp.

One step = one attention call over the whole batch, inputs resident in HBM.
Each step reads a different layer's pools (--layers, default 8 x 537 MB), so
the >= 2 x 256 MB working set defeats the 256 MB Infinity Cache and the rate
is HBM, not MALL. value = algorithmic bytes / time (GB/s):
    per row  512*L (K+V, f16) + 3584 (q) + 3584 (out) + 4*ceil(L/16) (page ids) + 8
Timing: the `steps` calls are recorded into one HIP graph, replayed at least 5 times
(and at least 100 calls in all), each replay between HIP events; the median replay
gives ms_per_step ("timing" in the line). The roofline fraction is against the
nominal 8 TB/s; its duration (us_per_launch) is the time per entry-point call, every
kernel the call launches (roofline.kernel) and the gaps between calls. The rocprofv3
kernel trace under profiles/ gives each kernel's own average.

The default line also carries:
  probe / ceiling_gbs  hand-written read kernels (llm-inference-engine_amd/probe): a 70 MB
                       and a 256 MB contiguous stream over rotated buffers, and the page
                       walk of this very batch with no arithmetic;
  plan_off             the same call with the work list located by the kernel, and
                       host_plan_build_us, the host's cost of the list per step;
  config2_append       the RoPE + paged append at 64 and 131,072 rows per launch, and a
                       device copy's read + write rate (its ceiling) from the same run;
  config4_decode       the long-context decode (24 layers, batch 1, 32k, bf16) per layer;
  config5_prefill      the 4,000-token prefill's MFMA fraction and the mixed step;
  cpu_baseline         the reference's own CPU attention (oracle/_ref: src/ops.cpp +
                       src/threadpool.cpp, -O3 -mavx2 -mfma) on the same batch, rows
                       gathered to contiguous fp32 first (timed apart), with the host's
                       physical core count and the threads used; its GB/s counts the
                       CPU's own fp32-cache bytes.

Other configs print the same JSON shape:
  --config 1  the reference's own CPU case (one layer, 512 positions, fp32), GPU and CPU
  --config 2  RoPE + paged append, 64 rows (+ --sweep: rows per launch up to 131,072)
  --config 4  long-context decode, 24 layers, batch 1, 32k context, bf16
  --config 5  mixed step: 48 decode rows + a 4,000-token prefill (MFMA), f16
  --config 6  the whole decode step: 24-layer Qwen2.5-0.5B-shaped decoder, batch 64, f16
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

NH, NKV, HD, THETA, PAGE = 14, 2, 64, 1e6, 16
QD, KVD = NH * HD, NKV * HD
HBM_PEAK_GBS = 8000.0
METRIC = "paged decode-attn HBM GB/s (% of 8 TB/s) + attn tok/s at batch 64, 1 GPU"
KV_CODES = {"f32": 0, "f16": 1, "bf16": 2}
KV_BYTES = {"f32": 4, "f16": 2, "bf16": 2}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def decode_bytes(lens, kv_bytes: int) -> int:
    """Algorithmic HBM bytes of one decode-attention launch: per row of context L, the K
    and V rows of its L positions, its query read and its output written (f32), one page
    id per page, and its position and sequence."""
    return int(sum(2 * KVD * kv_bytes * L + 2 * QD * 4 + 4 * math.ceil(L / PAGE) + 8 for L in lens))


def make_tables(rng, lens, num_pages, max_pages):
    perm = rng.permutation(num_pages).astype(np.int32)
    tables = np.zeros((len(lens), max_pages), np.int32)
    nxt = 0
    for s, n in enumerate(lens):
        k = (int(n) + PAGE - 1) // PAGE
        tables[s, :k] = perm[nxt:nxt + k]
        nxt += k
    return tables


def fill_pool(torch, n_rows, kv, gen, dev):
    dt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[kv]
    return torch.randn((n_rows, KVD), generator=gen, device=dev, dtype=dt)


EAGER = False  # --eager: launch every timed step from Python (for counter collection)


TIMING = {}  # how the last time_steps call was measured (reported in the JSON line)


def time_steps(torch, step, steps, warmup, stream):
    """Runs `warmup` eager steps, then times exactly `steps` steps, in ms per step.

    The timed steps are recorded once into a HIP graph and replayed: from Python each
    ctypes launch costs about as much host time as the kernels take on the GPU, so
    eager launches would measure the host. The library allocates and memsets nothing
    inside a call, so its launches record as plain kernel nodes. The graph is replayed
    once untimed, then at least 5 times (and at least 100 steps in all), each replay
    between two HIP events on the launch stream with a synchronize on both sides; the
    result is the median replay's time per step.
    """
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    replays = max(5, -(-100 // max(steps, 1)))
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    per_step = []
    if EAGER:
        for r in range(replays):
            torch.cuda.synchronize()
            start.record(stream)
            for i in range(steps):
                step(warmup + r * steps + i)
            end.record(stream)
            torch.cuda.synchronize()
            per_step.append(start.elapsed_time(end) / steps)
    else:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(steps):
                step(warmup + i)
        graph.replay()
        torch.cuda.synchronize()
        for _ in range(replays):
            torch.cuda.synchronize()
            start.record(stream)
            graph.replay()
            end.record(stream)
            torch.cuda.synchronize()
            per_step.append(start.elapsed_time(end) / steps)
    med = float(np.median(per_step))
    TIMING.clear()
    TIMING.update({"replays": replays, "steps_per_replay": steps, "launches": replays * steps,
                   "median_ms_per_step": round(med, 6),
                   "mean_ms_per_step": round(float(np.mean(per_step)), 6),
                   "min_ms_per_step": round(float(np.min(per_step)), 6),
                   "max_ms_per_step": round(float(np.max(per_step)), 6)})
    return med


def cpu_baseline_decode(O, lens, k_host, v_host, tables, kv, q_host, budget_s=10.0):
    """Reference CPU attention per row over a contiguous fp32 gather of its pages."""
    use_ref = O.ref_available()
    # The reference parallelises attention over the query heads only
    # (src/ops.cpp:78): more than n_heads threads would sit idle.
    cores = min(O.physical_cores(), NH)
    if use_ref:
        O.ref().ref_set_num_threads(cores)
    gather_s, attn_s, batches = [], [], 0
    t_start = time.perf_counter()
    while True:
        g_tot = a_tot = 0.0
        for r, L in enumerate(lens):
            t0 = time.perf_counter()
            idx = (tables[r, np.arange(L) // PAGE].astype(np.int64) * PAGE + np.arange(L) % PAGE)
            kc = np.ascontiguousarray(k_host[idx], np.float32)
            vc = np.ascontiguousarray(v_host[idx], np.float32)
            t1 = time.perf_counter()
            if use_ref:
                O.ref_attention(q_host[r], kc, vc, L - 1, NH, NKV, HD)
            else:
                O.attention(q_host[r], kc, vc, L - 1, NH, NKV, HD, threads=cores)
            t2 = time.perf_counter()
            g_tot += t1 - t0
            a_tot += t2 - t1
        gather_s.append(g_tot)
        attn_s.append(a_tot)
        batches += 1
        if time.perf_counter() - t_start >= budget_s:
            break
    t = float(np.median(attn_s))
    return {
        # The CPU's own algorithmic bytes: its cache is fp32 (4 bytes per element)
        # whatever the GPU pools hold.
        "value": round(decode_bytes(lens, 4) / t / 1e9, 3),
        "unit": "GB/s",
        "bytes": "fp32 cache (the CPU path has no 16-bit cache)",
        "cores": cores,
        "threads": cores,
        "physical_cores": O.physical_cores(),
        "kind": "reference" if use_ref else "port",
        "sample": (f"the full batch ({len(lens)} rows, same contexts), {batches} passes in "
                   f"{time.perf_counter() - t_start:.1f} s; median attention time per batch "
                   f"{t * 1e3:.1f} ms; per-row gather to contiguous fp32 (excluded) "
                   f"{float(np.median(gather_s)) * 1e3:.1f} ms"),
        "attn_tok_per_s": round(len(lens) / t, 1),
    }


def _cpu_threads(O):
    cores = min(O.physical_cores(), NH)  # the reference splits attention over heads only
    if O.ref_available():
        O.ref().ref_set_num_threads(cores)
    return cores


def _ref_attention(O, q, k, v, pos0, cores):
    if O.ref_available():
        return O.ref_attention(q, k, v, pos0, NH, NKV, HD)
    return O.attention(q, k, v, pos0, NH, NKV, HD, threads=cores)


def cpu_baseline_append(O, q, k, v, pos, kv, budget_s=3.0):
    """Config 2 on the CPU: RoPE of q and k and the paged K/V write for the 64 rows, the
    oracle's restatement of the reference's rope + append (src/ops.cpp:34-55,
    src/model.cpp:70-75) in one C call per batch, into a compact pool holding the
    rows' pages (the write pattern is the same)."""
    T = len(pos)
    pos = np.ascontiguousarray(pos, np.int32)
    pi = pos.astype(np.int64) // PAGE
    max_pages = int(pi.max()) + 1
    tables = np.zeros((T, max_pages), np.int32)
    tables[np.arange(T), pi] = np.arange(T)  # row t's page is page t of the compact pool
    seqs = np.arange(T, dtype=np.int32)
    kvn = O.KV_NP[KV_CODES[kv]]
    kp = np.zeros((T * PAGE, KVD), kvn)
    vp = np.zeros((T * PAGE, KVD), kvn)
    lib = O.orc()
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    times, t_start = [], time.perf_counter()
    while True:
        qq = np.ascontiguousarray(q, np.float32).copy()
        t0 = time.perf_counter()
        lib.orc_rope_append_paged(ptr(qq), ptr(k), ptr(v), ptr(kp), ptr(vp), KV_CODES[kv], T,
                                  ptr(pos), ptr(seqs), ptr(tables), max_pages, PAGE, NH, NKV, HD,
                                  ctypes.c_float(THETA))
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start >= budget_s:
            break
    t = float(np.median(times))
    per_row = 1024 + 2 * KVD * KV_BYTES[kv] + 8 + 4 + 2 * QD * 4
    return {"value": round(T * per_row / t / 1e9, 3), "unit": "GB/s", "cores": 1, "threads": 1,
            "physical_cores": O.physical_cores(), "kind": "port",
            "sample": f"the 64 rows with q, {len(times)} batches; median {t * 1e6:.1f} us per batch "
                      f"(oracle/oracle.cpp, single thread, as the reference's rope runs)",
            "us_per_launch": round(t * 1e6, 2)}


def cpu_baseline_long(O, k_pools, v_pools, tabs, q, L, kv, layers, budget_s=8.0):
    """Config 4 on the CPU: per layer, the 32k-position row gathered to contiguous fp32
    (the self-test method, src/cuda/cuda_runner.cu:959-965; timed apart) and the
    reference's attention over it, on as many layers as the budget allows; the step
    time is the median layer time x 24."""
    cores = _cpu_threads(O)
    attn, gath, t_start, n = [], [], time.perf_counter(), 0
    while True:
        l = n % len(k_pools)
        t0 = time.perf_counter()
        idx = tabs[l][0, np.arange(L) // PAGE].astype(np.int64) * PAGE + np.arange(L) % PAGE
        kc = O.widen_kv(k_pools[l][idx], KV_CODES[kv]) if kv != "f32" else k_pools[l][idx]
        vc = O.widen_kv(v_pools[l][idx], KV_CODES[kv]) if kv != "f32" else v_pools[l][idx]
        t1 = time.perf_counter()
        _ref_attention(O, q[l], kc, vc, L - 1, cores)
        attn.append(time.perf_counter() - t1)
        gath.append(t1 - t0)
        n += 1
        if time.perf_counter() - t_start >= budget_s and n >= 2:
            break
    t = float(np.median(attn)) * layers
    per_layer = 2 * KVD * 4 * L + 2 * QD * 4 + 4 * (L // PAGE) + 8  # fp32 cache bytes
    return {"value": round(layers * per_layer / t / 1e9, 3), "unit": "GB/s", "cores": cores,
            "bytes": "fp32 cache (the CPU path has no 16-bit cache)",
            "threads": cores, "physical_cores": O.physical_cores(),
            "kind": "reference" if O.ref_available() else "port",
            "sample": f"{n} layers' attention over 32,768 positions (gather to contiguous fp32 "
                      f"excluded, median {float(np.median(gath)) * 1e3:.1f} ms); step = median "
                      f"layer x {layers}",
            "ms_per_step": round(t * 1e3, 2), "tok_per_s": round(1 / t, 2)}


def cpu_baseline_model(O, layer_bits, norms, embed_bits, x, kc, vc, pos, layers, reps=3):
    """Config 6 on the CPU with the reference's own code (oracle/_ref: src/matrix.cpp AVX2
    matmul, src/ops.cpp rmsnorm and attention, its thread pool): one layer's dense work for
    the 64 rows (rmsnorm, q/k/v, o_proj, rmsnorm, gate/up, SiLU in numpy, down; median of
    `reps`), the attention of a sample of rows over their contexts (gathered to contiguous
    fp32 beforehand) scaled to all 64, both x 24 layers, plus the LM head once."""
    import ctypes
    cores = _cpu_threads(O)
    R = O.ref()
    R.ref_matrix_create.restype = ctypes.c_void_p
    R.ref_matrix_create.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    R.ref_matrix_destroy.argtypes = [ctypes.c_void_p]
    R.ref_matrix_matmul.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int]
    mats = {n: (R.ref_matrix_create(w.ctypes.data, 1, w.shape[0], w.shape[1]), w.shape[0])
            for n, w in layer_bits.items()}
    B, H = x.shape
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    q_rows = np.random.default_rng(1).standard_normal((len(kc), QD), dtype=np.float32)

    def mm(name, inp):
        m, rows = mats[name]
        y = np.empty((B, rows), np.float32)
        R.ref_matrix_matmul(ptr(y), ptr(inp), ctypes.c_void_p(m), None, B)
        return y

    dense = []
    for _ in range(reps):
        t0 = time.perf_counter()
        xn = O.ref_rmsnorm(x, norms[0], 1e-6)
        mm("q", xn), mm("k", xn), mm("v", xn)
        x2 = x + mm("o", np.ascontiguousarray(xn))
        xn = O.ref_rmsnorm(x2, norms[1], 1e-6)
        g, u = mm("g", xn), mm("u", xn)
        mid = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
        mm("d", mid)
        dense.append(time.perf_counter() - t0)
    attn = []
    for i in range(len(kc)):
        t0 = time.perf_counter()
        _ref_attention(O, np.ascontiguousarray(q_rows[i:i + 1]), kc[i], vc[i], int(pos[i]), cores)
        attn.append(time.perf_counter() - t0)
    lm = R.ref_matrix_create(embed_bits.ctypes.data, 1, embed_bits.shape[0], embed_bits.shape[1])
    y = np.empty((B, embed_bits.shape[0]), np.float32)
    t0 = time.perf_counter()
    R.ref_matrix_matmul(ptr(y), ptr(x), ctypes.c_void_p(lm), None, B)
    t_lm = time.perf_counter() - t0
    R.ref_matrix_destroy(ctypes.c_void_p(lm))
    for m, _ in mats.values():
        R.ref_matrix_destroy(ctypes.c_void_p(m))
    t_layer = float(np.median(dense)) + float(np.mean(attn)) * B
    t = layers * t_layer + t_lm
    return {"value": round(B / t, 2), "unit": "tok/s", "cores": cores, "threads": cores,
            "physical_cores": O.physical_cores(),
            "kind": "reference" if O.ref_available() else "port",
            "sample": f"one layer's dense ops for {B} rows (median of {reps}: "
                      f"{float(np.median(dense)) * 1e3:.1f} ms), attention of {len(kc)} rows "
                      f"(mean {float(np.mean(attn)) * 1e3:.2f} ms per row, x {B}), the LM head "
                      f"once ({t_lm * 1e3:.0f} ms); step = {layers} layers + LM head",
            "ms_per_step": round(t * 1e3, 1)}


def cpu_baseline_mixed(O, pq_h, kc_pf, vc_pf, P, dq_h, dec_kv, budget_s=10.0):
    """Config 5 on the CPU: the reference's attention for the prompt's last rows (scaled
    to all 4,000 rows by their causal flop count) and for the 48 decode rows over
    their gathered contexts."""
    cores = _cpu_threads(O)
    sub = 400  # prompt rows timed: positions P - sub .. P - 1
    pf, dc, t_start = [], [], time.perf_counter()
    while True:
        t0 = time.perf_counter()
        _ref_attention(O, pq_h[P - sub:], kc_pf, vc_pf, P - sub, cores)
        t1 = time.perf_counter()
        for r, (kc, vc) in enumerate(dec_kv):
            _ref_attention(O, dq_h[r], kc, vc, len(kc) - 1, cores)
        t2 = time.perf_counter()
        pf.append(t1 - t0)
        dc.append(t2 - t1)
        if time.perf_counter() - t_start >= budget_s:
            break
    flops_sub = 4 * NH * HD * sum(p + 1 for p in range(P - sub, P))
    flops_all = 4 * NH * HD * P * (P + 1) // 2
    t_pf = float(np.median(pf)) * flops_all / flops_sub
    t = t_pf + float(np.median(dc))
    return {"value": round((len(dec_kv) + P) / t, 1), "unit": "rows/s", "cores": cores,
            "threads": cores, "physical_cores": O.physical_cores(),
            "kind": "reference" if O.ref_available() else "port",
            "sample": f"prompt rows {P - sub}..{P - 1} ({len(pf)} passes, scaled to the 4,000-row "
                      f"prefill by causal flops) + the 48 decode rows; gathers excluded",
            "prefill_s": round(t_pf, 4), "prefill_tflops": round(flops_all / t_pf / 1e12, 4),
            "decode_ms": round(float(np.median(dc)) * 1e3, 3)}


def bench_decode(args, torch, ie, O):
    dev = torch.device("cuda:0")
    kv = args.kv or "f16"
    rng = np.random.default_rng(args.seed)
    B, num_pages = 64, 65536
    lens = rng.integers(128, 4097, B)
    max_pages = 4096 // PAGE
    tables = make_tables(rng, lens, num_pages, max_pages)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    log(f"config 3: seed {args.seed}, {args.layers} layers x 2 x {num_pages} pages of {kv}")
    k_pools = [fill_pool(torch, num_pages * PAGE, kv, gen, dev) for _ in range(args.layers)]
    v_pools = [fill_pool(torch, num_pages * PAGE, kv, gen, dev) for _ in range(args.layers)]
    q = torch.randn((B, QD), generator=gen, device=dev, dtype=torch.float32)
    out = torch.empty((B, QD), device=dev, dtype=torch.float32)
    d_tab = torch.from_numpy(tables).to(dev)
    d_pos = torch.from_numpy((lens - 1).astype(np.int32)).to(dev)
    d_seq = torch.arange(B, dtype=torch.int32, device=dev)
    ct = args.chunk_tokens or ie.attention_chunk_tokens(B, 4096, KV_CODES[kv])
    nc = ie.attention_chunks(4096, ct)
    ws = ie.attention_workspace(B, NH, HD, nc)
    stream = torch.cuda.current_stream()
    # The work list the engine builds on the host for a decode step (the rows'
    # positions and sequences and the block table are host data there): one
    # dependent load before the first K/V byte instead of three. The positions are
    # fixed across steps here, so it is built and copied once.
    d_plan = None
    if args.plan == "on":
        d_plan = torch.from_numpy(ie.attention_plan((lens - 1).astype(np.int32),
                                                    np.arange(B, dtype=np.int32), tables, nc,
                                                    ct)).to(dev)

    def step(i):
        l = i % args.layers
        if d_plan is not None:
            ie.attention_planned(out, q, k_pools[l], v_pools[l], d_pos, d_seq, d_tab, max_pages,
                                 nc, ct, ws, d_plan, NH, NKV, HD)
        else:
            ie.attention(out, q, k_pools[l], v_pools[l], d_pos, d_seq, d_tab, max_pages, nc, ct,
                         ws, NH, NKV, HD)

    ms = time_steps(torch, step, args.steps, args.warmup, stream)
    timing = dict(TIMING)
    nbytes = decode_bytes(lens, KV_BYTES[kv])
    gbs = nbytes / (ms * 1e-3) / 1e9
    plan_extra = {}
    if d_plan is not None:
        # The same call with the work list located by the kernel instead (no host list),
        # and what building the list costs the host per step: ie_hip_attention_plan over
        # host arrays, called through ctypes (its call overhead included).
        def step_unplanned(i):
            l = i % args.layers
            ie.attention(out, q, k_pools[l], v_pools[l], d_pos, d_seq, d_tab, max_pages, nc,
                         ct, ws, NH, NKV, HD)

        ms_off = time_steps(torch, step_unplanned, args.steps, args.warmup, stream)
        pos_h = np.ascontiguousarray(lens - 1, np.int32)
        seq_h = np.arange(B, dtype=np.int32)
        tab_h = np.ascontiguousarray(tables, np.int32)
        n_plan = int(ie.lib().ie_hip_attention_plan_ints(B, nc, ct))
        plan_h = np.zeros(n_plan, np.int32)
        ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
        builds = []
        for _ in range(7):
            t0 = time.perf_counter()
            for _ in range(200):
                ie.lib().ie_hip_attention_plan(ptr(plan_h), n_plan, B, ptr(pos_h), ptr(seq_h),
                                               ptr(tab_h), B, max_pages, nc, ct)
            builds.append((time.perf_counter() - t0) / 200)
        gbs_off = nbytes / (ms_off * 1e-3) / 1e9
        plan_extra = {"plan_off": {"ms_per_step": round(ms_off, 5), "gbs": round(gbs_off, 2),
                                   "frac": round(gbs_off / HBM_PEAK_GBS, 4),
                                   "note": "ie_hip_attention: the kernel locates each "
                                           "workgroup's (row, chunk) and page ids itself"},
                      "host_plan_build_us": round(float(np.median(builds)) * 1e6, 2)}

    # Warm, for reference only: the same call repeated on one layer's pools, so the
    # pages it reads (70 MB) stay in the 256 MB Infinity Cache (MALL) between calls.
    def step_warm(i):
        ie.attention(out, q, k_pools[0], v_pools[0], d_pos, d_seq, d_tab, max_pages, nc, ct, ws,
                     NH, NKV, HD)

    ms_warm = time_steps(torch, step_warm, args.steps, args.warmup, stream)
    res = {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": kv,
        "data": "synthetic",
        "config": {"workload": "config 3: flash-decoding paged attention, batch 64, "
                               "L~U[128,4096], GQA 14q/2kv, head_dim 64, 16-token pages, "
                               f"65,536-page pools, {ct}-token split-K + LSE merge",
                   "kv_dtype": kv, "batch": B, "chunk_tokens": ct, "num_chunks": nc,
                   "layers_rotated": args.layers, "seed": args.seed,
                   "context_tokens": int(lens.sum()),
                   "work_list": "host-built (ie_hip_attention_plan)" if d_plan is not None
                   else "located on the device"},
        "attn_tok_per_s": round(B / (ms * 1e-3), 1),
        "context_tok_per_s": round(float(lens.sum()) / (ms * 1e-3), 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles("decode", kv, "f16", args),
                     "kernel": ("decode_partial_mfma_f32" if kv == "f32" else "decode_partial_mfma")
                               + " + decode_merge_kernel (one ie_hip_attention"
                               + ("_planned" if d_plan is not None else "") + " call)",
                     "us_per_launch": round(ms * 1e3, 3)},
        "algorithmic_bytes_per_step": nbytes,
        "timing": timing,
        **plan_extra,
        "warm_mall": {"ms_per_step": round(ms_warm, 5),
                      "gbs": round(nbytes / (ms_warm * 1e-3) / 1e9, 2),
                      "note": "one layer's pools repeated: pages resident in the Infinity Cache; "
                              "not the metric"},
    }
    if not args.no_probe:
        probe = hbm_probes(args, torch, stream, k_pools, v_pools, d_tab, lens, max_pages, ct, kv)
        if probe:
            res["probe"] = probe
            res["ceiling_gbs"] = probe["ceiling_gbs"]
            res["frac_of_ceiling"] = round(gbs / probe["ceiling_gbs"], 4)
    if not args.no_cpu:
        kh = O.widen_kv(k_pools[0].cpu().view(torch.int16).numpy().view(np.uint16), KV_CODES[kv]) \
            if kv != "f32" else k_pools[0].cpu().numpy()
        vh = O.widen_kv(v_pools[0].cpu().view(torch.int16).numpy().view(np.uint16), KV_CODES[kv]) \
            if kv != "f32" else v_pools[0].cpu().numpy()
        res["cpu_baseline"] = cpu_baseline_decode(O, [int(x) for x in lens], kh, vh, tables, kv,
                                                  q.cpu().numpy(), args.cpu_seconds)
    return res


def bench_append(args, torch, ie, O):
    """Config 2: fused RoPE + paged append, 64 rows; plus a rows-per-launch sweep."""
    dev = torch.device("cuda:0")
    kv = args.kv or "f16"
    rng = np.random.default_rng(args.seed)
    num_pages, max_pos = 65536, 4096
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    k_pool = fill_pool(torch, num_pages * PAGE, kv, gen, dev)
    v_pool = fill_pool(torch, num_pages * PAGE, kv, gen, dev)
    table = ie.rope_table(max_pos, HD, THETA).to(dev)
    stream = torch.cuda.current_stream()
    sweep = []
    rows_list = getattr(args, "append_rows", None) or \
        ([64] + ([256, 1024, 4096, 16384, 65536, 131072] if args.sweep else []))
    for rows in rows_list:
        seqs = max(1, rows // 64)
        max_pages = num_pages // seqs
        tables = rng.permutation(num_pages)[:seqs * max_pages].astype(np.int32).reshape(seqs, -1)
        pos = rng.integers(1, min(max_pos, max_pages * PAGE), rows).astype(np.int32)
        d_tab = torch.from_numpy(tables).to(dev)
        d_pos = torch.from_numpy(pos).to(dev)
        d_seq = torch.from_numpy((np.arange(rows) % seqs).astype(np.int32)).to(dev)
        q = torch.randn((rows, QD), generator=gen, device=dev)
        k = torch.randn((rows, KVD), generator=gen, device=dev)
        v = torch.randn((rows, KVD), generator=gen, device=dev)
        if rows == 64:
            cpu_in = (q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), pos.copy())
        modes = {"off": (False,), "on": (True,), "both": (False, True)}[args.append_q]
        for with_q in modes:
            def step(i):
                ie.rope_and_cache(q if with_q else None, k, v, k_pool, v_pool, table, d_pos, d_seq,
                                  d_tab, max_pages, NH, NKV, HD)
            ms = time_steps(torch, step, args.steps, args.warmup, stream)
            per_row = (1024 + 2 * KVD * KV_BYTES[kv] + 8 + 4) + (2 * QD * 4 if with_q else 0)
            sweep.append({"rows": rows, "with_q": with_q, "us_per_launch": round(ms * 1e3, 3),
                          "gbs": round(rows * per_row / (ms * 1e-3) / 1e9, 2)})
    mode = [s for s in sweep if s["with_q"] == (args.append_q == "on")] or sweep
    head = ([s for s in mode if s["rows"] == 64] or mode)[0]
    res = {
        "metric": "paged RoPE+KV append GB/s at batch 64 (K/V only), 1 GPU",
        "value": head["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(head["us_per_launch"] / 1e3, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "config 2: RoPE + paged KV append, 64 rows, pos~U[1,4096), "
                               "65,536-page pool", "kv_dtype": kv, "seed": args.seed},
        "roofline": {"bound": "hbm", "achieved": head["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / HBM_PEAK_GBS, 5),
                     "traffic": traffic_from_profiles("append", kv, "f16", args),
                     "kernel": "rope_append_kernel (one ie_hip_rope_and_cache call)",
                     "us_per_launch": head["us_per_launch"]},
        "sweep": sweep,
    }
    if not args.no_cpu and 64 in rows_list:
        res["cpu_baseline"] = cpu_baseline_append(O, *cpu_in, kv)
    return res


def bench_long(args, torch, ie, O):
    """Config 4: long-context decode, all 24 layers. Batch 1, context 32,768, bf16 KV in
    shuffled 16-token pages (one pool per layer), per layer a RoPE + append at position
    32,767 then attention over the 32,768 positions."""
    dev = torch.device("cuda:0")
    kv = args.kv or "bf16"
    rng = np.random.default_rng(args.seed)
    layers, L = 24, 32768
    pages = L // PAGE
    num_pages = 2 * pages  # half of each pool unused, so the row's pages are scattered
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    k_pools = [fill_pool(torch, num_pages * PAGE, kv, gen, dev) for _ in range(layers)]
    v_pools = [fill_pool(torch, num_pages * PAGE, kv, gen, dev) for _ in range(layers)]
    tabs = [torch.from_numpy(rng.permutation(num_pages)[:pages].astype(np.int32)[None, :]).to(dev)
            for _ in range(layers)]
    table = ie.rope_table(L, HD, THETA).to(dev)
    q = torch.randn((layers, 1, QD), generator=gen, device=dev)
    k = torch.randn((layers, 1, KVD), generator=gen, device=dev)
    v = torch.randn((layers, 1, KVD), generator=gen, device=dev)
    out = torch.empty((1, QD), device=dev)
    d_pos = torch.tensor([L - 1], dtype=torch.int32, device=dev)
    d_seq = torch.zeros(1, dtype=torch.int32, device=dev)
    ct = args.chunk_tokens or ie.attention_chunk_tokens(1, L, KV_CODES[kv])
    nc = ie.attention_chunks(L, ct)
    ws = ie.attention_workspace(1, NH, HD, nc)
    stream = torch.cuda.current_stream()

    # The layer's RoPE + append and attention in one launch where the library offers it
    # (16-bit caches at the matrix-core kernel's shapes), else the two calls.
    fused = not args.unfused and ie.rope_cache_attention_supported(KV_CODES[kv], NH, NKV, HD, ct)
    # Host-built work lists, one per layer (each layer's table differs), as the engine
    # builds them for a decode step.
    plans = None
    if args.plan == "on":
        plans = [torch.from_numpy(ie.attention_plan(np.array([L - 1], np.int32),
                                                    np.zeros(1, np.int32), tabs[l].cpu().numpy(),
                                                    nc, ct)).to(dev) for l in range(layers)]

    def step(i):
        for l in range(layers):
            if fused and plans is not None:
                ie.rope_cache_attention_planned(out, q[l], k[l], v[l], k_pools[l], v_pools[l],
                                                table, d_pos, d_seq, tabs[l], pages, nc, ct, ws,
                                                plans[l], NH, NKV, HD)
                continue
            if fused:
                ie.rope_cache_attention(out, q[l], k[l], v[l], k_pools[l], v_pools[l], table,
                                        d_pos, d_seq, tabs[l], pages, nc, ct, ws, NH, NKV, HD)
                continue
            ie.rope_and_cache(q[l], k[l], v[l], k_pools[l], v_pools[l], table, d_pos, d_seq,
                              tabs[l], pages, NH, NKV, HD)
            if plans is not None:
                ie.attention_planned(out, q[l], k_pools[l], v_pools[l], d_pos, d_seq, tabs[l],
                                     pages, nc, ct, ws, plans[l], NH, NKV, HD)
            else:
                ie.attention(out, q[l], k_pools[l], v_pools[l], d_pos, d_seq, tabs[l], pages, nc,
                             ct, ws, NH, NKV, HD)

    ms = time_steps(torch, step, args.steps, args.warmup, stream)
    per_layer = 2 * KVD * KV_BYTES[kv] * L + 2 * QD * 4 + 4 * pages + 8 + \
        (1024 + 2 * KVD * KV_BYTES[kv] + 12 + 2 * QD * 4)
    nbytes = layers * per_layer
    gbs = nbytes / (ms * 1e-3) / 1e9
    res = {
        "metric": "long-context decode step (24 layers, batch 1, 32k context) GB/s, 1 GPU",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": kv, "data": "synthetic",
        "config": {"workload": "config 4: 24 layers x (RoPE+append at 32,767, flash-decoding "
                               "over 32,768 positions), batch 1, shuffled 16-token pages",
                   "kv_dtype": kv, "chunk_tokens": ct, "num_chunks": nc, "seed": args.seed,
                   "layer_calls": ("rope_cache_attention" if fused
                                   else "rope_and_cache + attention")
                   + ("_planned" if plans is not None else ""),
                   "work_list": "host-built (ie_hip_attention_plan)" if plans is not None
                   else "located on the device"},
        "tok_per_s": round(1 / (ms * 1e-3), 1), "us_per_layer": round(ms * 1e3 / layers, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles("long" if fused else "long_unfused",
                                                      kv, "bf16", args),
                     "kernel": "24 x (decode_partial_mfma + decode_merge_kernel)" if fused
                               else "24 x (rope_append_kernel + decode_partial_mfma + "
                                    "decode_merge_kernel)",
                     "us_per_launch": round(ms * 1e3, 3)},
        "algorithmic_bytes_per_step": nbytes,
    }
    if not args.no_cpu:
        n_cpu = 3  # layers copied to the host for the CPU sample
        host = lambda t: (t.cpu().numpy() if kv == "f32" else
                          t.cpu().view(torch.int16).numpy().view(np.uint16))
        res["cpu_baseline"] = cpu_baseline_long(
            O, [host(k_pools[l]) for l in range(n_cpu)], [host(v_pools[l]) for l in range(n_cpu)],
            [tabs[l].cpu().numpy() for l in range(n_cpu)], [q[l].cpu().numpy() for l in range(n_cpu)],
            L, kv, layers)
    return res


def bench_mixed(args, torch, ie, O):
    """Config 5: one mixed serving step of one layer -- 48 decode rows (contexts
    U[256, 2048]) plus a 4,000-token chunked prefill written into fresh pages of a pool
    whose pages were churned (25% freed and re-allocated) first; f16 KV."""
    dev = torch.device("cuda:0")
    kv = args.kv or "f16"
    rng = np.random.default_rng(args.seed)
    num_pages, max_seq, n_dec, P = 65536, 8192, 48, 4000
    pool = ie.PagePool(num_pages, 64, max_seq)
    seqs = [pool.open_sequence() for _ in range(64)]
    lens = {s: int(rng.integers(256, 2049)) for s in seqs}
    for s in seqs:
        pool.ensure(s, lens[s])
    for s in rng.permutation(seqs)[:16]:  # 25% of the sequences finish: their pages go back
        pool.close_sequence(int(s))
        del lens[int(s)]
    dec = sorted(lens)[:n_dec]
    pf = pool.open_sequence()
    pool.ensure(pf, P)  # fresh pages for the prompt, most of them the freed ones
    for s in dec:       # each decode row appends its next token
        pool.ensure(s, lens[s] + 1)
    max_pages = pool.max_pages_per_seq
    d_tab = torch.zeros(pool.max_batch * max_pages, dtype=torch.int32, device=dev)
    pool.upload_tables(d_tab)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    k_pool = fill_pool(torch, num_pages * PAGE, kv, gen, dev)
    v_pool = fill_pool(torch, num_pages * PAGE, kv, gen, dev)
    table = ie.rope_table(max_seq, HD, THETA).to(dev)
    pq, pk, pv = (torch.randn((P, d), generator=gen, device=dev) for d in (QD, KVD, KVD))
    dq, dk, dv = (torch.randn((n_dec, d), generator=gen, device=dev) for d in (QD, KVD, KVD))
    p_pos = torch.arange(P, dtype=torch.int32, device=dev)
    p_seq = torch.full((P,), pf, dtype=torch.int32, device=dev)
    d_pos = torch.tensor([lens[s] for s in dec], dtype=torch.int32, device=dev)
    d_seq = torch.tensor(dec, dtype=torch.int32, device=dev)
    p_out = torch.empty((P, QD), device=dev)
    d_out = torch.empty((n_dec, QD), device=dev)
    ct = args.chunk_tokens or ie.attention_chunk_tokens(n_dec, 2049, KV_CODES[kv])
    nc = ie.attention_chunks(2049, ct)
    ws = ie.attention_workspace(n_dec, NH, HD, nc)
    stream = torch.cuda.current_stream()

    # The prompt as the engine's prompt step runs it (KvEngine::run): K/V appended, q
    # rotated inside the prefill kernel (ie_hip_rope_cache_attention_prefill), where the
    # library offers that; else the two calls (append rotating q in place, then prefill).
    pf_fused = ie.rope_cache_attention_prefill_supported(KV_CODES[kv], NH, NKV, HD)

    def prefill_two_calls(i):
        ie.rope_and_cache(pq, pk, pv, k_pool, v_pool, table, p_pos, p_seq, d_tab, max_pages,
                          NH, NKV, HD)
        ie.attention_prefill(p_out, pq, k_pool, v_pool, p_pos, p_seq, d_tab, max_pages, NH, NKV,
                             HD)

    def prefill(i):
        if not pf_fused:
            prefill_two_calls(i)
            return
        ie.rope_cache_attention_prefill(p_out, pq, pk, pv, k_pool, v_pool, table, p_pos, p_seq,
                                        d_tab, max_pages, NH, NKV, HD)

    def prefill_attn(i):
        ie.attention_prefill(p_out, pq, k_pool, v_pool, p_pos, p_seq, d_tab, max_pages, NH, NKV,
                             HD)

    # The decode rows as the engine's decode step runs them (KvEngine::run): RoPE +
    # append folded into the attention launch, reading a host-built work list, where the
    # library offers that (16-bit caches); else the two calls. The list is built once
    # (the positions do not change between steps; the engine builds it every step, its
    # host cost is the config-3 line's host_plan_build_us).
    fused = ie.rope_cache_attention_supported(KV_CODES[kv], NH, NKV, HD, ct)
    d_plan = None
    if fused:
        d_plan = torch.from_numpy(ie.attention_plan(
            d_pos.cpu().numpy(), d_seq.cpu().numpy(),
            d_tab.cpu().numpy().reshape(pool.max_batch, max_pages), nc, ct)).to(dev)

    def decode_two_calls(i):
        ie.rope_and_cache(dq, dk, dv, k_pool, v_pool, table, d_pos, d_seq, d_tab, max_pages,
                          NH, NKV, HD)
        ie.attention(d_out, dq, k_pool, v_pool, d_pos, d_seq, d_tab, max_pages, nc, ct, ws, NH,
                     NKV, HD)

    def decode(i):
        if not fused:
            decode_two_calls(i)
            return
        ie.rope_cache_attention_planned(d_out, dq, dk, dv, k_pool, v_pool, table, d_pos, d_seq,
                                        d_tab, max_pages, nc, ct, ws, d_plan, NH, NKV, HD)

    # The step as the engine runs it: one stream, the prefill then the decode rows
    # (step_serial, the reported ms_per_step). Beside it, a composition bound: the
    # prompt and the decode rows touch different sequences (different pages), so the
    # decode half can run on a second stream (default priority), forked from and
    # joined back into the launch stream -- two parallel branches of one graph, the
    # decode rows' short kernels filling the compute units the prefill's one
    # workgroup per unit leaves idle. No engine path schedules a step that way.
    side = torch.cuda.Stream(device=dev)

    def step(i):
        cur = torch.cuda.current_stream()
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            decode(i)
        prefill(i)
        cur.wait_stream(side)

    def step_serial(i):
        prefill(i)
        decode(i)

    ms_branches = time_steps(torch, step, args.steps, args.warmup, stream)
    ms = time_steps(torch, step_serial, args.steps, args.warmup, stream)
    ms_pf = time_steps(torch, prefill_attn, args.steps, args.warmup, stream)
    ms_dec = time_steps(torch, decode, args.steps, args.warmup, stream)
    ms_pfp = time_steps(torch, prefill, args.steps, args.warmup, stream)
    ms_pfp2 = (time_steps(torch, prefill_two_calls, args.steps, args.warmup, stream) if pf_fused
               else ms_pfp)
    ms_dec2 = time_steps(torch, decode_two_calls, args.steps, args.warmup, stream) if fused else ms_dec
    flops = 4 * NH * HD * P * (P + 1) // 2
    # Dense matrix peak of the type the prefill tiles run in: the 16-bit MFMA for
    # f16/bf16 caches, the fp32 MFMA for f32 caches (MI355X published figures).
    mfma_peak = 157.3 if kv == "f32" else 2500.0
    tflops = flops / (ms_pf * 1e-3) / 1e12
    dec_bytes = decode_bytes([lens[s] + 1 for s in dec], KV_BYTES[kv])
    res = {
        "metric": "mixed serving step (48 decode rows + 4,000-token prefill, one layer), 1 GPU",
        "value": round((n_dec + P) / (ms * 1e-3), 1), "unit": "rows/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": kv,
        "data": "synthetic",
        "config": {"workload": "config 5: 48 decode rows (L~U[256,2048]) + one 4,000-token "
                               "prefill into fresh pages after 25% page churn, one layer",
                   "kv_dtype": kv, "chunk_tokens": ct, "seed": args.seed},
        "step": "one stream: the prompt's append + prefill, then the decode rows (the engine's "
                "order and calls)",
        "ms_per_step_two_branches": round(ms_branches, 5),
        "two_branches_note": "a kernel-composition bound, not an engine path: the decode "
                             "half on a parallel graph branch beside the prefill",
        "prefill_attention_ms": round(ms_pf, 5),
        "prefill_tflops": round(tflops, 2),
        "prefill_part_ms": round(ms_pfp, 5),
        "prefill_part_calls": ("rope_cache_attention_prefill (the engine's prompt step)" if pf_fused
                               else "rope_and_cache + attention_prefill"),
        "prefill_part_two_calls_ms": round(ms_pfp2, 5),
        "decode_part_ms": round(ms_dec, 5),
        "decode_part_gbs": round(dec_bytes / (ms_dec * 1e-3) / 1e9, 2),
        "decode_part_calls": ("rope_cache_attention_planned (the engine's decode step)" if fused
                              else "rope_and_cache + attention"),
        "decode_part_two_calls_ms": round(ms_dec2, 5),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": mfma_peak,
                     "unit": "TFLOP/s", "frac": round(tflops / mfma_peak, 4), "traffic": None,
                     "kernel": ("prefill_mfma_f32_kernel" if kv == "f32" else "prefill_mfma_kernel")
                               + " (one ie_hip_attention_prefill call, causal 4,000 x 4,000, "
                                 "28.7 GFLOP)",
                     "us_per_launch": round(ms_pf * 1e3, 3)},
    }
    if not args.no_cpu:
        host = lambda t: (t.cpu().numpy() if kv == "f32" else
                          t.cpu().view(torch.int16).numpy().view(np.uint16))
        kh, vh = host(k_pool), host(v_pool)
        tab_h = d_tab.cpu().numpy().reshape(pool.max_batch, max_pages)

        def gather(sq, n):  # the sequence's positions 0..n-1, contiguous fp32
            idx = tab_h[sq, np.arange(n) // PAGE].astype(np.int64) * PAGE + np.arange(n) % PAGE
            kc, vc = kh[idx], vh[idx]
            if kv != "f32":
                kc, vc = O.widen_kv(kc, KV_CODES[kv]), O.widen_kv(vc, KV_CODES[kv])
            return np.ascontiguousarray(kc, np.float32), np.ascontiguousarray(vc, np.float32)

        kc_pf, vc_pf = gather(pf, P)
        res["cpu_baseline"] = cpu_baseline_mixed(O, pq.cpu().numpy(), kc_pf, vc_pf, P,
                                                 dq.cpu().numpy(),
                                                 [gather(sq, lens[sq] + 1) for sq in dec])
    return res


def _probe_lib():
    """libie_probe.so: the hand-written HBM probes (llm-inference-engine_amd/probe)."""
    path = os.path.join(ROOT, "llm-inference-engine_amd", "libie_probe.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    vp, i = ctypes.c_void_p, ctypes.c_int
    lib.ie_probe_read.argtypes = [vp, ctypes.c_size_t, i, vp, vp]
    lib.ie_probe_read_form.argtypes = [vp, ctypes.c_size_t, i, i, vp, vp]
    lib.ie_probe_pages.argtypes = [vp, vp, vp, vp, vp, vp, i, i, i, i, vp, vp]
    lib.ie_probe_pages_form.argtypes = [vp, vp, vp, vp, vp, vp, i, i, i, i, i, vp, vp]
    lib.ie_probe_pages_ring.argtypes = [vp, vp, vp, i, i, i, vp, vp]
    return lib


def hbm_probes(args, torch, stream, k_pools, v_pools, d_tab, lens, max_pages, ct, kv):
    """The read rate this device reaches with no arithmetic, measured as the decode call
    is (graph replays, median), with the kernels of llm-inference-engine_amd/probe:
      read_70MB   contiguous 16-byte loads of 70 MB (one attention call's size), over 8
                  buffers in turn (560 MB, twice the 256 MB Infinity Cache);
      read_256MB  the same for 256 MB over 4 buffers (1 GB): the large-stream rate;
      page_walk   config 3's own grid and block tables over the same rotated pools,
                  reading every K and V page of every (row, chunk) and nothing else.
    Each is timed in four load forms -- 16-byte loads into registers, plain or
    non-temporal, and LDS DMA, plain or non-temporal (the decode kernel reads K pages
    the second way and V pages the fourth) -- and reports the fastest (`*_form`).
    ceiling_gbs is read_70MB: what one 70 MB read of this device achieves per launch."""
    lib = _probe_lib()
    if lib is None:
        return None
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.zeros(1 << 20, dtype=torch.int32, device=dev)
    sp = lambda: torch.cuda.current_stream().cuda_stream  # the capture stream while recording
    out = {}
    forms = ("plain", "nontemporal", "dma", "dma_nontemporal")
    for mb, nbuf in ((70, 8), (256, 4)):
        nbytes = mb * 1000 * 1000 // 4096 * 4096  # whole 4 KB blocks for the DMA forms
        bufs = [torch.randint(0, 1 << 30, (nbytes // 4,), dtype=torch.int32, device=dev)
                for _ in range(nbuf)]

        best = None
        for fi, form in enumerate(forms):
            for per_cu in (4, 8, 16, 32):  # workgroups of 256 threads per compute unit
                def step(i, bufs=bufs, nbytes=nbytes, nbuf=nbuf, wgs=per_cu * cus, fi=fi):
                    rc = lib.ie_probe_read_form(bufs[i % nbuf].data_ptr(), nbytes, wgs, fi,
                                                sink.data_ptr(), sp())
                    assert rc == 0

                ms = time_steps(torch, step, max(args.steps, 40), 5, stream)
                if best is None or ms < best[0]:
                    best = (ms, per_cu, form)
        ms = best[0]
        out[f"read_{mb}MB_gbs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        out[f"read_{mb}MB_us"] = round(ms * 1e3, 3)
        out[f"read_{mb}MB_workgroups_per_cu"] = best[1]
        out[f"read_{mb}MB_form"] = best[2]
        del bufs
    rows, chunks = [], []
    for r, L in enumerate(lens):
        for c in range((int(L) + ct - 1) // ct):
            rows.append(r)
            chunks.append(c)
    d_r = torch.tensor(rows, dtype=torch.int32, device=dev)
    d_c = torch.tensor(chunks, dtype=torch.int32, device=dev)
    d_len = torch.tensor([int(L) for L in lens], dtype=torch.int32, device=dev)
    page_bytes = PAGE * KVD * KV_BYTES[kv]
    walk_bytes = 2 * page_bytes * sum((int(L) + PAGE - 1) // PAGE for L in lens)

    best = None
    for fi, form in enumerate(forms):
        def walk(i, fi=fi):
            l = i % len(k_pools)
            rc = lib.ie_probe_pages_form(k_pools[l].data_ptr(), v_pools[l].data_ptr(),
                                         d_tab.data_ptr(), d_r.data_ptr(), d_c.data_ptr(),
                                         d_len.data_ptr(), len(rows), max_pages, ct, page_bytes,
                                         fi, sink.data_ptr(), sp())
            assert rc == 0

        ms = time_steps(torch, walk, max(args.steps, 40), 5, stream)
        if best is None or ms < best[0]:
            best = (ms, form)
    ms = best[0]
    out["page_walk_gbs"] = round(walk_bytes / (ms * 1e-3) / 1e9, 1)
    out["page_walk_us"] = round(ms * 1e3, 3)
    out["page_walk_form"] = best[1]
    out["page_walk_bytes"] = walk_bytes

    # The same pages as one flat list, walked by persistent one-wave workgroups with
    # `ring` pages (K + V) in flight per wave: a shape of its own, not the kernel's.
    flat = []
    tab_h = d_tab.cpu().numpy()
    for r, L in enumerate(lens):
        flat.extend(int(x) for x in tab_h[r, :(int(L) + PAGE - 1) // PAGE])
    d_flat = torch.tensor(flat, dtype=torch.int32, device=dev)
    best = None
    sweep = {}
    if page_bytes == 4096:
        for ring, per_cu in ((1, 16), (2, 8), (2, 10), (4, 4), (4, 5), (8, 2), (2, 4), (4, 2)):
            waves = per_cu * cus
            if len(flat) > 64 * waves:
                continue

            def ring_walk(i, ring=ring, waves=waves):
                l = i % len(k_pools)
                rc = lib.ie_probe_pages_ring(k_pools[l].data_ptr(), v_pools[l].data_ptr(),
                                             d_flat.data_ptr(), len(flat), waves, ring,
                                             sink.data_ptr(), sp())
                assert rc == 0

            ms = time_steps(torch, ring_walk, max(args.steps, 40), 5, stream)
            sweep[f"r{ring}x{per_cu}"] = round(ms * 1e3, 3)
            if best is None or ms < best[0]:
                best = (ms, ring, per_cu)
    if best is not None:
        ms = best[0]
        out["page_ring_gbs"] = round(walk_bytes / (ms * 1e-3) / 1e9, 1)
        out["page_ring_us"] = round(ms * 1e3, 3)
        out["page_ring_shape"] = {"pages_in_flight_per_wave": best[1], "waves_per_cu": best[2]}
        out["page_ring_sweep_us"] = sweep
    out["ceiling_gbs"] = out["read_70MB_gbs"]
    return out


def extra_targets(args, torch, ie, O):
    """The north star's other two targets, measured in the default run so that one line
    carries all three: the RoPE + append (config 2: 64 rows, and 131,072 rows per launch,
    K/V only) and the 4,000-token prefill's MFMA fraction (config 5)."""
    import copy
    sub = copy.copy(args)
    sub.no_cpu, sub.kv, sub.chunk_tokens, sub.sweep = True, None, None, False
    sub.steps, sub.warmup = max(20, min(args.steps, 100)), 5
    sub.append_rows, sub.append_q = [64, 131072], "off"
    app = bench_append(sub, torch, ie, O)
    pts = {s["rows"]: s for s in app["sweep"] if not s["with_q"]}
    copy_gbs = copy_probe(torch)
    mix = bench_mixed(sub, torch, ie, O)
    sub4 = copy.copy(sub)
    sub4.steps = max(10, min(args.steps, 50))
    lng = bench_long(sub4, torch, ie, O)
    return {
        "config4_decode": {
            "us_per_layer": lng["us_per_layer"], "ms_per_step": lng["ms_per_step"],
            "gbs": lng["roofline"]["achieved"], "frac": lng["roofline"]["frac"],
            "traffic_per_step": lng["roofline"]["traffic"],
            "algorithmic_bytes_per_step": lng["algorithmic_bytes_per_step"],
            "kernel": lng["roofline"]["kernel"], "layer_calls": lng["config"]["layer_calls"]},
        "config2_append": {
            "rows_64": {"us_per_launch": pts[64]["us_per_launch"], "gbs": pts[64]["gbs"],
                        "frac": round(pts[64]["gbs"] / HBM_PEAK_GBS, 4)},
            "rows_131072": {"us_per_launch": pts[131072]["us_per_launch"],
                            "gbs": pts[131072]["gbs"],
                            "frac": round(pts[131072]["gbs"] / HBM_PEAK_GBS, 4),
                            "traffic": traffic_from_profiles("append_131072", "f16", "f16",
                                                             sub)},
            "target_frac": 0.60, "bytes_per_row": 1548,
            # The append reads 2/3 and writes 1/3 of its bytes: a device-to-device copy
            # (read + write, 2 GiB) measured in the same run is its ceiling.
            "copy_gbs": copy_gbs,
            "frac_of_copy": round(pts[131072]["gbs"] / copy_gbs, 4),
            "kernel": "rope_append_kernel (ie_hip_rope_and_cache, K/V only)"},
        "config5_prefill": {
            "us_per_launch": mix["roofline"]["us_per_launch"],
            "tflops": mix["roofline"]["achieved"], "frac": mix["roofline"]["frac"],
            "mixed_step_ms": mix["ms_per_step"],
            "prefill_part_ms": mix["prefill_part_ms"],
            "prefill_part_two_calls_ms": mix["prefill_part_two_calls_ms"],
            "mixed_step_two_branches_ms": mix["ms_per_step_two_branches"],
            "decode_part_gbs": mix["decode_part_gbs"],
            "kernel": mix["roofline"]["kernel"]},
    }


def bench_config1(args, torch, ie, O):
    """Config 1, the reference's own CPU case: one layer of one sequence, Qwen2.5-0.5B's
    attention shape -- rope(q) and rope(k) at position 511, k/v appended to a contiguous
    fp32 cache whose rows 0..510 are N(0,1), then decode attention over the 512 positions
    (src/model.cpp:62-77, src/ops.cpp:34-108). The CPU side runs the reference's own
    rope and attention (oracle/_ref) on its thread pool; the GPU side runs the same work on
    the paged path (f32 KV, 32 pages): ie_hip_rope_and_cache + ie_hip_attention."""
    rng = np.random.default_rng(args.seed)
    L, pos = 512, 511
    q = rng.standard_normal((1, QD), dtype=np.float32)
    k = rng.standard_normal((1, KVD), dtype=np.float32)
    v = rng.standard_normal((1, KVD), dtype=np.float32)
    kc = rng.standard_normal((L, KVD), dtype=np.float32)
    vc = rng.standard_normal((L, KVD), dtype=np.float32)
    dev = torch.device("cuda:0")
    # GPU: the same step on pages.
    pages = L // PAGE
    tables = rng.permutation(pages).astype(np.int32)[None, :]
    kp = np.zeros((pages * PAGE, KVD), np.float32)
    vp = np.zeros((pages * PAGE, KVD), np.float32)
    for i in range(pages):
        kp[tables[0, i] * PAGE:(tables[0, i] + 1) * PAGE] = kc[i * PAGE:(i + 1) * PAGE]
        vp[tables[0, i] * PAGE:(tables[0, i] + 1) * PAGE] = vc[i * PAGE:(i + 1) * PAGE]
    k_pool, v_pool = torch.from_numpy(kp).to(dev), torch.from_numpy(vp).to(dev)
    d_tab = torch.from_numpy(tables).to(dev)
    d_pos = torch.tensor([pos], dtype=torch.int32, device=dev)
    d_seq = torch.zeros(1, dtype=torch.int32, device=dev)
    dq0 = torch.from_numpy(q).to(dev)
    dq = dq0.clone()
    dk, dv = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    table = ie.rope_table(L, HD, THETA).to(dev)
    ct = ie.attention_chunk_tokens(1, L, ie.KV_F32)
    nc = ie.attention_chunks(L, ct)
    ws = ie.attention_workspace(1, NH, HD, nc)
    out = torch.empty((1, QD), device=dev)
    stream = torch.cuda.current_stream()

    def step(i):
        dq.copy_(dq0)
        ie.rope_and_cache(dq, dk, dv, k_pool, v_pool, table, d_pos, d_seq, d_tab, pages, NH, NKV,
                          HD)
        ie.attention(out, dq, k_pool, v_pool, d_pos, d_seq, d_tab, pages, nc, ct, ws, NH, NKV, HD)

    ms = time_steps(torch, step, args.steps, args.warmup, stream)
    timing = dict(TIMING)
    nbytes = 1024 * L + 2 * QD * 4 + 4 * pages + 8 + 1548 + 2 * QD * 4
    res = {
        "metric": "config 1: one decode step of one layer, 512 positions, fp32 KV (tok/s)",
        "value": round(1 / (ms * 1e-3), 1), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "config 1: rope(q), rope(k) at 511, append, attention over 512 "
                               "positions, 14q/2kv heads of 64, f32 KV", "seed": args.seed,
                   "chunk_tokens": ct},
        "timing": timing,
        "roofline": {"bound": "hbm", "achieved": round(nbytes / (ms * 1e-3) / 1e9, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 5),
                     "traffic": None, "kernel": "rope_append_kernel + decode_partial_mfma_f32 "
                                                "(+ merge): latency-bound at this size",
                     "us_per_launch": round(ms * 1e3, 3)},
    }
    if not args.no_cpu and O.ref_available():
        cores = O.physical_cores()
        O.ref().ref_set_num_threads(cores)  # the reference's pool: one thread per core
        times, t_start = [], time.perf_counter()
        while True:
            t0 = time.perf_counter()
            qr = O.ref_rope(q, NH, HD, pos, THETA)
            kr = O.ref_rope(k, NKV, HD, pos, THETA)
            kc[pos] = kr[0]
            vc[pos] = v[0]
            O.ref_attention(qr, kc, vc, pos, NH, NKV, HD)
            times.append(time.perf_counter() - t0)
            if time.perf_counter() - t_start >= min(args.cpu_seconds, 5.0) and len(times) >= 50:
                break
        t = float(np.median(times))
        res["cpu_baseline"] = {
            "value": round(1 / t, 1), "unit": "tok/s", "cores": cores, "threads": cores,
            "physical_cores": cores, "kind": "reference",
            "sample": f"the whole case, {len(times)} runs, median {t * 1e6:.1f} us (the "
                      f"reference's rope + attention on its thread pool; the append is a copy)"}
    return res


def traffic_from_profiles(key: str, kv: str, default_kv: str, args):
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE/WRITE_SIZE runs, as committed
    under profiles/: `key` for the workload's default KV type, `key_<kv>` for another.
    Null when that measurement has not been made, or when the chunk size is overridden
    (the counters were read at the library's own choice)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if args.chunk_tokens or not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get(key if kv == default_kv else f"{key}_{kv}")


def copy_probe(torch, n_bytes=2 << 30):
    """Device-to-device copy bandwidth (read + write), the measured HBM ceiling."""
    a = torch.empty(n_bytes // 4, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1.0)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(10):
        b.copy_(a)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / 10
    del a, b
    return round(2 * n_bytes / (ms * 1e-3) / 1e9, 1)


def bench_model(args, torch, ie, O):
    """Config 6: the whole decode step around the path -- a 24-layer Qwen2.5-0.5B decoder
    (hidden 896, intermediate 4,864, 14/2 heads, tied LM head over 151,936 tokens) with
    random BF16 weights, one new token for each of config 3's 64 rows (L ~ U[128, 4096],
    f16 KV, shuffled 16-token pages, one pool pair per layer). Per layer: rmsnorm folded
    into q/k/v (one launch), RoPE + paged append + attention (one launch), o_proj into the
    residual, rmsnorm folded into gate/up + SiLU (one launch), down into the residual;
    then the final norm and the logits of every row (src/cuda/cuda_runner.cu:418-470)."""
    dev = torch.device("cuda:0")
    kv = args.kv or "f16"
    rng = np.random.default_rng(args.seed)
    layers, B, H, I, V = 24, 64, 896, 4864, 151936
    lens = rng.integers(128, 4097, B)
    max_pages = 4096 // PAGE
    num_pages = 2 * int(sum((int(n) + PAGE - 1) // PAGE for n in lens))
    tabs = [torch.from_numpy(make_tables(rng, lens, num_pages, max_pages)).to(dev)
            for _ in range(layers)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    log(f"config 6: seed {args.seed}, {layers} layers, {num_pages} pages per pool, {kv} KV")
    k_pools = [fill_pool(torch, num_pages * PAGE, kv, gen, dev) for _ in range(layers)]
    v_pools = [fill_pool(torch, num_pages * PAGE, kv, gen, dev) for _ in range(layers)]

    def w(rows, cols, s):  # BF16 weights [rows, cols], N(0, s^2)
        return (torch.randn((rows, cols), generator=gen, device=dev) * s).to(torch.bfloat16)

    def vec(n, base, s):
        return base + s * torch.randn(n, generator=gen, device=dev)

    Wl = []
    for _ in range(layers):
        Wl.append(dict(inorm=vec(H, 1.0, 0.1), pnorm=vec(H, 1.0, 0.1),
                       q=w(QD, H, 0.04), k=w(KVD, H, 0.04), v=w(KVD, H, 0.04),
                       bq=vec(QD, 0.0, 0.1), bk=vec(KVD, 0.0, 0.1), bv=vec(KVD, 0.0, 0.1),
                       o=w(H, QD, 0.03), g=w(I, H, 0.03), u=w(I, H, 0.03), d=w(H, I, 0.015)))
    int8 = args.weights == "int8"

    def mat(wb):  # BF16 weights, or INT8 with row scales (src/matrix.cpp:84-97)
        if not int8:
            return ie.matrix(wb), (wb,)
        wf = wb.float()
        amax = wf.abs().amax(dim=1)
        sc = torch.where(amax > 0, amax / 127.0, torch.ones_like(amax))
        q8 = torch.round(wf / sc[:, None]).clamp(-127, 127).to(torch.int8)
        return ie.matrix(q8, sc), (q8, sc)

    for t in Wl:  # Wq, Wk, Wv stacked for the one-launch q/k/v projection
        t["qkv"] = torch.cat([t["q"], t["k"], t["v"]]).contiguous()
        t["bqkv"] = torch.cat([t["bq"], t["bk"], t["bv"]]).contiguous()
    keep = []
    M = []
    for t in Wl:
        mm = {}
        for n in ("qkv", "o", "g", "u", "d"):
            mm[n], kp_ = mat(t[n])
            keep.append(kp_)
        M.append(mm)
    E = w(V, H, 1.0)
    m_e, keep_e = mat(E)
    final_norm = vec(H, 1.0, 0.1)
    ids = torch.from_numpy(rng.integers(0, V, B).astype(np.int32)).to(dev)
    x = torch.empty((B, H), device=dev)
    xn = torch.empty((B, H), device=dev)
    q = torch.empty((B, QD), device=dev)
    k = torch.empty((B, KVD), device=dev)
    v = torch.empty((B, KVD), device=dev)
    attn = torch.empty((B, QD), device=dev)
    mid = torch.empty((B, I), device=dev)
    logits = torch.empty((B, V), device=dev)
    table = ie.rope_table(4096, HD, THETA).to(dev)
    d_pos = torch.from_numpy((lens - 1).astype(np.int32)).to(dev)
    d_seq = torch.arange(B, dtype=torch.int32, device=dev)
    ct = args.chunk_tokens or ie.attention_chunk_tokens(B, 4096, KV_CODES[kv])
    nc = ie.attention_chunks(4096, ct)
    ws = ie.attention_workspace(B, NH, HD, nc)
    if not ie.rope_cache_attention_supported(KV_CODES[kv], NH, NKV, HD, ct):
        sys.exit("config 6 needs the one-launch decode step (16-bit KV)")
    eps = 1e-6
    stream = torch.cuda.current_stream()

    def step(i):
        ie.embedding(x, ids, m_e)
        for l in range(layers):
            t, m = Wl[l], M[l]
            ie.rmsnorm_qkv_proj(q, k, v, x, t["inorm"], eps, m["qkv"], t["bqkv"])
            ie.rope_cache_attention(attn, q, k, v, k_pools[l], v_pools[l], table, d_pos, d_seq,
                                    tabs[l], max_pages, nc, ct, ws, NH, NKV, HD)
            ie.matmul(x, attn, m["o"], accumulate=True)
            ie.rmsnorm_gate_up_silu(mid, x, t["pnorm"], eps, m["g"], m["u"])
            ie.matmul(x, mid, m["d"], accumulate=True)
        ie.rmsnorm(xn, x, final_norm, eps)
        ie.matmul(logits, xn, m_e)

    ms = time_steps(torch, step, args.steps, args.warmup, stream)
    assert bool(torch.isfinite(logits).all()), "non-finite logits"
    wb = 1 if int8 else 2  # bytes per weight, plus a 4-byte scale per row for INT8
    w_bytes = wb * (QD * H + 2 * KVD * H + H * QD + 2 * I * H + H * I) + \
        (4 * (QD + 2 * KVD + H + 2 * I + H) if int8 else 0)
    kv_bytes = decode_bytes(lens, KV_BYTES[kv])
    nbytes = layers * (w_bytes + kv_bytes) + wb * V * H + (4 * V if int8 else 0) + 4 * B * V
    gbs = nbytes / (ms * 1e-3) / 1e9
    res = {
        "metric": "decode step (24-layer Qwen2.5-0.5B shape, batch 64) tok/s, 1 GPU",
        "value": round(B / (ms * 1e-3), 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": kv, "data": "synthetic",
        "config": {"workload": "config 6: 24 layers x (rmsnorm+q/k/v, RoPE+append+attention, "
                               "o_proj, rmsnorm+gate/up+SiLU, down) + final norm + tied LM "
                               "head, batch 64, L~U[128,4096], random BF16 weights",
                   "kv_dtype": kv, "weights": args.weights, "chunk_tokens": ct,
                   "num_chunks": nc, "seed": args.seed},
        "us_per_layer": round((ms * 1e3) / layers, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "the whole step (one graph replay)",
                     "us_per_launch": round(ms * 1e3, 3)},
        "algorithmic_bytes_per_step": nbytes,
        "bytes_note": "weights once per step, KV as config 3 per layer, the logits written; "
                      "activations (under 3%) not counted",
    }
    if not args.no_cpu and not int8 and O.ref_available():
        bits = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16).copy()
        t0 = Wl[0]
        layer_bits = {n: bits(t0[n]) for n in ("q", "k", "v", "o", "g", "u", "d")}
        norms = [t0["inorm"].cpu().numpy(), t0["pnorm"].cpu().numpy()]
        x_h = torch.randn((B, H), generator=gen, device=dev).cpu().numpy()
        host = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)
        kp0, vp0, tab0 = host(k_pools[0]), host(v_pools[0]), tabs[0].cpu().numpy()
        kcs, vcs, ps = [], [], []
        for r in range(8):  # a sample of rows, gathered to contiguous fp32
            L = int(lens[r])
            idx = tab0[r, np.arange(L) // PAGE].astype(np.int64) * PAGE + np.arange(L) % PAGE
            kcs.append(O.widen_kv(kp0[idx], KV_CODES[kv]))
            vcs.append(O.widen_kv(vp0[idx], KV_CODES[kv]))
            ps.append(L - 1)
        res["cpu_baseline"] = cpu_baseline_model(O, layer_bits, norms, bits(E), x_h, kcs, vcs,
                                                 ps, layers)
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 4, 5, 6])
    ap.add_argument("--kv", choices=list(KV_CODES), default=None)
    ap.add_argument("--chunk-tokens", type=int, default=None)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--impl", choices=["auto", "valu", "mfma"], default="auto")
    ap.add_argument("--seed", type=int, default=20263)
    ap.add_argument("--unfused", action="store_true",
                    help="config 4: RoPE + append and attention as two calls per layer")
    ap.add_argument("--weights", choices=["bf16", "int8"], default="bf16",
                    help="config 6: weight storage (INT8 with row scales, as --dtype int8)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--sweep", action="store_true", help="config 2: rows-per-launch sweep")
    ap.add_argument("--append-rows", default=None,
                    help="config 2: comma-separated rows per launch to time instead of the "
                         "default (64, or the sweep); one size alone gives per-dispatch "
                         "counters of that size")
    ap.add_argument("--plan", choices=["on", "off"], default="on",
                    help="configs 3 and 4: the decode work list built on the host "
                         "(ie_hip_attention_plan), as the engine does, or located by the kernel")
    ap.add_argument("--append-q", choices=["off", "on", "both"], default="both",
                    help="config 2: time the append without q (K/V only), with q rotated in "
                         "place, or both (the headline is K/V only unless 'on'); one mode "
                         "alone gives per-dispatch counters of that mode")
    ap.add_argument("--probe", action="store_true", help="also measure device copy bandwidth")
    ap.add_argument("--no-probe", action="store_true",
                    help="config 3: skip the HBM read probes (ceiling_gbs)")
    ap.add_argument("--no-extras", action="store_true",
                    help="config 3: skip the config-2 append and config-5 prefill keys")
    ap.add_argument("--eager", action="store_true",
                    help="launch the timed steps one by one instead of replaying a graph "
                         "(host-bound timing; for rocprofv3 counter runs)")
    ap.add_argument("--probe-only", action="store_true",
                    help="only the device copy (the plain copy kernel that rocprofv3 byte "
                         "counters are calibrated on)")
    args = ap.parse_args()
    if args.append_rows:
        args.append_rows = [int(x) for x in args.append_rows.split(",")]
    global EAGER
    EAGER = args.eager
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this path has no multi-GPU mode (the paged KV "
              "cache would shard by sequence, one pool per GPU, with no exchange); run with "
              "--gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import __graft_entry__ as g
    import oracle as O

    ie = g.load()
    ie.lib()
    ie.set_attention_impl({"auto": ie.IMPL_AUTO, "valu": ie.IMPL_VALU, "mfma": ie.IMPL_MFMA}[args.impl])
    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")
    if args.probe_only:
        print(json.dumps({"measured_copy_gbs": copy_probe(torch), "copy_bytes": 2 << 30}),
              flush=True)
        return
    res = {1: bench_config1, 2: bench_append, 3: bench_decode, 4: bench_long, 5: bench_mixed,
           6: bench_model}[args.config](
        args, torch, ie, O)
    if args.config == 3 and not args.no_extras and args.impl == "auto" and not args.kv:
        res.update(extra_targets(args, torch, ie, O))
    if args.probe:
        res["measured_copy_gbs"] = copy_probe(torch)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
