"""The C++ engine layer (include/ie_hip_engine.hpp) on the GPU, through its
self-test driver (tests/engine/engine_selftest.cpp, built by build()).

The driver runs a serving sequence through ie::hip::KvEngine -- prompts of
1/17/62/255/500/1000/3000 rows, a prompt continuing at 500, decode graphs of
batch 1, 4 and 5 (recorded once, replayed, rows reordered), a mixed direct step
of two decodes and a 30-row prompt, page reuse after closing sequences, and the
reference's errors (KV cache full, too long, closed sequence) -- and after every
step checks both page pools of both layers byte for byte against the CPU oracle,
the device page table against the host one, attention against the oracle (f32:
compare() <= 1e-5; f16/bf16: 2e-3 absolute), the step's path, and page
conservation. These are the situations of the reference's run_selftest
(src/cuda/cuda_runner.cu:849-1018).
"""
from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "engine", "_bin", "engine_selftest")


def test_driver_built_and_linked():
    """CPU: the driver exists and its libraries resolve (libie_hip.so, liborc.so)."""
    assert os.path.exists(BIN), "engine_selftest not built: run __graft_entry__.build()"
    out = subprocess.run(["ldd", BIN], capture_output=True, text=True, check=True).stdout
    assert "not found" not in out, out
    assert "libie_hip.so" in out and "liborc.so" in out


@pytest.mark.gpu
@pytest.mark.parametrize("kv", ["f32", "f16", "bf16"])
def test_engine_selftest(kv):
    print(f"engine_selftest {kv}", flush=True)
    r = subprocess.run([BIN, kv], capture_output=True, text=True, timeout=110)
    print(r.stdout[-6000:], r.stderr[-2000:], flush=True)
    fails = [l for l in r.stdout.splitlines() if l.startswith("FAIL")]
    assert r.returncode == 0 and not fails, "\n".join(fails) or f"exit status {r.returncode}"
    assert " checks, 0 failures" in r.stdout


MODEL_BIN = os.path.join(ROOT, "tests", "engine", "_bin", "model_selftest")


def test_model_driver_built_and_linked():
    """CPU: the decode-step driver (tests/engine/model_selftest.cpp) exists and links."""
    assert os.path.exists(MODEL_BIN), "model_selftest not built: run __graft_entry__.build()"
    out = subprocess.run(["ldd", MODEL_BIN], capture_output=True, text=True, check=True).stdout
    assert "not found" not in out, out


@pytest.mark.gpu
@pytest.mark.parametrize("kv,weights", [("f32", "bf16"), ("f16", "bf16"), ("f32", "int8")])
def test_model_selftest(kv, weights):
    """A 2-layer Qwen2 decoder (Qwen2.5-0.5B layer shape) through KvEngine + DecoderModel
    (include/ie_hip_model.hpp): prompts, decode graphs and a replay; after every step the
    residual stream and logits against the reference's CPU forward restated on the oracle."""
    print(f"model_selftest {kv} {weights}", flush=True)
    r = subprocess.run([MODEL_BIN, kv, weights], capture_output=True, text=True, timeout=110)
    print(r.stdout[-6000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and " checks, 0 failures" in r.stdout


RUNNER_BIN = os.path.join(ROOT, "tests", "engine", "_bin", "runner_selftest")
REF_SRC = "/root/reference/src"


def test_runner_driver_built_and_linked():
    """CPU: the Runner/BatchRunner driver (tests/engine/runner_selftest.cpp) exists and
    links libie_hip.so and the reference's CPU Runner (oracle/_ref/libieref_model.so). It
    is built only where the reference checkout is (its headers are compiled in place)."""
    if not os.path.exists(RUNNER_BIN):
        if os.path.isdir(REF_SRC):
            pytest.fail("runner_selftest not built: run __graft_entry__.build()")
        pytest.skip("no reference checkout here and no prebuilt driver")
    out = subprocess.run(["ldd", RUNNER_BIN], capture_output=True, text=True, check=True).stdout
    assert "not found" not in out, out
    assert "libie_hip.so" in out and "libieref_model.so" in out


@pytest.mark.gpu
@pytest.mark.parametrize("kv,weights", [("f32", "bf16"), ("f16", "bf16"), ("bf16", "bf16"),
                                        ("f32", "int8")])
def test_runner_selftest(kv, weights):
    """ie::hip::make_runner / make_batch_runner through the reference's own Runner and
    BatchRunner interfaces, against the reference's own CPU Runner on the same weights:
    prefill, decode, greedy, close and reuse, errors, stage reports; batch invariance end
    to end (logits bit for bit); the continuous-batching scheduler's --check."""
    if not os.path.exists(RUNNER_BIN):
        pytest.skip("runner_selftest not built (no reference checkout where the tree was built)")
    print(f"runner_selftest {kv} {weights}", flush=True)
    r = subprocess.run([RUNNER_BIN, kv, weights], capture_output=True, text=True, timeout=200)
    print(r.stdout[-8000:], r.stderr[-2000:], flush=True)
    fails = [l for l in r.stdout.splitlines() if l.startswith("FAIL")]
    assert r.returncode == 0 and not fails, "\n".join(fails) or f"exit status {r.returncode}"
    assert " checks, 0 failures" in r.stdout
