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


def test_checkpoint_writer_round_trip(tmp_path):
    """CPU: the checkpoint the GPU test serves (tests/checkpoint.py) is a valid
    safetensors file -- read back by the safetensors package, an independent reader,
    every tensor's BF16 bits equal torch's round-to-nearest-even of the float32
    weights -- and config.json has the keys the reference's load_config reads
    (src/config.cpp:16-26)."""
    import json
    import torch
    from safetensors.torch import load_file
    from checkpoint import write_checkpoint
    want = write_checkpoint(str(tmp_path), seed=5, layers=1, inter=64, vocab=32, tie=False)
    got = load_file(str(tmp_path / "model.safetensors"))
    assert sorted(got) == sorted(want)
    for name, x in want.items():
        ref = torch.from_numpy(x).to(torch.bfloat16)
        assert got[name].dtype == torch.bfloat16 and tuple(got[name].shape) == x.shape, name
        assert torch.equal(got[name].view(torch.int16), ref.view(torch.int16)), name
    cfg = json.load(open(tmp_path / "config.json"))
    for key in ("hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
                "num_key_value_heads", "vocab_size", "rms_norm_eps", "rope_theta",
                "tie_word_embeddings"):
        assert key in cfg, key


@pytest.mark.gpu
@pytest.mark.parametrize("kv", ["f32", "f16"])
def test_runner_checkpoint(tmp_path, kv):
    """safetensors -> device weights through the drop-in: a 2-layer checkpoint on disk
    (untied LM head, q/k/v biases) read by the reference's own loader (load_config,
    SafeTensorsFile, load_weights as BF16 and INT8), served by make_batch_runner and
    by the reference's CPU Runner from the same Weights; prompt and decode logits
    agree within the runner self-test's tolerance."""
    if not os.path.exists(RUNNER_BIN):
        pytest.skip("runner_selftest not built (no reference checkout where the tree was built)")
    from checkpoint import write_checkpoint
    write_checkpoint(str(tmp_path))
    print(f"runner_selftest {kv} --checkpoint {tmp_path}", flush=True)
    r = subprocess.run([RUNNER_BIN, kv, "bf16", "--checkpoint", str(tmp_path)],
                       capture_output=True, text=True, timeout=200)
    print(r.stdout[-8000:], r.stderr[-2000:], flush=True)
    fails = [l for l in r.stdout.splitlines() if l.startswith("FAIL")]
    assert r.returncode == 0 and not fails, "\n".join(fails) or f"exit status {r.returncode}"
    assert " checks, 0 failures" in r.stdout and "---- checkpoint" in r.stdout
