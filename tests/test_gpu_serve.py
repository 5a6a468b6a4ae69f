"""The reference's OpenAI-compatible server over the MI355X drop-in.

tests/engine/serve_selftest.cpp compiles the reference's src/server.cpp (its
continuous-batching Engine, :104-368, started by run_server, :372-409) with the
reference's tokenizer and sampler in place from the checkout, and serves
ie::hip::make_batch_runner through it on 127.0.0.1: ten completions requests served
one at a time, then the same ten at once beside a streamed request whose client
disconnects after three chunks. Every burst reply must equal the reply served alone
(text, finish reason, token count: greedy decoding on a batch-invariant engine), the
burst must run batched, and every KV page -- the cancelled request's included -- must
be back in the pool once the engine drains. The server logs each retired request on
stderr; the cancelled one must retire as "cancelled"."""
from __future__ import annotations

import os
import socket
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SERVE_BIN = os.path.join(ROOT, "tests", "engine", "_bin", "serve_selftest")
REF_SRC = "/root/reference/src"


def test_serve_driver_built_and_linked():
    """CPU: the server driver exists and links libie_hip.so and the reference's CPU code."""
    if not os.path.exists(SERVE_BIN):
        if os.path.isdir(REF_SRC):
            pytest.fail("serve_selftest not built: run __graft_entry__.build()")
        pytest.skip("no reference checkout here and no prebuilt driver")
    out = subprocess.run(["ldd", SERVE_BIN], capture_output=True, text=True, check=True).stdout
    assert "not found" not in out, out
    assert "libie_hip.so" in out and "libieref_model.so" in out


def free_port() -> int:
    with socket.socket(socket.AF_INET, socket.SOCK_STREAM) as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


@pytest.mark.gpu
@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_server_over_the_drop_in(kv):
    if not os.path.exists(SERVE_BIN):
        pytest.skip("serve_selftest not built (no reference checkout where the tree was built)")
    port = free_port()
    print(f"serve_selftest {port} {kv}", flush=True)
    r = subprocess.run([SERVE_BIN, str(port), kv], capture_output=True, text=True, timeout=200)
    print(r.stdout[-6000:], r.stderr[-3000:], flush=True)
    fails = [l for l in r.stdout.splitlines() if l.startswith("FAIL")]
    assert r.returncode == 0 and not fails, "\n".join(fails) or f"exit status {r.returncode}"
    assert " checks, 0 failed" in r.stdout
    assert "| cancelled]" in r.stderr, "the disconnected stream did not retire as cancelled"
