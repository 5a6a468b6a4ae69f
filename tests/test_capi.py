"""The C-ABI library loads, exports every entry point include/ie_hip.h declares,
and validates arguments on the host (no GPU calls are made here)."""
from __future__ import annotations

import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "ie_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(ie_(?:hip|pages)_\w+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_bound_set(ie):
    assert declared_functions() == sorted(ie.EXPORTED)


@pytest.mark.parametrize("name", declared_functions())
def test_symbol_exported(ie, name):
    assert hasattr(ie.lib(), name)


def test_no_oracle_linked():
    """The product library must not depend on the CPU oracle."""
    import subprocess
    lib = os.path.join(ROOT, "llm-inference-engine_amd", "libie_hip.so")
    out = subprocess.run(["ldd", lib], capture_output=True, text=True).stdout
    assert "orc" not in out and "ieref" not in out
    syms = subprocess.run(["nm", "-D", lib], capture_output=True, text=True).stdout
    assert "orc_" not in syms and "ref_" not in syms


def test_version(ie):
    assert "gfx950" in ie.lib().ie_hip_version().decode()


def test_rope_table_matches_oracle(ie, O):
    got = ie.rope_table(33000, 64, 1e6).numpy()
    want = O.rope_table(33000, 64, 1e6)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got = ie.rope_table(100, 128, 1e4).numpy()
    assert np.array_equal(got.view(np.uint32), O.rope_table(100, 128, 1e4).view(np.uint32))


def _layout(ie, page_size=16, dtype=1, num_pages=4):
    return ie.KvLayout(0x1000, 4, page_size, dtype, num_pages)


def test_argument_checks(ie):
    L = ie.lib()
    kv = _layout(ie)
    fake = 0x1000
    # rope_and_cache
    assert L.ie_hip_rope_and_cache(fake, fake, fake, fake, fake, fake, 10, 1, fake, fake,
                                   _layout(ie, page_size=32), 14, 2, 64, None) == ie.EINVAL
    assert "page size must be 16" in ie.last_error()
    assert L.ie_hip_rope_and_cache(fake, fake, fake, fake, fake, fake, 10, 1, fake, fake, kv, 14, 2,
                                   96, None) == ie.EINVAL
    assert L.ie_hip_rope_and_cache(fake, fake, fake, fake, fake, fake, 10, 1, fake, fake,
                                   _layout(ie, dtype=7), 14, 2, 64, None) == ie.EINVAL
    assert L.ie_hip_rope_and_cache(None, None, fake, fake, fake, fake, 10, 1, fake, fake, kv, 14, 2,
                                   64, None) == ie.EINVAL
    assert L.ie_hip_rope_and_cache(None, fake, fake, fake, fake, fake, 10, 0, fake, fake, kv, 14, 2,
                                   64, None) == ie.OK  # T == 0: nothing to do
    # attention
    assert L.ie_hip_attention(fake, fake, fake, fake, 1, fake, fake, kv, 1, 64, fake, 14, 2, 128,
                              None) == ie.EINVAL
    assert L.ie_hip_attention(fake, fake, fake, fake, 1, fake, fake, kv, 1, 64, fake, 18, 2, 64,
                              None) == ie.EINVAL  # group 9
    assert "at most 8 query heads" in ie.last_error()
    assert L.ie_hip_attention(fake, fake, fake, fake, 1, fake, fake, kv, 1, 40, fake, 14, 2, 64,
                              None) == ie.EINVAL  # chunk not a multiple of 16
    assert L.ie_hip_attention(fake, fake, fake, fake, 1, fake, fake, kv, 0, 64, fake, 14, 2, 64,
                              None) == ie.EINVAL
    # prefill
    assert L.ie_hip_attention_prefill_supported(14, 2, 64) == 1
    assert L.ie_hip_attention_prefill_supported(14, 2, 128) == 0
    assert L.ie_hip_attention_prefill_supported(18, 2, 64) == 0
    assert L.ie_hip_attention_prefill(fake, fake, fake, fake, 1, fake, fake, kv, 18, 2, 64,
                                      None) == ie.EINVAL
    # gathers
    assert L.ie_hip_gather_rows(fake, fake, fake, -1, 4, None) == ie.EINVAL
    assert L.ie_hip_gather_rows(fake, fake, fake, 0, 4, None) == ie.OK
    assert L.ie_hip_gather_kv(fake, fake, kv, 0, 5, 12, None) == ie.EINVAL


def test_chunk_helpers(ie):
    assert ie.attention_chunks(4096, 512) == 8
    assert ie.attention_chunks(4097, 512) == 9
    assert ie.attention_chunks(1, 16) == 1
    # 16-bit caches (matrix-core kernel): 192-token chunks where rows x chunks at full
    # context reach 4 workgroups per compute unit, 64 where rows x 64-token chunks give
    # at most two, else 128 (small grids take one wave per page pair); float32: 192
    # where that reaches 4 workgroups per compute unit, else the largest of 128 and 64
    # that still gives two, else 32. No GPU here: the helper assumes MI355X's 256
    # compute units.
    assert ie.attention_chunk_tokens(64, 4096, ie.KV_F16) == 192   # 64 x 22 = 1,408
    assert ie.attention_chunk_tokens(64, 4096, ie.KV_BF16) == 192
    assert ie.attention_chunk_tokens(64, 2880, ie.KV_F16) == 128   # 64 x 15 < 1,024
    assert ie.attention_chunk_tokens(48, 2049, ie.KV_F16) == 128   # 48 x 11
    assert ie.attention_chunk_tokens(1, 32768, ie.KV_F16) == 64    # 1 x 512 <= 512
    assert ie.attention_chunk_tokens(1, 8192, ie.KV_BF16) == 64     # 1 x 128
    assert ie.attention_chunk_tokens(2, 32768, ie.KV_BF16) == 128   # 2 x 512 > 512
    assert ie.attention_chunk_tokens(16, 4096, ie.KV_F16) == 128    # 16 x 64 > 512
    assert ie.attention_chunk_tokens(8, 131072, ie.KV_BF16) == 192  # 8 x 683
    assert ie.attention_chunk_tokens(64, 4096, ie.KV_F32) == 192
    assert ie.attention_chunk_tokens(48, 2049, ie.KV_F32) == 128   # 48 x 11 < 1,024
    assert ie.attention_chunk_tokens(1, 32768, ie.KV_F32) == 64
    assert ie.attention_chunk_tokens(1, 1, ie.KV_F32) == 32
    n = ie.lib().ie_hip_attention_workspace_bytes(64, 14, 64, 8)
    assert n >= 64 * 14 * 8 * 66 * 4


def test_switches_and_trace_ranges(ie):
    """The process-wide switches return the previous setting and ignore unknown values;
    ROCTX ranges push and pop without a device (and a null name pushes nothing)."""
    assert ie.set_prefill_rounding(ie.PREFILL_SPLIT) == ie.PREFILL_SINGLE
    assert ie.set_prefill_rounding(7) == ie.PREFILL_SPLIT  # unknown: kept
    assert ie.set_prefill_rounding(ie.PREFILL_SINGLE) == ie.PREFILL_SPLIT
    assert ie.set_attention_impl(ie.IMPL_VALU) == ie.IMPL_AUTO
    assert ie.set_attention_impl(ie.IMPL_AUTO) == ie.IMPL_VALU
    L = ie.lib()
    L.ie_hip_range_push(b"outer")
    L.ie_hip_range_push(b"inner")
    L.ie_hip_range_push(None)
    L.ie_hip_range_pop()
    L.ie_hip_range_pop()
