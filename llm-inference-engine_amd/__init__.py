"""Host-side Python mirror of the gfx950 paged KV-cache library (libie_hip.so).

The library's C ABI is declared in include/ie_hip.h; this module binds it with
ctypes and offers the reference's kernel-launcher interface
(src/cuda/kernels.cuh:69-102) over torch tensors, plus the page allocator
(src/cuda/cuda_runner.cu:191-313) as a class. torch supplies device memory
and streams only; all compute happens in the HIP kernels. Nothing here falls
back to a CPU implementation: every entry point raises if libie_hip.so is
missing or a call fails.

The package directory name is not an identifier; load it with ``load()`` from
``__graft_entry__`` or import it through importlib (tests do).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libie_hip.so")
PAGE_SIZE = 16
KV_F32, KV_F16, KV_BF16 = 0, 1, 2
KV_NAMES = {"f32": KV_F32, "f16": KV_F16, "bf16": KV_BF16}

# Status codes (include/ie_hip.h).
OK, EINVAL, ELAUNCH, EFULL, ERANGE, ESEQ = 0, 1, 2, 3, 4, 5


class IeHipError(RuntimeError):
    """A libie_hip call returned a nonzero status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class KvLayout(ctypes.Structure):
    """ie_kv_layout: the reference's KvLayout (src/cuda/kernels.cuh:33-38) + pool size."""

    _fields_ = [("tables", ctypes.c_void_p), ("max_pages", ctypes.c_int32),
                ("page_size", ctypes.c_int32), ("kv_dtype", ctypes.c_int32),
                ("num_pages", ctypes.c_int32)]


class Matrix(ctypes.Structure):
    """ie_matrix: the reference's DeviceMatrix (src/cuda/kernels.cuh:40-46), BF16 bits or
    INT8 values with one f32 scale per row."""

    _fields_ = [("data", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("int8", ctypes.c_int32),
                ("rows", ctypes.c_int32), ("cols", ctypes.c_int32)]


_vp, _i, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
_SIGS = {
    "ie_hip_last_error": (ctypes.c_char_p, []),
    "ie_hip_version": (ctypes.c_char_p, []),
    "ie_hip_set_attention_impl": (_i, [_i]),
    "ie_hip_rope_table": (_i, [_vp, _i, _i, _f]),
    "ie_hip_set_prefill_rounding": (_i, [_i]),
    "ie_hip_range_push": (None, [ctypes.c_char_p]),
    "ie_hip_range_pop": (None, []),
    "ie_hip_rope_and_cache": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, KvLayout, _i, _i,
                                   _i, _vp]),
    "ie_hip_attention_chunk_tokens": (_i, [_i, _i, _i]),
    "ie_hip_attention_chunks": (_i, [_i, _i]),
    "ie_hip_attention_workspace_bytes": (ctypes.c_size_t, [_i, _i, _i, _i]),
    "ie_hip_attention": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _vp, KvLayout, _i, _i, _vp, _i, _i, _i,
                              _vp]),
    "ie_hip_attention_noalloc": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _vp, KvLayout, _i, _i, _i, _i,
                                      _i, _vp]),
    "ie_hip_attention_plan_ints": (ctypes.c_size_t, [_i, _i, _i]),
    "ie_hip_attention_plan": (_i, [_vp, ctypes.c_size_t, _i, _vp, _vp, _vp, _i, _i, _i, _i]),
    "ie_hip_attention_planned": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _vp, KvLayout, _i, _i, _vp, _vp,
                                      ctypes.c_size_t, _i, _i, _i, _vp]),
    "ie_hip_rope_cache_attention_planned": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp,
                                                 _vp, KvLayout, _i, _i, _vp, _vp, ctypes.c_size_t,
                                                 _i, _i, _i, _vp]),
    "ie_hip_rope_cache_attention_supported": (_i, [_i, _i, _i, _i, _i]),
    "ie_hip_rope_cache_attention": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp,
                                         KvLayout, _i, _i, _vp, _i, _i, _i, _vp]),
    "ie_hip_attention_prefill_supported": (_i, [_i, _i, _i]),
    "ie_hip_attention_prefill": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _vp, KvLayout, _i, _i, _i, _vp]),
    "ie_hip_rope_cache_attention_prefill_supported": (_i, [_i, _i, _i, _i]),
    "ie_hip_rope_cache_attention_prefill": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp,
                                                 _vp, KvLayout, _i, _i, _i, _vp]),
    "ie_hip_gather_rows": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "ie_hip_gather_kv": (_i, [_vp, _vp, KvLayout, _i, _i, _i, _vp]),
    "ie_hip_argmax_rows": (_i, [_vp, _vp, _i, _i, _vp]),
    "ie_hip_embedding": (_i, [_vp, _vp, Matrix, _i, _vp]),
    "ie_hip_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _f, _vp]),
    "ie_hip_matmul": (_i, [_vp, _vp, Matrix, _vp, _i, _i, _vp]),
    "ie_hip_gate_up_silu": (_i, [_vp, _vp, Matrix, Matrix, _i, _vp]),
    "ie_hip_qkv_proj": (_i, [_vp, _vp, _vp, _vp, Matrix, _vp, _i, _i, _i, _vp]),
    "ie_hip_rmsnorm_qkv_proj": (_i, [_vp, _vp, _vp, _vp, _vp, _f, Matrix, _vp, _i, _i, _i, _vp]),
    "ie_hip_rmsnorm_gate_up_silu": (_i, [_vp, _vp, _vp, _f, Matrix, Matrix, _i, _vp]),
    "ie_pages_create": (_vp, [_i, _i, _i]),
    "ie_pages_destroy": (None, [_vp]),
    "ie_pages_open_sequence": (_i, [_vp]),
    "ie_pages_close_sequence": (_i, [_vp, _i]),
    "ie_pages_ensure": (_i, [_vp, _i, _i]),
    "ie_pages_sequence_length": (_i, [_vp, _i]),
    "ie_pages_set_sequence_length": (_i, [_vp, _i, _i]),
    "ie_pages_sequence_pages": (_i, [_vp, _i, _vp, _i]),
    "ie_pages_total_pages": (_i, [_vp]),
    "ie_pages_free_pages": (_i, [_vp]),
    "ie_pages_max_batch": (_i, [_vp]),
    "ie_pages_max_seq_len": (_i, [_vp]),
    "ie_pages_max_pages_per_seq": (_i, [_vp]),
    "ie_pages_host_tables": (_vp, [_vp]),
    "ie_pages_upload_tables": (_i, [_vp, _vp, _vp, _vp]),
    "ie_pages_for": (_i, [_i]),
}
EXPORTED = tuple(_SIGS)

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded libie_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(there is no fallback implementation)")
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def last_error() -> str:
    return lib().ie_hip_last_error().decode()


def _check(rc: int) -> None:
    if rc != OK:
        raise IeHipError(rc, last_error())


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream=None) -> int:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _dtype_code(t) -> int:
    import torch
    return {torch.float32: KV_F32, torch.float16: KV_F16, torch.bfloat16: KV_BF16}[t.dtype]


def layout(tables, max_pages: int, num_pages: int, kv_dtype: int) -> KvLayout:
    return KvLayout(tables.data_ptr(), max_pages, PAGE_SIZE, kv_dtype, num_pages)


def torch_kv_dtype(kv_dtype: int):
    import torch
    return {KV_F32: torch.float32, KV_F16: torch.float16, KV_BF16: torch.bfloat16}[kv_dtype]


IMPL_AUTO, IMPL_VALU, IMPL_MFMA = 0, 1, 2


def set_attention_impl(impl: int) -> int:
    """Process-wide attention kernel choice (AUTO / VALU / MFMA); returns the previous one."""
    return int(lib().ie_hip_set_attention_impl(impl))


PREFILL_SINGLE, PREFILL_SPLIT = 0, 1


def set_prefill_rounding(mode: int) -> int:
    """Process-wide operand precision of the f16 matrix-core prefill (SINGLE: q and P
    rounded once to f16; SPLIT: hi + lo halves); returns the previous one."""
    return int(lib().ie_hip_set_prefill_rounding(mode))


# ------------------------------------------------------------ kernels ----
def rope_table(n_pos: int, head_dim: int, theta: float):
    """Host RoPE table [n_pos, head_dim] (cos | sin) as a CPU float32 tensor."""
    import torch
    t = torch.empty((n_pos, head_dim), dtype=torch.float32)
    _check(lib().ie_hip_rope_table(t.data_ptr(), n_pos, head_dim, theta))
    return t


def rope_and_cache(q, k, v, k_pool, v_pool, table, row_pos, row_seq, tables, max_pages: int,
                   n_heads: int, n_kv_heads: int, head_dim: int, stream=None) -> None:
    """rope_and_cache (src/cuda/kernels.cuh:72-74); q may be None (append only)."""
    T = row_pos.numel()
    kv = layout(tables, max_pages, k_pool.numel() // (PAGE_SIZE * n_kv_heads * head_dim),
                _dtype_code(k_pool))
    _check(lib().ie_hip_rope_and_cache(_ptr(q), _ptr(k), _ptr(v), _ptr(k_pool), _ptr(v_pool),
                                       _ptr(table), table.shape[0], T, _ptr(row_pos),
                                       _ptr(row_seq), kv, n_heads, n_kv_heads, head_dim,
                                       _stream(stream)))


def attention_chunk_tokens(T: int, max_context: int, kv_dtype: int = KV_F16) -> int:
    """Chunk size for T rows of up to max_context tokens (kv_dtype picks the kernel)."""
    return int(lib().ie_hip_attention_chunk_tokens(T, max_context, kv_dtype))


def attention_chunks(context: int, chunk_tokens: int) -> int:
    return int(lib().ie_hip_attention_chunks(context, chunk_tokens))


def attention_workspace(T: int, n_heads: int, head_dim: int, num_chunks: int, device="cuda"):
    import torch
    n = int(lib().ie_hip_attention_workspace_bytes(T, n_heads, head_dim, num_chunks))
    return torch.zeros(max(n, 256), dtype=torch.uint8, device=device)


def attention(out, q, k_pool, v_pool, row_pos, row_seq, tables, max_pages: int, num_chunks: int,
              chunk_tokens: int, workspace, n_heads: int, n_kv_heads: int, head_dim: int,
              stream=None) -> None:
    """Flash-decoding attention (src/cuda/kernels.cuh:84-87)."""
    T = row_pos.numel()
    kv = layout(tables, max_pages, k_pool.numel() // (PAGE_SIZE * n_kv_heads * head_dim),
                _dtype_code(k_pool))
    _check(lib().ie_hip_attention(_ptr(out), _ptr(q), _ptr(k_pool), _ptr(v_pool), T, _ptr(row_pos),
                                  _ptr(row_seq), kv, num_chunks, chunk_tokens, _ptr(workspace),
                                  n_heads, n_kv_heads, head_dim, _stream(stream)))


NOALLOC_SCRATCH_BYTES = 16 << 20  # IE_HIP_NOALLOC_SCRATCH_BYTES


def attention_noalloc(out, q, k_pool, v_pool, row_pos, row_seq, tables, max_pages: int,
                      num_chunks: int, chunk_tokens: int, n_heads: int, n_kv_heads: int,
                      head_dim: int, stream=None) -> None:
    """attention() with the library's fixed device scratch in place of a workspace."""
    T = row_pos.numel()
    kv = layout(tables, max_pages, k_pool.numel() // (PAGE_SIZE * n_kv_heads * head_dim),
                _dtype_code(k_pool))
    _check(lib().ie_hip_attention_noalloc(_ptr(out), _ptr(q), _ptr(k_pool), _ptr(v_pool), T,
                                          _ptr(row_pos), _ptr(row_seq), kv, num_chunks,
                                          chunk_tokens, n_heads, n_kv_heads, head_dim,
                                          _stream(stream)))


def attention_plan_ints(T: int, num_chunks: int, chunk_tokens: int) -> int:
    return int(lib().ie_hip_attention_plan_ints(T, num_chunks, chunk_tokens))


def attention_plan(row_pos, row_seq, tables, num_chunks: int, chunk_tokens: int):
    """The decode work list for one launch, built on the host from host copies (numpy
    int32) of the rows' positions and sequences and of the block table [seqs, max_pages];
    returns it as a numpy int32 array (copy it to the device for attention_planned)."""
    import numpy as np
    row_pos = np.ascontiguousarray(row_pos, dtype=np.int32)
    row_seq = np.ascontiguousarray(row_seq, dtype=np.int32)
    tables = np.ascontiguousarray(tables, dtype=np.int32)
    T = row_pos.size
    n = int(lib().ie_hip_attention_plan_ints(max(T, 1), num_chunks, chunk_tokens))
    if n == 0:
        raise IeHipError(EINVAL, "attention_plan: bad chunk arguments")
    plan = np.zeros(n, np.int32)
    _check(lib().ie_hip_attention_plan(plan.ctypes.data, n, T, row_pos.ctypes.data,
                                       row_seq.ctypes.data, tables.ctypes.data, tables.shape[0],
                                       tables.shape[1], num_chunks, chunk_tokens))
    return plan


def attention_planned(out, q, k_pool, v_pool, row_pos, row_seq, tables, max_pages: int,
                      num_chunks: int, chunk_tokens: int, workspace, plan, n_heads: int,
                      n_kv_heads: int, head_dim: int, stream=None) -> None:
    """attention() with a device copy of attention_plan()'s work list."""
    T = row_pos.numel()
    kv = layout(tables, max_pages, k_pool.numel() // (PAGE_SIZE * n_kv_heads * head_dim),
                _dtype_code(k_pool))
    _check(lib().ie_hip_attention_planned(_ptr(out), _ptr(q), _ptr(k_pool), _ptr(v_pool), T,
                                          _ptr(row_pos), _ptr(row_seq), kv, num_chunks,
                                          chunk_tokens, _ptr(workspace), _ptr(plan), plan.numel(),
                                          n_heads, n_kv_heads, head_dim, _stream(stream)))


def rope_cache_attention_planned(out, q, k, v, k_pool, v_pool, table, row_pos, row_seq, tables,
                                 max_pages: int, num_chunks: int, chunk_tokens: int, workspace,
                                 plan, n_heads: int, n_kv_heads: int, head_dim: int,
                                 stream=None) -> None:
    """rope_cache_attention() with a device copy of attention_plan()'s work list."""
    T = row_pos.numel()
    kv = layout(tables, max_pages, k_pool.numel() // (PAGE_SIZE * n_kv_heads * head_dim),
                _dtype_code(k_pool))
    _check(lib().ie_hip_rope_cache_attention_planned(
        _ptr(out), _ptr(q), _ptr(k), _ptr(v), _ptr(k_pool), _ptr(v_pool), _ptr(table),
        table.shape[0], T, _ptr(row_pos), _ptr(row_seq), kv, num_chunks, chunk_tokens,
        _ptr(workspace), _ptr(plan), plan.numel(), n_heads, n_kv_heads, head_dim,
        _stream(stream)))


def rope_cache_attention_supported(kv_dtype: int, n_heads: int, n_kv_heads: int, head_dim: int,
                                   chunk_tokens: int) -> bool:
    return bool(lib().ie_hip_rope_cache_attention_supported(kv_dtype, n_heads, n_kv_heads,
                                                            head_dim, chunk_tokens))


def rope_cache_attention(out, q, k, v, k_pool, v_pool, table, row_pos, row_seq, tables,
                         max_pages: int, num_chunks: int, chunk_tokens: int, workspace,
                         n_heads: int, n_kv_heads: int, head_dim: int, stream=None) -> None:
    """rope_and_cache + attention of one decode step in one launch (q is not modified)."""
    T = row_pos.numel()
    kv = layout(tables, max_pages, k_pool.numel() // (PAGE_SIZE * n_kv_heads * head_dim),
                _dtype_code(k_pool))
    _check(lib().ie_hip_rope_cache_attention(_ptr(out), _ptr(q), _ptr(k), _ptr(v), _ptr(k_pool),
                                             _ptr(v_pool), _ptr(table), table.shape[0], T,
                                             _ptr(row_pos), _ptr(row_seq), kv, num_chunks,
                                             chunk_tokens, _ptr(workspace), n_heads, n_kv_heads,
                                             head_dim, _stream(stream)))


def rope_cache_attention_prefill_supported(kv_dtype: int, n_heads: int, n_kv_heads: int,
                                           head_dim: int) -> bool:
    return bool(lib().ie_hip_rope_cache_attention_prefill_supported(kv_dtype, n_heads, n_kv_heads,
                                                                    head_dim))


def rope_cache_attention_prefill(out, q, k, v, k_pool, v_pool, table, row_pos, row_seq, tables,
                                 max_pages: int, n_heads: int, n_kv_heads: int, head_dim: int,
                                 stream=None) -> None:
    """rope_and_cache + attention_prefill of one prompt chunk, q rotated inside the prefill
    kernel (q is not modified)."""
    T = row_pos.numel()
    kv = layout(tables, max_pages, k_pool.numel() // (PAGE_SIZE * n_kv_heads * head_dim),
                _dtype_code(k_pool))
    _check(lib().ie_hip_rope_cache_attention_prefill(_ptr(out), _ptr(q), _ptr(k), _ptr(v),
                                                     _ptr(k_pool), _ptr(v_pool), _ptr(table),
                                                     table.shape[0], T, _ptr(row_pos),
                                                     _ptr(row_seq), kv, n_heads, n_kv_heads,
                                                     head_dim, _stream(stream)))


def attention_prefill_supported(n_heads: int, n_kv_heads: int, head_dim: int) -> bool:
    return bool(lib().ie_hip_attention_prefill_supported(n_heads, n_kv_heads, head_dim))


def attention_prefill(out, q, k_pool, v_pool, row_pos, row_seq, tables, max_pages: int,
                      n_heads: int, n_kv_heads: int, head_dim: int, stream=None) -> None:
    """Prompt attention (src/cuda/kernels.cuh:93-96)."""
    T = row_pos.numel()
    kv = layout(tables, max_pages, k_pool.numel() // (PAGE_SIZE * n_kv_heads * head_dim),
                _dtype_code(k_pool))
    _check(lib().ie_hip_attention_prefill(_ptr(out), _ptr(q), _ptr(k_pool), _ptr(v_pool), T,
                                          _ptr(row_pos), _ptr(row_seq), kv, n_heads, n_kv_heads,
                                          head_dim, _stream(stream)))


def gather_rows(dst, src, rows, stream=None) -> None:
    """dst[r] = src[rows[r]] (src/cuda/kernels.cuh:101-102)."""
    _check(lib().ie_hip_gather_rows(_ptr(dst), _ptr(src), _ptr(rows), rows.numel(), src.shape[-1],
                                    _stream(stream)))


def argmax_rows(out, logits, stream=None) -> None:
    """out[r] = first index of the maximum of logits[r] (src/cuda/kernels.cuh:106)."""
    _check(lib().ie_hip_argmax_rows(_ptr(out), _ptr(logits), logits.shape[0], logits.shape[1],
                                    _stream(stream)))


def matrix(data, scale=None) -> Matrix:
    """An ie_matrix over a device tensor of BF16 bits (int16/uint16/bfloat16) or INT8
    values [rows, cols] and, for INT8, its f32 row scales."""
    import torch
    int8 = data.dtype == torch.int8
    if int8 and scale is None:
        raise ValueError("INT8 weights need their row scales")
    return Matrix(data.data_ptr(), scale.data_ptr() if int8 else None, int(int8), data.shape[0],
                  data.shape[1])


def embedding(x, ids, e: Matrix, stream=None) -> None:
    """x[t] = E[ids[t]] widened to f32 (src/cuda/kernels.cuh:48-49)."""
    _check(lib().ie_hip_embedding(_ptr(x), _ptr(ids), e, ids.numel(), _stream(stream)))


def rmsnorm(y, x, weight, eps: float, stream=None) -> None:
    """y = x / rms(x) * weight per row (src/cuda/kernels.cuh:51-53)."""
    dim = weight.numel()
    _check(lib().ie_hip_rmsnorm(_ptr(y), _ptr(x), _ptr(weight), x.numel() // dim, dim, eps,
                                _stream(stream)))


def matmul(y, x, w: Matrix, bias=None, accumulate: bool = False, stream=None) -> None:
    """y (+)= x . W^T * scale + bias (src/cuda/kernels.cuh:55-62)."""
    _check(lib().ie_hip_matmul(_ptr(y), _ptr(x), w, _ptr(bias), x.numel() // w.cols,
                               int(accumulate), _stream(stream)))


def qkv_proj(q, k, v, x, w_qkv: Matrix, b_qkv=None, stream=None) -> None:
    """q, k, v = x . [Wq; Wk; Wv]^T + [bq; bk; bv] in one launch."""
    q_dim, kv_dim = q.shape[-1], k.shape[-1]
    _check(lib().ie_hip_qkv_proj(_ptr(q), _ptr(k), _ptr(v), _ptr(x), w_qkv, _ptr(b_qkv),
                                 x.numel() // w_qkv.cols, q_dim, kv_dim, _stream(stream)))


def gate_up_silu(out, x, w_gate: Matrix, w_up: Matrix, stream=None) -> None:
    """out = silu(x . Wg^T) * (x . Wu^T) (src/cuda/kernels.cuh:64-66)."""
    _check(lib().ie_hip_gate_up_silu(_ptr(out), _ptr(x), w_gate, w_up, x.numel() // w_gate.cols,
                                     _stream(stream)))


def rmsnorm_qkv_proj(q, k, v, x, norm, eps: float, w_qkv: Matrix, b_qkv=None,
                     stream=None) -> None:
    """qkv_proj(rmsnorm(x, norm, eps)) in one launch (no reference counterpart)."""
    q_dim, kv_dim = q.shape[-1], k.shape[-1]
    _check(lib().ie_hip_rmsnorm_qkv_proj(_ptr(q), _ptr(k), _ptr(v), _ptr(x), _ptr(norm), eps,
                                         w_qkv, _ptr(b_qkv), x.numel() // w_qkv.cols, q_dim,
                                         kv_dim, _stream(stream)))


def rmsnorm_gate_up_silu(out, x, norm, eps: float, w_gate: Matrix, w_up: Matrix,
                         stream=None) -> None:
    """gate_up_silu(rmsnorm(x, norm, eps)) in one launch (no reference counterpart)."""
    _check(lib().ie_hip_rmsnorm_gate_up_silu(_ptr(out), _ptr(x), _ptr(norm), eps, w_gate, w_up,
                                             x.numel() // w_gate.cols, _stream(stream)))


def gather_kv(dst, pool, tables, max_pages: int, seq: int, length: int, kv_dim: int,
              stream=None) -> None:
    """Contiguous fp32 copy of one sequence's paged rows."""
    kv = layout(tables, max_pages, pool.numel() // (PAGE_SIZE * kv_dim), _dtype_code(pool))
    _check(lib().ie_hip_gather_kv(_ptr(dst), _ptr(pool), kv, seq, length, kv_dim, _stream(stream)))


# -------------------------------------------------------- page allocator ----
class PagePool:
    """The BatchRunner page allocator (src/cuda/cuda_runner.cu:191-313), host side."""

    def __init__(self, num_pages: int, max_batch: int, max_seq_len: int):
        self._h = lib().ie_pages_create(num_pages, max_batch, max_seq_len)
        if not self._h:
            raise IeHipError(EINVAL, last_error())

    def close(self) -> None:
        if self._h:
            lib().ie_pages_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def open_sequence(self) -> int:
        return int(lib().ie_pages_open_sequence(self._h))

    def close_sequence(self, seq: int) -> None:
        _check(lib().ie_pages_close_sequence(self._h, seq))

    def ensure(self, seq: int, length: int) -> None:
        _check(lib().ie_pages_ensure(self._h, seq, length))

    def sequence_length(self, seq: int) -> int:
        return int(lib().ie_pages_sequence_length(self._h, seq))

    def set_sequence_length(self, seq: int, length: int) -> None:
        _check(lib().ie_pages_set_sequence_length(self._h, seq, length))

    def pages(self, seq: int) -> list[int]:
        n = lib().ie_pages_sequence_pages(self._h, seq, None, 0)
        buf = (ctypes.c_int32 * max(n, 1))()
        lib().ie_pages_sequence_pages(self._h, seq, buf, n)
        return list(buf[:n])

    @property
    def total_pages(self) -> int:
        return int(lib().ie_pages_total_pages(self._h))

    @property
    def free_pages(self) -> int:
        return int(lib().ie_pages_free_pages(self._h))

    @property
    def max_batch(self) -> int:
        return int(lib().ie_pages_max_batch(self._h))

    @property
    def max_seq_len(self) -> int:
        return int(lib().ie_pages_max_seq_len(self._h))

    @property
    def max_pages_per_seq(self) -> int:
        return int(lib().ie_pages_max_pages_per_seq(self._h))

    def host_tables(self) -> list[int]:
        n = self.max_batch * self.max_pages_per_seq
        p = lib().ie_pages_host_tables(self._h)
        return list((ctypes.c_int32 * n).from_address(p))

    def upload_tables(self, device_tables, stream=None) -> bool:
        up = ctypes.c_int(0)
        _check(lib().ie_pages_upload_tables(self._h, device_tables.data_ptr(), _stream(stream),
                                            ctypes.byref(up)))
        return bool(up.value)


def pages_for(tokens: int) -> int:
    return int(lib().ie_pages_for(tokens))
