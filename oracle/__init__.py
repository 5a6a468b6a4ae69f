"""CPU oracle for the paged KV-cache path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker. The product
library (``llm-inference-engine_amd``) never imports it.

Two native libraries sit behind these wrappers:

* ``liborc.so`` -- this directory's own C++ restatement of the reference CPU
  path (``oracle.cpp``; every function cites the reference file:line it
  follows, ``oracle.h`` says what pins it).
* ``_ref/libieref.so`` -- the reference's own ``src/ops.cpp`` and
  ``src/threadpool.cpp`` compiled in place by ``oracle/Makefile``. Present only
  where it was built; used to pin the restatement and as the CPU baseline.

Also here: the LIFO page allocator restated in Python (``allocator.py``) and
the reference's error metric (``compare``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORC_PATH = os.path.join(HERE, "liborc.so")
REF_PATH = os.path.join(HERE, "_ref", "libieref.so")

KV_F32, KV_F16, KV_BF16 = 0, 1, 2
KV_NP = {KV_F32: np.float32, KV_F16: np.uint16, KV_BF16: np.uint16}

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p


def build() -> None:
    """Compile liborc.so (and _ref/libieref.so when the reference is present)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class _Lib:
    def __init__(self, path: str):
        self.path = path
        self.lib = ctypes.CDLL(path)


_orc = None
_ref = None


def orc() -> ctypes.CDLL:
    global _orc
    if _orc is None:
        if not os.path.exists(ORC_PATH):
            build()
        lib = ctypes.CDLL(ORC_PATH)
        lib.orc_f32_to_f16.restype = ctypes.c_uint16
        lib.orc_f32_to_f16.argtypes = [ctypes.c_float]
        lib.orc_f16_to_f32.restype = ctypes.c_float
        lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        lib.orc_bf16_to_f32.restype = ctypes.c_float
        lib.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_kv_offset.restype = ctypes.c_size_t
        lib.orc_compare.restype = ctypes.c_double
        lib.orc_physical_cores.restype = ctypes.c_int
        _orc = lib
    return _orc


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref() -> ctypes.CDLL:
    """The reference's own CPU ops (oracle/_ref). Raises if it was not built."""
    global _ref
    if _ref is None:
        if not ref_available():
            raise FileNotFoundError(f"{REF_PATH} not built (needs the reference checkout)")
        _ref = ctypes.CDLL(REF_PATH)
        _ref.ref_num_threads.restype = ctypes.c_int
        _ref.ref_physical_cores.restype = ctypes.c_int
    return _ref


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# --------------------------------------------------------------- rope ----
def inv_freq(head_dim: int, theta: float) -> np.ndarray:
    out = np.empty(head_dim // 2, np.float32)
    orc().orc_inv_freq(_ptr(out), ctypes.c_int(head_dim), ctypes.c_float(theta))
    return out


def rope_table(n_pos: int, head_dim: int, theta: float) -> np.ndarray:
    out = np.empty((n_pos, head_dim), np.float32)
    orc().orc_rope_table(_ptr(out), ctypes.c_int(n_pos), ctypes.c_int(head_dim), ctypes.c_float(theta))
    return out


def rope(x: np.ndarray, n_heads: int, head_dim: int, pos0: int, theta: float) -> np.ndarray:
    y = _c(x, np.float32).copy()
    T = y.size // (n_heads * head_dim)
    orc().orc_rope(_ptr(y), T, n_heads, head_dim, pos0, ctypes.c_float(theta))
    return y


def ref_rope(x: np.ndarray, n_heads: int, head_dim: int, pos0: int, theta: float) -> np.ndarray:
    y = _c(x, np.float32).copy()
    T = y.size // (n_heads * head_dim)
    ref().ref_rope(_ptr(y), T, n_heads, head_dim, pos0, ctypes.c_float(theta))
    return y


# ----------------------------------------------------- softmax / attn ----
def softmax(x: np.ndarray) -> np.ndarray:
    y = _c(x, np.float32).copy()
    orc().orc_softmax(_ptr(y), y.size)
    return y


def ref_softmax(x: np.ndarray) -> np.ndarray:
    y = _c(x, np.float32).copy()
    ref().ref_softmax(_ptr(y), y.size)
    return y


def attention(q, k, v, pos0, n_heads, n_kv_heads, head_dim, threads=1) -> np.ndarray:
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    T = q.size // (n_heads * head_dim)
    out = np.empty_like(q)
    orc().orc_attention(_ptr(out), _ptr(q), _ptr(k), _ptr(v), T, pos0, n_heads, n_kv_heads,
                        head_dim, threads)
    return out


def ref_attention(q, k, v, pos0, n_heads, n_kv_heads, head_dim) -> np.ndarray:
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    T = q.size // (n_heads * head_dim)
    out = np.empty_like(q)
    ref().ref_attention(_ptr(out), _ptr(q), _ptr(k), _ptr(v), T, pos0, n_heads, n_kv_heads, head_dim)
    return out


def physical_cores() -> int:
    return int(orc().orc_physical_cores())


# ------------------------------------------------------ 16-bit rounding ----
def round_to_kv(x: np.ndarray, kv_dtype: int) -> np.ndarray:
    """fp32 -> pool element type (uint16 bit patterns for f16/bf16)."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, KV_NP[kv_dtype])
    orc().orc_round_to_kv(_ptr(out), _ptr(x), ctypes.c_size_t(x.size), kv_dtype)
    return out


def widen_kv(x: np.ndarray, kv_dtype: int) -> np.ndarray:
    x = _c(x, KV_NP[kv_dtype])
    out = np.empty(x.shape, np.float32)
    orc().orc_widen_kv(_ptr(out), _ptr(x), ctypes.c_size_t(x.size), kv_dtype)
    return out


# ------------------------------------------------------------ paging ----
def kv_offset(tables, max_pages, page_size, seq, pos, kv_dim) -> int:
    t = _c(tables, np.int32)
    return int(orc().orc_kv_offset(_ptr(t), max_pages, page_size, seq, pos, kv_dim))


def rope_append_paged(q, k, v, k_pool, v_pool, kv_dtype, row_pos, row_seq, tables, max_pages,
                      n_heads, n_kv_heads, head_dim, theta, page_size=16):
    """Returns (q rotated, k_pool, v_pool) -- the pools are updated copies."""
    q = _c(q, np.float32).copy()
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    kp = _c(k_pool, KV_NP[kv_dtype]).copy()
    vp = _c(v_pool, KV_NP[kv_dtype]).copy()
    rp = _c(row_pos, np.int32)
    rs = _c(row_seq, np.int32)
    tb = _c(tables, np.int32)
    orc().orc_rope_append_paged(_ptr(q), _ptr(k), _ptr(v), _ptr(kp), _ptr(vp), kv_dtype, rp.size,
                                _ptr(rp), _ptr(rs), _ptr(tb), max_pages, page_size, n_heads,
                                n_kv_heads, head_dim, ctypes.c_float(theta))
    return q, kp, vp


def gather_kv(pool, kv_dtype, tables, max_pages, seq, length, kv_dim, page_size=16) -> np.ndarray:
    p = _c(pool, KV_NP[kv_dtype])
    tb = _c(tables, np.int32)
    out = np.empty((length, kv_dim), np.float32)
    orc().orc_gather_kv(_ptr(out), _ptr(p), kv_dtype, _ptr(tb), max_pages, page_size, seq, length,
                        kv_dim)
    return out


def paged_attention(q, k_pool, v_pool, kv_dtype, row_pos, row_seq, tables, max_pages, n_heads,
                    n_kv_heads, head_dim, threads=1, page_size=16) -> np.ndarray:
    q = _c(q, np.float32)
    kp = _c(k_pool, KV_NP[kv_dtype])
    vp = _c(v_pool, KV_NP[kv_dtype])
    rp = _c(row_pos, np.int32)
    rs = _c(row_seq, np.int32)
    tb = _c(tables, np.int32)
    out = np.empty((rp.size, n_heads * head_dim), np.float32)
    orc().orc_paged_attention(_ptr(out), _ptr(q), _ptr(kp), _ptr(vp), kv_dtype, rp.size, _ptr(rp),
                              _ptr(rs), _ptr(tb), max_pages, page_size, n_heads, n_kv_heads,
                              head_dim, threads)
    return out


def gather_rows(src: np.ndarray, rows) -> np.ndarray:
    src = _c(src, np.float32)
    rows = _c(rows, np.int32)
    dim = src.shape[-1]
    out = np.empty((rows.size, dim), np.float32)
    orc().orc_gather_rows(_ptr(out), _ptr(src), _ptr(rows), rows.size, dim)
    return out


def compare(got, want):
    """The reference's metric: (max|got-want| / max|want|, max abs err, worst index)."""
    g = _c(got, np.float32).ravel()
    w = _c(want, np.float32).ravel()
    assert g.size == w.size
    mae = ctypes.c_double()
    worst = ctypes.c_size_t()
    rel = orc().orc_compare(_ptr(g), _ptr(w), ctypes.c_size_t(w.size), ctypes.byref(mae),
                            ctypes.byref(worst))
    return float(rel), float(mae.value), int(worst.value)


# ------------------------------------------------ the decode step's layer ----
W_F32, W_BF16, W_I8 = 0, 1, 2  # weight formats (src/matrix.h:4-12)


def _weight_array(w: np.ndarray, w_dtype: int) -> np.ndarray:
    return _c(w, {W_F32: np.float32, W_BF16: np.uint16, W_I8: np.int8}[w_dtype])


def matmul(x, w, w_dtype: int, scale=None, bias=None, threads: int = 8) -> np.ndarray:
    """y = x . W^T (* row scale for I8) + bias: the reference's scalar matmul
    (src/matrix.cpp:131-146,247-265). x: [T, cols]; w: [rows, cols] as f32, bf16 bits
    (uint16) or int8."""
    x = _c(x, np.float32)
    w = _weight_array(w, w_dtype)
    rows, cols = w.shape
    T = x.size // cols
    y = np.empty((T, rows), np.float32)
    sc = None if scale is None else _c(scale, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    orc().orc_matmul(_ptr(y), _ptr(x), _ptr(w), w_dtype, None if sc is None else _ptr(sc),
                     None if b is None else _ptr(b), T, rows, cols, threads)
    return y


def quantize_i8(w) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric int8 quantization (src/matrix.cpp:84-97): (q [rows, cols], scale [rows])."""
    w = _c(w, np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    orc().orc_quantize_i8(_ptr(q), _ptr(s), _ptr(w), rows, cols)
    return q, s


def row_to_f32(w, w_dtype: int, r: int, scale=None) -> np.ndarray:
    """Row r widened to f32 (src/matrix.cpp:60-67)."""
    w = _weight_array(w, w_dtype)
    out = np.empty(w.shape[1], np.float32)
    sc = None if scale is None else _c(scale, np.float32)
    orc().orc_row_to_f32(_ptr(out), _ptr(w), w_dtype, None if sc is None else _ptr(sc),
                         w.shape[1], r)
    return out


def rmsnorm(x, weight, eps: float) -> np.ndarray:
    """src/ops.cpp:23-32."""
    x = _c(x, np.float32)
    weight = _c(weight, np.float32)
    dim = weight.size
    y = np.empty_like(x)
    orc().orc_rmsnorm(_ptr(y), _ptr(x), _ptr(weight), x.size // dim, dim, ctypes.c_float(eps))
    return y


def silu_mul(gate, up) -> np.ndarray:
    """silu(gate) * up, elementwise (src/ops.cpp:68, src/model.cpp:86)."""
    g = _c(gate, np.float32).copy()
    u = _c(up, np.float32)
    orc().orc_silu_mul(_ptr(g), _ptr(u), ctypes.c_size_t(g.size))
    return g


def ref_matmul_bf16(x, w_bits, dtype: int, bias=None, kernel: int = 0):
    """The reference's own ie::matmul on a bf16-bits matrix stored as `dtype`
    (0 F32, 1 BF16, 2 I8), kernel 0 scalar / 1 AVX2 (oracle/_ref). Returns
    (y, i8 scales or None, i8 values or None)."""
    x = _c(x, np.float32)
    w = _c(w_bits, np.uint16)
    rows, cols = w.shape
    T = x.size // cols
    y = np.empty((T, rows), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    sc = np.empty(rows, np.float32) if dtype == W_I8 else None
    q = np.empty((rows, cols), np.int8) if dtype == W_I8 else None
    ref().ref_matmul_bf16(_ptr(y), _ptr(x), _ptr(w), dtype, None if b is None else _ptr(b), T,
                          rows, cols, kernel, None if sc is None else _ptr(sc),
                          None if q is None else _ptr(q))
    return y, sc, q


def ref_rmsnorm(x, weight, eps: float) -> np.ndarray:
    x = _c(x, np.float32)
    weight = _c(weight, np.float32)
    y = np.empty_like(x)
    ref().ref_rmsnorm(_ptr(y), _ptr(x), _ptr(weight), x.size // weight.size, weight.size,
                      ctypes.c_float(eps))
    return y


def ref_silu(x: float) -> float:
    f = ref().ref_silu
    f.restype, f.argtypes = ctypes.c_float, [ctypes.c_float]
    return float(f(x))


def ref_row_to_f32(w_bits, dtype: int, r: int) -> np.ndarray:
    w = _c(w_bits, np.uint16)
    out = np.empty(w.shape[1], np.float32)
    ref().ref_row_to_f32(_ptr(out), _ptr(w), dtype, w.shape[0], w.shape[1], r)
    return out
