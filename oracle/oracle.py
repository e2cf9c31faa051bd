"""numpy front end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY. This module is the checker, never the product:
only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import it. Each wrapper names the reference lines its C function restates
(paths relative to the stratorys/metal-infer-rs root).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"

_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)


class _AttnArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("q_stride", ctypes.c_int64 * 3),
        ("k", ctypes.c_void_p),
        ("k_stride", ctypes.c_int64 * 3),
        ("v", ctypes.c_void_p),
        ("v_stride", ctypes.c_int64 * 3),
        ("tokens", ctypes.c_uint32),
        ("q_heads", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("kv_length", ctypes.c_uint32),
        ("causal", ctypes.c_uint32),
        ("query_offset", ctypes.c_uint32),
        ("rows", ctypes.c_void_p),
        ("n_rows", ctypes.c_uint32),
        ("out_f16", ctypes.c_void_p),
        ("out_f32", ctypes.c_void_p),
        ("out_f64", ctypes.c_void_p),
        ("threads", ctypes.c_int),
    ]


_lib = None


def build() -> None:
    """Compile liboracle.so from oracle/attn_oracle.c (the committed recipe)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        handle = ctypes.CDLL(str(_LIB_PATH))
        handle.orc_f32_to_f16.restype = ctypes.c_uint16
        handle.orc_f32_to_f16.argtypes = [ctypes.c_float]
        handle.orc_f16_to_f32.restype = ctypes.c_float
        handle.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        handle.orc_f32_to_f16_array.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        handle.orc_f16_to_f32_array.argtypes = [_u16p, _f32p, ctypes.c_size_t]
        handle.orc_xorshift_seed.restype = ctypes.c_uint64
        handle.orc_xorshift_seed.argtypes = [ctypes.c_uint64]
        handle.orc_xorshift_next_f64.restype = ctypes.c_double
        handle.orc_xorshift_next_f64.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        handle.orc_xorshift_jump.restype = ctypes.c_uint64
        handle.orc_xorshift_jump.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        handle.orc_fill_normal_f16.argtypes = [
            ctypes.c_uint64, _u16p, ctypes.c_size_t, ctypes.c_int]
        handle.orc_fill_uniform_u32.argtypes = [
            ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, _u32p, ctypes.c_size_t]
        handle.orc_attention.restype = ctypes.c_int
        handle.orc_attention.argtypes = [ctypes.POINTER(_AttnArgs)]
        handle.orc_qk_norm_rope.restype = ctypes.c_int
        handle.orc_qk_norm_rope.argtypes = [
            _u16p, _u16p, _u16p, _u16p, ctypes.c_uint32, ctypes.c_uint32,
            ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float,
            ctypes.c_float, _u16p, _u16p]
        handle.orc_rms_norm.restype = ctypes.c_int
        handle.orc_rms_norm.argtypes = [_u16p, _u16p, ctypes.c_uint64, ctypes.c_uint32,
                                        ctypes.c_float, _u16p, _f32p]
        handle.orc_rope.restype = ctypes.c_int
        handle.orc_rope.argtypes = [_u16p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                    ctypes.c_uint32, ctypes.c_float, _u16p]
        handle.orc_matmul.restype = ctypes.c_int
        handle.orc_matmul.argtypes = [_u16p, _u16p, ctypes.c_uint32, ctypes.c_uint32,
                                      ctypes.c_uint32, _u16p, _f32p, ctypes.c_int]
        _lib = handle
    return _lib


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


# ----------------------------------------------------------------- f16 ----

def f32_to_f16(values) -> np.ndarray:
    """f32 -> f16 bits, RNE (half::f16::from_f32, context.rs:770)."""
    src = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(src.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(src.ctypes.data_as(_f32p), out.ctypes.data_as(_u16p), src.size)
    return out


def f16_to_f32(bits) -> np.ndarray:
    """f16 bits -> f32 (f16::to_f32, tensor.rs:244)."""
    src = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(src.shape, dtype=np.float32)
    lib().orc_f16_to_f32_array(src.ctypes.data_as(_u16p), out.ctypes.data_as(_f32p), src.size)
    return out


# ----------------------------------------------------------- generator ----

def xorshift_draws(seed: int, count: int) -> np.ndarray:
    """`count` XorShift64 draws in [0, 1) (qwen3.rs:1011-1034)."""
    state = ctypes.c_uint64(lib().orc_xorshift_seed(seed))
    return np.array([lib().orc_xorshift_next_f64(ctypes.byref(state)) for _ in range(count)])


def xorshift_jump(state: int, steps: int) -> int:
    return int(lib().orc_xorshift_jump(state, steps))


def normal_f16(seed: int, shape, threads: int | None = None) -> np.ndarray:
    """Seeded N(0,1) values as f16 bits, filled in logical (C) order."""
    out = np.empty(shape, dtype=np.uint16)
    lib().orc_fill_normal_f16(seed, out.ctypes.data_as(_u16p), out.size,
                              threads or default_threads())
    return out


def uniform_u32(seed: int, lo: int, hi: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    lib().orc_fill_uniform_u32(seed, lo, hi, out.ctypes.data_as(_u32p), n)
    return out


# ----------------------------------------------------------- attention ----

def _strides(array: np.ndarray) -> tuple[int, int, int]:
    if array.ndim != 3 or array.dtype != np.uint16:
        raise ValueError("expected a rank-3 uint16 (f16 bits) array")
    return tuple(s // 2 for s in array.strides)


def attention(q, k, v, *, q_heads: int, kv_heads: int, head_dim: int,
              causal: bool = True, query_offset: int = 0, rows=None,
              want=("f16", "f32"), threads: int | None = None) -> dict:
    """Restatement of attention_reference_f16 (transformer.metal:1579-1612).

    q is [T, Hq, D], k/v are [L, Hkv, D] f16-bit arrays (any strides, so a
    head-major cache can be passed as a transposed view). Returns a dict with
    the requested outputs ("f16" bits, "f32", "f64"), each [rows, Hq, D].
    """
    T, hq, d = q.shape
    L = k.shape[0]
    if hq != q_heads or d != head_dim or k.shape != (L, kv_heads, head_dim) or v.shape != k.shape:
        raise ValueError("attention shapes do not match the configuration")
    row_array = None if rows is None else np.ascontiguousarray(rows, dtype=np.uint32)
    n_rows = T if row_array is None else row_array.size
    out = {}
    if "f16" in want:
        out["f16"] = np.empty((n_rows, hq, d), dtype=np.uint16)
    if "f32" in want:
        out["f32"] = np.empty((n_rows, hq, d), dtype=np.float32)
    if "f64" in want:
        out["f64"] = np.empty((n_rows, hq, d), dtype=np.float64)
    args = _AttnArgs()
    args.q, args.k, args.v = q.ctypes.data, k.ctypes.data, v.ctypes.data
    args.q_stride[:] = _strides(q)
    args.k_stride[:] = _strides(k)
    args.v_stride[:] = _strides(v)
    args.tokens, args.q_heads, args.kv_heads, args.head_dim = T, q_heads, kv_heads, head_dim
    args.kv_length, args.causal, args.query_offset = L, int(bool(causal)), query_offset
    args.rows = row_array.ctypes.data if row_array is not None else None
    args.n_rows = n_rows
    args.out_f16 = out["f16"].ctypes.data if "f16" in out else None
    args.out_f32 = out["f32"].ctypes.data if "f32" in out else None
    args.out_f64 = out["f64"].ctypes.data if "f64" in out else None
    args.threads = threads or default_threads()
    if lib().orc_attention(ctypes.byref(args)) != 0:
        raise ValueError("oracle rejected the attention geometry")
    return out


def qk_norm_rope(q, k, q_weight, k_weight, *, offset: int, theta: float, epsilon: float):
    """Restatement of qk_norm_rope_cache_f16 (transformer.metal:1533-1577).

    Returns (query_out [T, Hq, D], key_rows [T, Hkv, D]) as f16 bits; the key
    rows are what the kernel writes into the cache at `offset`.
    """
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    qw = np.ascontiguousarray(q_weight, dtype=np.uint16)
    kw = np.ascontiguousarray(k_weight, dtype=np.uint16)
    T, hq, d = q.shape
    hkv = k.shape[1]
    q_out = np.empty_like(q)
    k_out = np.empty_like(k)
    rc = lib().orc_qk_norm_rope(
        q.ctypes.data_as(_u16p), k.ctypes.data_as(_u16p), qw.ctypes.data_as(_u16p),
        kw.ctypes.data_as(_u16p), T, hq, hkv, d, offset, theta, epsilon,
        q_out.ctypes.data_as(_u16p), k_out.ctypes.data_as(_u16p))
    if rc != 0:
        raise ValueError("oracle rejected the Q/K transform geometry")
    return q_out, k_out


def rms_norm(x, weight, *, epsilon: float):
    """Restatement of rms_norm_f16 (transformer.metal:1318-1340) over the last
    dimension. Returns (f16 bits, unrounded f32), both of x's shape."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(weight, dtype=np.uint16)
    width = x.shape[-1]
    out = np.empty_like(x)
    out32 = np.empty(x.shape, dtype=np.float32)
    rc = lib().orc_rms_norm(x.ctypes.data_as(_u16p), w.ctypes.data_as(_u16p), x.size // width,
                            width, epsilon, out.ctypes.data_as(_u16p), out32.ctypes.data_as(_f32p))
    if rc != 0:
        raise ValueError("oracle rejected the RMSNorm geometry")
    return out, out32


def rope(x, *, offset: int, theta: float):
    """Restatement of rope_f16 (transformer.metal:1514-1531) on [T, H, D]."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    T, h, d = x.shape
    out = np.empty_like(x)
    rc = lib().orc_rope(x.ctypes.data_as(_u16p), T, h, d, offset, theta, out.ctypes.data_as(_u16p))
    if rc != 0:
        raise ValueError("oracle rejected the RoPE geometry")
    return out


def matmul(x, weight, threads: int | None = None):
    """Restatement of matmul_f16 (transformer.metal:70-93): x [m, k] times
    weight [n, k] transposed. Returns (f16 bits [m, n], unrounded f32)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(weight, dtype=np.uint16)
    m, k = x.shape
    n = w.shape[0]
    assert w.shape[1] == k
    out = np.empty((m, n), dtype=np.uint16)
    out32 = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul(x.ctypes.data_as(_u16p), w.ctypes.data_as(_u16p), m, n, k,
                     out.ctypes.data_as(_u16p), out32.ctypes.data_as(_f32p),
                     default_threads() if threads is None else threads)
    return out, out32
