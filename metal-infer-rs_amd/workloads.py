"""Seeded synthetic inputs for the five BASELINE attention configurations.

Values come from XorShift64 (crates/metal-infer-models/src/qwen3.rs:1011-1034)
feeding Box-Muller (z = sqrt(-2 ln(1 - u1)) cos(2 pi u2), two draws per
value), rounded f64 -> f32 -> f16 with round-to-nearest-even. Arrays are
filled in logical order: Q[t][h][d], K[pos][kvh][d], V[pos][kvh][d]; for the
batched decode, the 32 lengths are drawn first, then K and V sequence by
sequence from one stream each. Config c uses stream seeds 0x4D490000 + 16c
(+0 Q, +1 K, +2 V, +3 lengths).

The generator itself is native (libmi_bench.so, include/mi_bench.h): the
stream is split across threads by GF(2) jump-ahead and stays bit-identical to
a sequential walk.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "libmi_bench.so"
_lib = None


def _bench_lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise ImportError(f"{_LIB_PATH} is missing: build with make -C metal-infer-rs_amd")
        lib = ctypes.CDLL(str(_LIB_PATH))
        lib.mi_bench_fill_normal_f16.argtypes = [ctypes.c_uint64, ctypes.c_void_p,
                                                 ctypes.c_size_t, ctypes.c_int32]
        lib.mi_bench_fill_uniform_u32.argtypes = [ctypes.c_uint64, ctypes.c_uint32,
                                                  ctypes.c_uint32, ctypes.c_void_p,
                                                  ctypes.c_size_t]
        _lib = lib
    return _lib


def normal_f16(seed: int, n: int, threads: int | None = None) -> np.ndarray:
    """n seeded N(0,1) values as f16 bits, in stream order."""
    out = np.empty(n, dtype=np.uint16)
    threads = threads or max(1, min(16, os.cpu_count() or 1))
    _bench_lib().mi_bench_fill_normal_f16(seed, out.ctypes.data, n, threads)
    return out


def uniform_u32(seed: int, lo: int, hi: int, n: int) -> np.ndarray:
    """lo + floor(u * (hi - lo + 1)) from n sequential draws."""
    out = np.empty(n, dtype=np.uint32)
    _bench_lib().mi_bench_fill_uniform_u32(seed, lo, hi, out.ctypes.data, n)
    return out


def config_seed(config: int) -> int:
    return 0x4D490000 + 16 * config


def compare_inputs(tokens: int, length: int, q_heads: int, kv_heads: int,
                   head_dim: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """The attention bench's closed-form inputs
    (crates/metal-infer-cli/src/bin/bench.rs:973-981): over the flat index i,
    Q = (i % 43) / 43 - 0.5, K = (i % 37) / 37 - 0.25, V = (i % 29) / 29, in
    f32 and then rounded to f16 (round to nearest even, as tensor_f16 does).
    Returns f16 bits shaped [T, Hq, D], [L, Hkv, D], [L, Hkv, D]."""
    f = np.float32

    def pattern(n, mod, offset):
        i = np.arange(n, dtype=np.int64)
        return ((i % mod).astype(f) / f(mod) - f(offset)).astype(np.float16).view(np.uint16)

    q = pattern(tokens * q_heads * head_dim, 43, 0.5).reshape(tokens, q_heads, head_dim)
    k = pattern(length * kv_heads * head_dim, 37, 0.25).reshape(length, kv_heads, head_dim)
    v = pattern(length * kv_heads * head_dim, 29, 0.0).reshape(length, kv_heads, head_dim)
    return q, k, v


@dataclass
class AttentionCase:
    """One BASELINE configuration (1-based index `config`)."""
    config: int
    kind: str            # "prefill" | "decode" | "batched_decode"
    tokens: int          # T (query tokens per sequence)
    q_heads: int
    kv_heads: int
    head_dim: int
    kv_length: int       # L (per sequence max for the batched decode)
    query_offset: int
    batch: int = 1
    lengths: np.ndarray | None = None
    description: str = ""
    q: np.ndarray | None = field(default=None, repr=False)   # [B*T or T, Hq, D]
    k: np.ndarray | None = field(default=None, repr=False)   # [L, Hkv, D] or list per seq
    v: np.ndarray | None = field(default=None, repr=False)

    @property
    def group(self) -> int:
        return self.q_heads // self.kv_heads

    def visible_pairs(self) -> int:
        """Causally visible (query, key) pairs per query head."""
        if self.kind == "batched_decode":
            return int(np.sum(self.lengths, dtype=np.int64))
        if self.kind == "decode":
            return self.kv_length
        return sum(min(self.kv_length, self.query_offset + t + 1) for t in range(self.tokens))

    def flops(self) -> int:
        """4 * D per visible pair per query head (QK^T and PV multiply-adds)."""
        return 4 * self.head_dim * self.q_heads * self.visible_pairs()

    def algorithmic_bytes(self) -> int:
        """Each active K/V byte once, plus Q and O."""
        row = self.kv_heads * self.head_dim * 2
        if self.kind == "batched_decode":
            kv = 2 * row * int(np.sum(self.lengths, dtype=np.int64))
        else:
            kv = 2 * row * self.kv_length
        qo = 2 * self.batch * self.tokens * self.q_heads * self.head_dim * 2
        return kv + qo


_GEOMETRY = {
    1: dict(kind="prefill", tokens=128, q_heads=16, kv_heads=8, head_dim=128, kv_length=128,
            query_offset=0, description="c1 causal prefill T=128, Qwen3-0.6B (16/8/128)"),
    2: dict(kind="decode", tokens=1, q_heads=16, kv_heads=8, head_dim=128, kv_length=2048,
            query_offset=2047, description="c2 decode L=2048, Qwen3-0.6B (16/8/128)"),
    3: dict(kind="prefill", tokens=2048, q_heads=16, kv_heads=8, head_dim=128, kv_length=2048,
            query_offset=0, description="c3 causal prefill T=2048, Qwen3-0.6B (16/8/128)"),
    4: dict(kind="batched_decode", tokens=1, q_heads=32, kv_heads=8, head_dim=128,
            kv_length=8192, query_offset=0, batch=32,
            description="c4 batched decode B=32, L~U[1024,8192], Qwen3-8B (32/8/128)"),
    5: dict(kind="prefill", tokens=4096, q_heads=64, kv_heads=8, head_dim=128, kv_length=20480,
            query_offset=16384,
            description="c5 chunked prefill T=4096 on a 16384 cache, Qwen3-32B (64/8/128)"),
}


def case(config: int, generate: bool = True) -> AttentionCase:
    """Geometry (and, if generate, the seeded inputs) of BASELINE config c."""
    c = AttentionCase(config=config, **_GEOMETRY[config])
    base = config_seed(config)
    if c.kind == "batched_decode":
        c.lengths = uniform_u32(base + 3, 1024, 8192, c.batch)
    if not generate:
        return c
    c.q = normal_f16(base + 0, c.batch * c.tokens * c.q_heads * c.head_dim).reshape(
        c.batch * c.tokens, c.q_heads, c.head_dim)
    row = c.kv_heads * c.head_dim
    if c.kind == "batched_decode":
        total = int(np.sum(c.lengths, dtype=np.int64))
        kflat = normal_f16(base + 1, total * row)
        vflat = normal_f16(base + 2, total * row)
        c.k, c.v, pos = [], [], 0
        for length in c.lengths.tolist():
            c.k.append(kflat[pos * row:(pos + length) * row].reshape(length, c.kv_heads, c.head_dim))
            c.v.append(vflat[pos * row:(pos + length) * row].reshape(length, c.kv_heads, c.head_dim))
            pos += length
    else:
        c.k = normal_f16(base + 1, c.kv_length * row).reshape(c.kv_length, c.kv_heads, c.head_dim)
        c.v = normal_f16(base + 2, c.kv_length * row).reshape(c.kv_length, c.kv_heads, c.head_dim)
    return c


def head_major(logical: np.ndarray, capacity: int | None = None) -> np.ndarray:
    """[L, Hkv, D] logical rows -> [Hkv, capacity, D] head-major storage."""
    L, H, D = logical.shape
    capacity = capacity or L
    out = np.zeros((H, capacity, D), dtype=logical.dtype)
    out[:, :L, :] = logical.transpose(1, 0, 2)
    return out
