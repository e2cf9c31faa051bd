"""Shared helpers for the parity tests: layouts, runs, and the oracle check."""
from __future__ import annotations

import numpy as np

import mi_attn
import oracle

# north_star: max-abs error <= 2e-3 against the reference CPU path (the f32
# oracle, unrounded), with f32 accumulation.
TOL = 2e-3

KINDS = {"reference": mi_attn.REFERENCE, "tiled": mi_attn.TILED,
         "flash-prefill": mi_attn.FLASH_PREFILL, "decode-split-kv": mi_attn.DECODE_SPLIT_KV,
         "flash-decode": mi_attn.FLASH_DECODE}


def f16(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def upload_kv(ctx, logical: np.ndarray, layout: str, capacity: int | None = None):
    """Device copy of [L, H, D] rows; returns (owner, [L, H, D] view)."""
    L, H, D = logical.shape
    capacity = capacity or L
    if layout == "position_major":       # the reference's [cap, Hkv, D]
        store = np.zeros((capacity, H, D), dtype=np.uint16)
        store[:L] = logical
        owner = ctx.tensor(store)
        return owner, owner.prefix(L)
    if layout == "head_major":           # this build's cache: [Hkv, cap, D]
        store = np.zeros((H, capacity, D), dtype=np.uint16)
        store[:, :L] = logical.transpose(1, 0, 2)
        owner = ctx.tensor(store)
        return owner, owner.view((L, H, D), (D, capacity * D, 1))
    if layout == "reversed":             # head-major, last position first in memory
        store = np.zeros((H, capacity, D), dtype=np.uint16)
        store[:, capacity - L:] = logical[::-1].transpose(1, 0, 2)
        owner = ctx.tensor(store)
        return owner, owner.view((L, H, D), (-D, capacity * D, 1), offset=(capacity - 1) * D)
    raise ValueError(layout)


def run_attention(ctx, q, k, v, *, hq, hkv, d, off, kind, causal=True, layout="head_major",
                  block=None, threads=None):
    qt = ctx.tensor(np.ascontiguousarray(q))
    ko, kview = upload_kv(ctx, k, layout)
    vo, vview = upload_kv(ctx, v, layout)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, causal, off)
    out = ctx.empty(q.shape)
    batch = ctx.begin_batch()
    if block is not None:
        batch.attention_flash_decode_with_configuration(qt, kview, vview, cfg, block,
                                                        threads or 256, out=out)
    else:
        batch.attention(qt, kview, vview, cfg, KINDS[kind] if isinstance(kind, str) else kind,
                        out=out)
    batch.finish()
    return ctx.download(out)


def oracle_attention(q, k, v, *, hq, hkv, d, off, causal=True, rows=None, want=("f16", "f32")):
    return oracle.attention(q, k, v, q_heads=hq, kv_heads=hkv, head_dim=d, causal=causal,
                            query_offset=off, rows=rows, want=want)


def max_abs(gpu_bits: np.ndarray, expected: np.ndarray) -> float:
    """Largest |got - expected|. An element that is NaN on both sides (the
    reference's 0/0 for a row with no visible key) counts as a match; a NaN
    on one side only makes the result NaN, which fails every `<= tol` check."""
    got = f16(gpu_bits).astype(np.float64)
    exp = np.broadcast_to(np.asarray(expected, dtype=np.float64), got.shape)
    diff = np.abs(got - exp)
    diff[np.isnan(got) & np.isnan(exp)] = 0.0
    return float(diff.max()) if diff.size else 0.0


def assert_parity(gpu_bits: np.ndarray, ref: dict, tol: float = TOL, label: str = "") -> float:
    """GPU f16 output vs the f32 oracle (unrounded) within `tol`."""
    err = max_abs(gpu_bits, ref["f32"])
    assert err <= tol, f"{label}: max-abs error {err:.3e} > {tol:.1e}"
    return err
