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
    diff = np.abs(f16(gpu_bits).astype(np.float64) - np.asarray(expected, dtype=np.float64))
    return float(np.nanmax(diff)) if diff.size else 0.0


def assert_parity(gpu_bits: np.ndarray, ref: dict, tol: float = TOL, label: str = "") -> float:
    """GPU f16 output vs the f32 oracle (unrounded) within `tol`."""
    err = max_abs(gpu_bits, ref["f32"])
    assert err <= tol, f"{label}: max-abs error {err:.3e} > {tol:.1e}"
    return err
