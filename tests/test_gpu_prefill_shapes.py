"""Seeded random prefill geometries against the oracle: head_dim 32 / 64 /
128 / 256, GQA ratios 1-8, query offsets, causal and not, token counts that
give split plans (ordered pieces or the (row tile, KV head, split) grid) and
unsplit ones, ragged row tiles. Every query row of a sample (the first and
last token, and 30 seeded ones) is checked against the f32 oracle within
2e-3, and the plan the library chose is recorded in the failure label."""
from __future__ import annotations

import numpy as np
import pytest

import mi_attn
from helpers import assert_parity, oracle_attention, run_attention

pytestmark = pytest.mark.gpu

CASES = 40


def _geometry(i: int):
    rng = np.random.default_rng(9000 + i)
    d = int(rng.choice([32, 64, 128, 256]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 4, 8]))
    T = int(rng.integers(33, 1400))
    causal = bool(rng.random() < 0.8)
    off = int(rng.choice([0, rng.integers(1, 3000)])) if causal else 0
    L = off + T if causal else int(T + rng.integers(0, 900))
    return rng, d, hkv * g, hkv, T, off, L, causal


@pytest.mark.parametrize("i", range(CASES))
def test_random_prefill_geometry(ctx, i):
    rng, d, hq, hkv, T, off, L, causal = _geometry(i)
    q = rng.standard_normal((T, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    geo = dict(hq=hq, hkv=hkv, d=d, off=off)
    info = ctx.plan(ctx.tensor(q), ctx.tensor(k), ctx.tensor(v),
                    mi_attn.AttentionConfig(hq, hkv, d, causal, off), mi_attn.FLASH_PREFILL)
    assert info["kernel"] == "attn_prefill", info
    out = run_attention(ctx, q, k, v, kind="flash-prefill", causal=causal, **geo)
    rows = np.unique(np.concatenate([[0, T - 1], rng.integers(0, T, 30)]))
    ref = oracle_attention(q, k, v, causal=causal, rows=rows, want=("f32",), **geo)
    label = (f"case {i}: d={d} hq={hq} hkv={hkv} T={T} off={off} L={L} causal={causal} "
             f"grid={info['grid']} splits={info['splits']}")
    assert_parity(out[rows], ref, label=label)


def test_random_geometries_cover_both_split_grids(ctx):
    """The sample above includes ordered split plans (grid (pieces, KV heads,
    1) with several splits), unordered split plans and unsplit plans."""
    kinds = set()
    for i in range(CASES):
        _, d, hq, hkv, T, off, L, causal = _geometry(i)
        q = ctx.empty((T, hq, d))
        k = ctx.empty((L, hkv, d))
        info = ctx.plan(q, k, k, mi_attn.AttentionConfig(hq, hkv, d, causal, off),
                        mi_attn.FLASH_PREFILL)
        if info["splits"] == 1:
            kinds.add("unsplit")
        else:
            kinds.add("ordered" if info["grid"][2] == 1 else "grid")
        q.free()
        k.free()
    assert kinds == {"unsplit", "ordered", "grid"}, kinds
