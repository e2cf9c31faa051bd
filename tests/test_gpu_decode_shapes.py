"""Seeded random batched-decode geometries against the oracle: 1-48
sequences, GQA ratios 1-16, head_dim 128 (the stream-K MFMA kernel and its
merge launch) and 64 (the rows kernel), per-sequence lengths from 0 to past
the cache capacity (clamped), head-major and token-major caches, the default
plan and explicit split sizes (the rows kernel, splits merged inside the
launch). Every sequence is checked (a zero-length one must be NaN, the
reference's 0/0), a second call must be bit-identical, and the
no-allocation entry point must agree bit for bit where its buffer holds the
partials."""
from __future__ import annotations

import numpy as np
import pytest

import mi_attn
from helpers import assert_parity, oracle_attention

pytestmark = pytest.mark.gpu

CASES = 30


def _geometry(i: int):
    rng = np.random.default_rng(7000 + i)
    d = int(rng.choice([128, 128, 64]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 4, 8, 16]))
    B = int(rng.integers(1, 49))
    cap = int(rng.integers(16, 1500))
    lengths = rng.integers(0, cap + 40, B)
    lengths[rng.random(B) < 0.1] = 0
    block = int(rng.choice([0, 0, 0, 64, 192]))
    token_major = bool(rng.random() < 0.3)
    return rng, d, hkv * g, hkv, B, cap, lengths.astype(np.uint32), block, token_major


@pytest.mark.parametrize("i", range(CASES))
def test_random_batched_decode_geometry(ctx, i):
    rng, d, hq, hkv, B, cap, lengths, block, token_major = _geometry(i)
    q = rng.standard_normal((B, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((B, cap, hkv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((B, cap, hkv, d)).astype(np.float16).view(np.uint16)
    if token_major:
        kt, vt = ctx.tensor(k), ctx.tensor(v)
        kview, vview = kt, vt
    else:  # head-major storage [B, Hkv, cap, D] seen as [B, cap, Hkv, D]
        kt = ctx.tensor(np.ascontiguousarray(k.transpose(0, 2, 1, 3)))
        vt = ctx.tensor(np.ascontiguousarray(v.transpose(0, 2, 1, 3)))
        view = ((B, cap, hkv, d), (hkv * cap * d, d, cap * d, 1))
        kview, vview = kt.view(*view), vt.view(*view)
    qt, lt = ctx.tensor(q), ctx.tensor(lengths, mi_attn.U32)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    label = (f"case {i}: d={d} hq={hq} hkv={hkv} B={B} cap={cap} block={block} "
             f"token_major={token_major}")
    outs = []
    for _ in range(2):
        batch = ctx.begin_batch()
        out = batch.attention_decode_batched(qt, kview, vview, lt, cfg, block)
        batch.finish()
        outs.append(ctx.download(out))
    got = outs[0]
    assert np.array_equal(got.view(np.uint16), outs[1].view(np.uint16)), label
    for b in range(B):
        n = min(int(lengths[b]), cap)
        if n == 0:
            assert np.isnan(got[b].view(np.float16).astype(np.float32)).all(), label
            continue
        ref = oracle_attention(q[b:b + 1], k[b, :n], v[b, :n], hq=hq, hkv=hkv, d=d, off=n - 1)
        assert_parity(got[b:b + 1], ref, label=f"{label} seq {b} len {n}")
    fixed = ctx.empty(q.shape)
    batch = ctx.begin_batch()
    try:
        batch.attention_decode_batched_noalloc(qt, kview, vview, lt, cfg, block, fixed)
    except mi_attn.MiError as err:  # partials larger than the fixed buffer
        batch.abandon()
        assert err.name == "MI_ERR_RESOURCE", (label, err)
    else:
        batch.finish()
        assert np.array_equal(ctx.download(fixed).view(np.uint16), got.view(np.uint16)), label


def test_random_decode_geometries_cover_both_kernels():
    """The sample above holds stream-K calls (head_dim 128, default plan),
    rows-kernel calls by default (head_dim 64) and with explicit splits,
    both cache layouts, zero lengths and lengths past the capacity."""
    kinds, layouts, zero, clamped = set(), set(), 0, 0
    for i in range(CASES):
        _, d, _, _, _, cap, lengths, block, token_major = _geometry(i)
        kinds.add("stream" if d == 128 and block == 0 else "rows-default" if block == 0 else "rows-split")
        layouts.add(token_major)
        zero += int((lengths == 0).any())
        clamped += int((lengths > cap).any())
    assert kinds == {"stream", "rows-default", "rows-split"}, kinds
    assert layouts == {True, False}
    assert zero > 0 and clamped > 0
