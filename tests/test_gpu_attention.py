"""GPU parity of the attention kernels, through the C ABI, against the oracle.

The bar (north_star): max-abs error <= 2e-3 against the f32 oracle
(attention_reference_f16 restated, unrounded) on identical inputs; the
golden fixtures (torch float64 SDPA) are checked with the same bound. The
reference tests' own tolerance was 0.02 (gpu.rs:6).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import mi_attn
import ref_cases
import workloads
from helpers import (KINDS, TOL, assert_parity, f16, max_abs, oracle_attention, run_attention,
                     upload_kv)

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden" / "attention_golden.npz"


@pytest.fixture(scope="module")
def golden():
    data = np.load(GOLDEN, allow_pickle=False)
    return {name: data[name] for name in data["__names__"].tolist()}


CASES = ref_cases.attention_cases()


@pytest.mark.parametrize("case", CASES, ids=lambda c: c["name"])
def test_reference_cases_all_kinds(ctx, case, golden):
    """gpu.rs:613-808 / ops.rs:1416-1476 shapes and inputs, every kind."""
    q, k, v = ref_cases.build(case)
    geo = dict(hq=case["hq"], hkv=case["hkv"], d=case["d"], off=case["off"])
    ref = oracle_attention(q, k, v, **geo)
    for kind in case["kinds"]:
        for layout in ("head_major", "position_major"):
            out = run_attention(ctx, q, k, v, kind=kind, layout=layout, **geo)
            label = f"{case['name']}/{kind}/{layout}"
            assert_parity(out, ref, label=label)
            assert max_abs(out, golden[case["name"]]) <= TOL, label


@pytest.mark.parametrize("L", [1, 63, 64, 65, 256, 640, 8192])
def test_flash_decode_block_and_thread_grid(ctx, L):
    """gpu.rs:729-768: every (block, threads) configuration."""
    case = next(c for c in CASES if c["name"] == f"decode_blocks_L{L}")
    q, k, v = ref_cases.build(case)
    geo = dict(hq=2, hkv=1, d=128, off=L - 1)
    ref = oracle_attention(q, k, v, **geo)
    for block in (32, 64, 128, 256):
        for threads in (128, 256):
            out = run_attention(ctx, q, k, v, kind="flash-decode", block=block, threads=threads,
                                **geo)
            assert_parity(out, ref, label=f"L={L} block={block} threads={threads}")


def test_reference_kind_is_the_exact_two_pass_softmax(ctx):
    """The GPU Reference kernel follows the oracle's operation order: only
    expf may differ (by an ulp), so outputs agree to within one f16 ulp."""
    rng = np.random.default_rng(5)
    T, L, hq, hkv, d = 17, 40, 8, 2, 64
    q = rng.standard_normal((T, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    geo = dict(hq=hq, hkv=hkv, d=d, off=L - T)
    ref = oracle_attention(q, k, v, **geo)
    out = run_attention(ctx, q, k, v, kind="reference", **geo)
    ulps = np.abs(out.astype(np.int32) - ref["f16"].astype(np.int32))
    assert ulps.max() <= 1
    assert (ulps != 0).mean() < 0.01
    assert_parity(out, ref)


# -------------------------------------------------- BASELINE configs ------

def _prefill_parity(ctx, c, kind, rows=None):
    geo = dict(hq=c.q_heads, hkv=c.kv_heads, d=c.head_dim, off=c.query_offset)
    out = run_attention(ctx, c.q, c.k, c.v, kind=kind, **geo)
    ref = oracle_attention(c.q, c.k, c.v, rows=rows, **geo)
    got = out if rows is None else out[rows]
    return assert_parity(got, ref, label=f"c{c.config}/{kind}")


def test_c1_prefill_seeded(ctx):
    c = workloads.case(1)
    for kind in ("flash-prefill", "tiled", "reference"):
        _prefill_parity(ctx, c, kind)


def test_c2_decode_seeded(ctx):
    c = workloads.case(2)
    for kind in ("flash-decode", "decode-split-kv", "reference"):
        _prefill_parity(ctx, c, kind)


def test_c3_prefill_seeded(ctx):
    c = workloads.case(3)
    _prefill_parity(ctx, c, "flash-prefill")


def tile_rows(T: int, G: int, block_m: int, rng) -> np.ndarray:
    """Query tokens covering every row tile of the packed (token, head in
    group) dimension: the first and last token of each tile of `block_m`
    packed rows plus one seeded interior token. Every query head of those
    tokens is checked, so every (row tile, KV head) piece is."""
    tokens = []
    for row0 in range(0, T * G, block_m):
        first, last = row0 // G, min(T - 1, (row0 + block_m - 1) // G)
        tokens += [first, last]
        if last - first >= 2:
            tokens.append(int(rng.integers(first + 1, last)))
    return np.unique(np.asarray(tokens))


def test_c5_chunked_prefill_seeded(ctx):
    """4096 new tokens on a 16384-position cache, GQA 8:1 (256-row tiles of
    32 tokens, 128 per KV head): the first, last and one interior token of
    every row tile, all 64 heads, against the oracle."""
    c = workloads.case(5)
    rows = tile_rows(c.tokens, c.group, 256, np.random.default_rng(55))
    assert len(rows) == 3 * 128
    err = _prefill_parity(ctx, c, "flash-prefill", rows=rows)
    print(f"c5 {len(rows)} rows x 64 heads max-abs {err:.2e}")


def test_c5_chunked_prefill_full_output(ctx):
    """Every one of c5's 4096 x 64 output rows against the oracle (the f32
    restatement over all 16384 + 4096 keys; several seconds of host time on
    the oracle's threads)."""
    c = workloads.case(5)
    err = _prefill_parity(ctx, c, "flash-prefill")
    print(f"c5 all {c.tokens} tokens x 64 heads max-abs {err:.2e}")


@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (32, 8), (64, 8), (16, 1)])
def test_flash_prefill_gqa_ratios_and_offsets(ctx, d, hq, hkv):
    rng = np.random.default_rng(hq * 100 + hkv + d)
    for T, off, causal in ((1, 0, True), (7, 100, True), (100, 0, True), (300, 37, True),
                           (65, 0, False), (129, 500, True)):
        L = off + T if causal else T + 40
        q = rng.standard_normal((T, hq, d)).astype(np.float16).view(np.uint16)
        k = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
        v = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
        geo = dict(hq=hq, hkv=hkv, d=d, off=off)
        out = run_attention(ctx, q, k, v, kind="flash-prefill", causal=causal, **geo)
        ref = oracle_attention(q, k, v, causal=causal, **geo)
        assert_parity(out, ref, label=f"T={T} off={off} causal={causal}")


@pytest.mark.parametrize("hq,hkv,T,off,causal", [
    (64, 8, 4100, 3, True),      # ragged last row tile, GQA 8
    (8, 8, 33000, 0, True),      # MHA: a row tile spans 256 tokens
    (32, 8, 8200, 0, False)])
def test_flash_prefill_256_row_tiles(ctx, hq, hkv, T, off, causal):
    """Grids of at least four 256-row workgroups per CU run the 8-wave row
    tile; the first, last and one interior token of every 256-row tile (all
    heads) are checked against the oracle."""
    rng = np.random.default_rng(T + hq)
    L = off + T if causal else T + 40
    q = rng.standard_normal((T, hq, 128)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((L, hkv, 128)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((L, hkv, 128)).astype(np.float16).view(np.uint16)
    geo = dict(hq=hq, hkv=hkv, d=128, off=off)
    info = ctx.plan(ctx.tensor(q), ctx.tensor(k), ctx.tensor(v),
                    mi_attn.AttentionConfig(hq, hkv, 128, causal, off), mi_attn.FLASH_PREFILL)
    assert info["kernel"] == "attn_prefill" and info["block_threads"] == 512, info
    out = run_attention(ctx, q, k, v, kind="flash-prefill", causal=causal, **geo)
    rows = tile_rows(T, hq // hkv, 256, rng)
    ref = oracle_attention(q, k, v, causal=causal, rows=rows, **geo)
    assert_parity(out[rows], ref, label=f"T={T} hq={hq}")


@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("T,off,L,causal", [
    (300, 100, 477, True),   # 77 cached keys past the last row's window
    (300, 100, 250, True),   # cache shorter than the window: late rows see all L keys
    (300, 0, 70, False),     # fewer keys than query rows
    (129, 0, 1, False),      # one key
    (200, 5000, 5200, True)])  # long offset, split plan
def test_flash_prefill_key_length_edges(ctx, d, T, off, L, causal):
    """FlashPrefill where the key count is not offset + T: keys past every
    row's causal window (they must have no influence), a cache shorter than
    the causal window (the availability min(L, offset + t + 1) of
    transformer.metal:1589-1590), fewer keys than rows, and a single key."""
    hq, hkv = 16, 4
    rng = np.random.default_rng(T + L + d)
    q = rng.standard_normal((T, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    geo = dict(hq=hq, hkv=hkv, d=d, off=off)
    info = ctx.plan(ctx.tensor(q), ctx.tensor(k), ctx.tensor(v),
                    mi_attn.AttentionConfig(hq, hkv, d, causal, off), mi_attn.FLASH_PREFILL)
    assert info["kernel"] == "attn_prefill", info
    out = run_attention(ctx, q, k, v, kind="flash-prefill", causal=causal, **geo)
    ref = oracle_attention(q, k, v, causal=causal, **geo)
    assert_parity(out, ref, label=f"T={T} off={off} L={L} causal={causal} plan={info}")


@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("offset,pad,kernel", [(8, 8, "attn_prefill"), (4, 4, "attn_rows")])
def test_flash_prefill_strided_output(ctx, d, offset, pad, kernel):
    """FlashPrefill into a strided view of a larger buffer (rows padded by
    `pad` elements, the view starting `offset` elements in). Rows that are
    16-byte aligned take the MFMA kernel, whose output leaves LDS as 16-byte
    chunks of whole rows; 8-byte-aligned rows take the rows kernel. Both match
    the oracle, and every element outside the view (padding, the ragged last
    row tile's rows past the last token) keeps its sentinel."""
    rng = np.random.default_rng(d + offset)
    T, hq, hkv = 203, 8, 2  # 812 packed rows: the last 128-row tile is ragged
    q = rng.standard_normal((T, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((T, hkv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((T, hkv, d)).astype(np.float16).view(np.uint16)
    row = d + pad
    sentinel = np.uint16(0x7BFF)  # f16 65504: no attention output reaches it
    host = np.full(offset + T * hq * row + 64, sentinel, dtype=np.uint16)
    buf = ctx.tensor(host)
    out = buf.view((T, hq, d), (hq * row, row, 1), offset)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    ctx.take_kernel_profiles()
    ctx.set_kernel_profiling(True)
    try:
        batch = ctx.begin_batch()
        batch.attention(ctx.tensor(q), ctx.tensor(k), ctx.tensor(v), cfg, mi_attn.FLASH_PREFILL,
                        out=out)
        batch.finish()
        names = [name for name, _ in ctx.take_kernel_profiles()]
    finally:
        ctx.set_kernel_profiling(False)
    assert kernel in names, names
    got = ctx.download(buf)
    inside = np.zeros(host.shape, dtype=bool)
    idx = offset + (np.arange(T * hq)[:, None] * row + np.arange(d)[None, :])
    inside[idx.ravel()] = True
    assert (got[~inside] == sentinel).all(), "a store left the output view"
    ref = oracle_attention(q, k, v, causal=True, hq=hq, hkv=hkv, d=d, off=0)
    assert_parity(got[idx].reshape(T, hq, d), ref, label=f"d={d} offset={offset} pad={pad}")


@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("hq,hkv,T,off,causal", [
    (8, 8, 700, 37, True), (16, 8, 1000, 300, True), (64, 8, 520, 37, True),
    (16, 1, 333, 300, True), (8, 2, 1500, 0, True), (8, 8, 520, 0, False)])
def test_flash_prefill_key_splits(ctx, d, hq, hkv, T, off, causal):
    """Small grids run heavy row tiles in several key splits plus a merge
    pass. These geometries include row tiles whose last split starts past
    the causal limit of their first rows (such rows see no key there)."""
    rng = np.random.default_rng(T * 7 + hq + d)
    L = off + T if causal else T + 40
    q = rng.standard_normal((T, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    geo = dict(hq=hq, hkv=hkv, d=d, off=off)
    info = ctx.plan(ctx.tensor(q), ctx.tensor(k), ctx.tensor(v),
                    mi_attn.AttentionConfig(hq, hkv, d, causal, off), mi_attn.FLASH_PREFILL)
    # Split unless the row tiles alone fill the resident workgroups (two per
    # CU, one at head_dim 256).
    resident = ctx.compute_units * (1 if d == 256 else 2)
    assert info["kernel"] == "attn_prefill", info
    assert info["splits"] > 1 or info["grid"][0] * info["grid"][1] >= resident, info
    out = run_attention(ctx, q, k, v, kind="flash-prefill", causal=causal, **geo)
    ref = oracle_attention(q, k, v, causal=causal, **geo)
    assert_parity(out, ref, label=f"splits={info['splits']} T={T} off={off}")


def _moving_max_inputs(rng, T, L, hq, hkv, d, pattern):
    """Q/K/V whose scores move along the keys by far more than the kernels'
    lazy-rescale thresholds (2^8 for decode, an f16 overflow of the weights
    for prefill): every query of a GQA group leans on one direction per KV
    head, and key j carries amp(j) times that direction, so the raw score
    grows as amp(j) |base|^2 (up to ~6 D, i.e. 70-140 binades of weight)."""
    g = hq // hkv
    base = rng.standard_normal((hkv, d))
    q = np.repeat(base[None, :, None, :], g, axis=2).reshape(1, hq, d)
    q = q + 0.3 * rng.standard_normal((T, hq, d))
    pos = np.arange(L) / max(L - 1, 1)
    if pattern == "rising":
        amp = 6.0 * pos
    elif pattern == "falling":
        amp = 6.0 * (1.0 - pos)
    else:  # spikes: ~1% of the keys, anywhere, each far above the rest
        amp = np.where(rng.random(L) < 0.01, rng.uniform(2.0, 6.0, L), 0.0)
    k = 0.5 * rng.standard_normal((L, hkv, d)) + amp[:, None, None] * base[None]
    v = rng.standard_normal((L, hkv, d))
    as16 = lambda a: a.astype(np.float16).view(np.uint16)  # noqa: E731
    return as16(q), as16(k), as16(v)


@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("hq,hkv,T,off,pattern", [
    (16, 8, 1000, 300, "rising"),    # key splits
    (64, 8, 520, 2000, "rising"),
    (16, 8, 1000, 300, "spikes"),
    (8, 8, 700, 37, "spikes"),
    (16, 1, 333, 3000, "falling")])
def test_flash_prefill_reference_max_moves(ctx, d, hq, hkv, T, off, pattern):
    """The prefill kernels move a row's reference max only when a weight
    overflows f16 (or the row has none yet). Scores that climb, fall or spike
    by tens of binades along the keys make that happen in the middle of the
    key loop, in either key half of a tile and in every key split."""
    rng = np.random.default_rng(T + 13 * hq + d + len(pattern))
    L = off + T
    q, k, v = _moving_max_inputs(rng, T, L, hq, hkv, d, pattern)
    geo = dict(hq=hq, hkv=hkv, d=d, off=off)
    out = run_attention(ctx, q, k, v, kind="flash-prefill", **geo)
    ref = oracle_attention(q, k, v, **geo)
    assert_parity(out, ref, label=f"{pattern} T={T} off={off}")


@pytest.mark.parametrize("pattern", ["rising", "falling", "spikes"])
@pytest.mark.parametrize("kind", ["flash-decode", "decode-split-kv"])
def test_decode_reference_max_moves(ctx, kind, pattern):
    """The decode kernels' lazy rescale (the reference max moves when a
    score outgrows it by 2^8) under scores that move by tens of binades."""
    rng = np.random.default_rng(len(kind) * 7 + len(pattern))
    L, hq, hkv, d = 5000, 16, 8, 128
    q, k, v = _moving_max_inputs(rng, 1, L, hq, hkv, d, pattern)
    geo = dict(hq=hq, hkv=hkv, d=d, off=L - 1)
    out = run_attention(ctx, q, k, v, kind=kind, **geo)
    assert_parity(out, oracle_attention(q, k, v, **geo), label=f"{kind} {pattern}")


@pytest.mark.parametrize("pattern", ["rising", "spikes"])
def test_batched_decode_reference_max_moves(ctx, pattern):
    """The stream-K batched decode (split units merged in a second launch)
    under scores that move by tens of binades along each sequence."""
    rng = np.random.default_rng(91 + len(pattern))
    B, hq, hkv, d, cap = 6, 32, 8, 128, 4000
    lengths = [4000, 1, 2500, 3999, 700, 1800]
    qs, ks, vs = [], [], []
    for b in range(B):
        q, k, v = _moving_max_inputs(rng, 1, cap, hq, hkv, d, pattern)
        qs.append(q[0])
        ks.append(k)
        vs.append(v)
    q, k, v = np.stack(qs), np.stack(ks), np.stack(vs)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    lt = ctx.tensor(np.asarray(lengths, np.uint32), mi_attn.U32)
    batch = ctx.begin_batch()
    out = batch.attention_decode_batched(ctx.tensor(q), ctx.tensor(k), ctx.tensor(v), lt, cfg, 0)
    batch.finish()
    got = ctx.download(out)
    for b, n in enumerate(lengths):
        ref = oracle_attention(q[b:b + 1], k[b, :n], v[b, :n], hq=hq, hkv=hkv, d=d, off=n - 1)
        assert_parity(got[b:b + 1], ref, label=f"{pattern} sequence {b} L={n}")


def test_c4_batched_decode_seeded(ctx):
    """B=32 sequences, lengths ~ U[1024, 8192], one launch over all of them."""
    c = workloads.case(4)
    B, hq, hkv, d, cap = c.batch, c.q_heads, c.kv_heads, c.head_dim, c.kv_length
    kstore = np.zeros((B, hkv, cap, d), dtype=np.uint16)
    vstore = np.zeros((B, hkv, cap, d), dtype=np.uint16)
    for b in range(B):
        kstore[b, :, : c.lengths[b]] = c.k[b].transpose(1, 0, 2)
        vstore[b, :, : c.lengths[b]] = c.v[b].transpose(1, 0, 2)
    kt, vt = ctx.tensor(kstore), ctx.tensor(vstore)
    view = ((B, cap, hkv, d), (hkv * cap * d, d, cap * d, 1))
    kview, vview = kt.view(*view), vt.view(*view)
    qt = ctx.tensor(c.q)
    lengths = ctx.tensor(c.lengths, mi_attn.U32)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    for block in (0, 256, 1024):
        ctx.take_kernel_profiles()
        ctx.set_kernel_profiling(True)
        try:
            batch = ctx.begin_batch()
            out = batch.attention_decode_batched(qt, kview, vview, lengths, cfg, block)
            batch.finish()
            names = [name for name, _ in ctx.take_kernel_profiles()]
        finally:
            ctx.set_kernel_profiling(False)
        # Default: stream-K MFMA kernel and its merge; explicit split sizes:
        # rows kernel.
        assert names == (["attn_decode_stream", "attn_decode_stream_merge"] if block == 0
                         else ["attn_rows_batched"]), names
        got = ctx.download(out)
        worst = 0.0
        for b in range(B):
            ref = oracle_attention(c.q[b:b + 1], c.k[b], c.v[b], hq=hq, hkv=hkv, d=d,
                                   off=int(c.lengths[b]) - 1)
            worst = max(worst, assert_parity(got[b:b + 1], ref, label=f"seq {b} block {block}"))
        print(f"c4 block={block}: max-abs {worst:.2e}")


def stream_scratch_bytes(ctx, B, hq, hkv, limit=16 << 20):
    """Scratch of a default head_dim-128 batched decode in a buffer of
    `limit` bytes: per head of a unit's head chunk one f32 partial (max, sum,
    acc[128]) in each of 8 fixed slots per unit, one overflow slot per
    workgroup (2 per CU) and unit, and one u32 piece descriptor per unit; or,
    when that exceeds the buffer, the compact layout without the fixed
    slots."""
    g = hq // hkv
    chunk = next(c for c in (16, 8, 4, 2, 1) if g % c == 0)
    units = B * hkv * (g // chunk)
    fixed = ((8 * units + 2 * ctx.compute_units + units) * chunk * 130 + units) * 4
    compact = ((2 * ctx.compute_units + units) * chunk * 130 + units) * 4
    return fixed if fixed <= limit else compact


def _batched_case(ctx, seed, B, hq, hkv, d, cap, lengths):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((B, cap, hkv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((B, cap, hkv, d)).astype(np.float16).view(np.uint16)
    # head-major per sequence: [B, Hkv, cap, D] storage, [B, cap, Hkv, D] view
    kt = ctx.tensor(np.ascontiguousarray(k.transpose(0, 2, 1, 3)))
    vt = ctx.tensor(np.ascontiguousarray(v.transpose(0, 2, 1, 3)))
    view = ((B, cap, hkv, d), (hkv * cap * d, d, cap * d, 1))
    return q, k, v, kt, vt, kt.view(*view), vt.view(*view), ctx.tensor(
        np.asarray(lengths, np.uint32), mi_attn.U32)


def _check_batched(got, q, k, v, lengths, hq, hkv, d, cap, label):
    for b in range(q.shape[0]):
        n = min(int(lengths[b]), cap)
        ref = oracle_attention(q[b:b + 1], k[b, :n], v[b, :n], hq=hq, hkv=hkv, d=d, off=n - 1)
        assert_parity(got[b:b + 1], ref, label=f"{label} seq {b} len {n}")


@pytest.mark.parametrize("hq,hkv,d", [(8, 8, 128), (16, 8, 64), (32, 4, 128), (64, 4, 64)])
def test_batched_decode_gqa_ratios_and_ragged_lengths(ctx, hq, hkv, d):
    """The batched decode (splits merged inside the launch) for GQA 1, 2, 8
    and 16, ragged lengths including 1 and one above the capacity (clamped),
    several split sizes, and two launches in a row (the arrival counters must
    be back at zero after each)."""
    B, cap = 5, 700
    lengths = [1, 700, 333, 64, 900]
    q, k, v, kt, vt, kview, vview, lt = _batched_case(ctx, hq + d, B, hq, hkv, d, cap, lengths)
    qt = ctx.tensor(q)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    for block in (0, 64, 100, 700):
        for rep in range(2):
            batch = ctx.begin_batch()
            out = batch.attention_decode_batched(qt, kview, vview, lt, cfg, block)
            batch.finish()
            _check_batched(ctx.download(out), q, k, v, lengths, hq, hkv, d, cap,
                           f"G={hq // hkv} d={d} block={block} rep={rep}")


@pytest.mark.parametrize("B,hq,hkv,cap,lengths", [
    # GQA 16 (one 16-head chunk), GQA 32 (two chunks), GQA 3 and 12 (chunks
    # of 1 and 4), with zero-length sequences between others.
    (6, 32, 2, 300, [300, 0, 17, 0, 299, 1]),
    (3, 64, 2, 520, [520, 7, 519]),
    (4, 12, 4, 260, [0, 260, 33, 129]),
    (5, 48, 4, 140, [140, 1, 70, 0, 139]),
    # One long sequence: every unit is split over many workgroups, so the
    # last piece merges dozens of partials (several merge rounds).
    (1, 16, 8, 20000, [20000]),
    # Many short sequences: one workgroup's segment covers many units.
    (1024, 8, 2, 24, [(b * 7) % 25 for b in range(1024)]),
    # GQA 16 over 512 sequences (2048 units of 16 heads).
    (512, 64, 4, 20, [1 + (b * 5) % 20 for b in range(512)]),
    # 8192 units.
    (1024, 32, 8, 12, [1 + (b * 3) % 12 for b in range(1024)]),
])
def test_batched_decode_stream_k(ctx, B, hq, hkv, cap, lengths):
    """The default batched decode at head_dim 128 runs the stream-K MFMA
    kernel: workgroups take equal shares of all sequences' keys, and a merge
    launch combines the pieces of every split unit. Checked against the
    oracle for every sequence (a zero-length one gives NaN, as the
    reference's 0/0), three times in a row (every call bit-identical), and
    bit-identical to the no-allocation entry point (its partials in the
    library's fixed buffer) where they fit there."""
    d = 128
    q, k, v, kt, vt, kview, vview, lt = _batched_case(ctx, B + hq + cap, B, hq, hkv, d, cap, lengths)
    qt = ctx.tensor(q)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    first = None
    for rep in range(3):
        ctx.take_kernel_profiles()
        ctx.set_kernel_profiling(True)
        try:
            batch = ctx.begin_batch()
            out = batch.attention_decode_batched(qt, kview, vview, lt, cfg, 0)
            batch.finish()
            names = [name for name, _ in ctx.take_kernel_profiles()]
        finally:
            ctx.set_kernel_profiling(False)
        assert names == ["attn_decode_stream", "attn_decode_stream_merge"], names
        got = ctx.download(out)
        if first is None:
            first = got
        else:
            assert (got == first).all(), f"rep {rep} differs from the first call"
        if rep == 0 and stream_scratch_bytes(ctx, B, hq, hkv) <= 16 << 20:
            two = ctx.empty(q.shape)
            batch = ctx.begin_batch()
            batch.attention_decode_batched_noalloc(qt, kview, vview, lt, cfg, 0, two)
            batch.finish()
            assert (ctx.download(two) == got).all(), "differs from the no-allocation call"
        for b in range(B):
            n = min(int(lengths[b]), cap)
            if B > 64 and b % 41 != 0 and n != 0:
                continue
            if n == 0:
                assert np.isnan(got[b].view(np.float16).astype(np.float32)).all(), f"seq {b}"
                continue
            ref = oracle_attention(q[b:b + 1], k[b, :n], v[b, :n], hq=hq, hkv=hkv, d=d, off=n - 1)
            assert_parity(got[b:b + 1], ref, label=f"B={B} G={hq // hkv} seq {b} len {n} rep {rep}")


def test_batched_decode_stream_k_token_major_cache(ctx):
    """The stream-K kernel on a token-major cache ([B, C, Hkv, D] contiguous,
    so a key row's stride is Hkv * D rather than D)."""
    B, hq, hkv, d, cap = 4, 32, 8, 128, 1000
    lengths = [1000, 3, 517, 0]
    rng = np.random.default_rng(77)
    q = rng.standard_normal((B, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((B, cap, hkv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((B, cap, hkv, d)).astype(np.float16).view(np.uint16)
    kt, vt = ctx.tensor(k), ctx.tensor(v)
    lt = ctx.tensor(np.asarray(lengths, np.uint32), mi_attn.U32)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    ctx.take_kernel_profiles()
    ctx.set_kernel_profiling(True)
    try:
        batch = ctx.begin_batch()
        out = batch.attention_decode_batched(ctx.tensor(q), kt, vt, lt, cfg, 0)
        batch.finish()
        names = [name for name, _ in ctx.take_kernel_profiles()]
    finally:
        ctx.set_kernel_profiling(False)
    assert names == ["attn_decode_stream", "attn_decode_stream_merge"], names
    got = ctx.download(out)
    for b in range(B):
        n = lengths[b]
        if n == 0:
            assert np.isnan(got[b].view(np.float16).astype(np.float32)).all()
            continue
        ref = oracle_attention(q[b:b + 1], k[b, :n], v[b, :n], hq=hq, hkv=hkv, d=d, off=n - 1)
        assert_parity(got[b:b + 1], ref, label=f"token-major seq {b} len {n}")


def test_batched_decode_beyond_the_stream_batch_limit(ctx):
    """Past the stream kernel's batch limit the rows kernel serves the call."""
    B, hq, hkv, d, cap = 1025, 8, 8, 128, 8
    lengths = [1 + b % 8 for b in range(B)]
    q, k, v, kt, vt, kview, vview, lt = _batched_case(ctx, 9, B, hq, hkv, d, cap, lengths)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    ctx.take_kernel_profiles()
    ctx.set_kernel_profiling(True)
    try:
        batch = ctx.begin_batch()
        out = batch.attention_decode_batched(ctx.tensor(q), kview, vview, lt, cfg, 0)
        batch.finish()
        names = [name for name, _ in ctx.take_kernel_profiles()]
    finally:
        ctx.set_kernel_profiling(False)
    assert names == ["attn_rows_batched"], names
    got = ctx.download(out)
    for b in range(0, B, 97):
        n = lengths[b]
        ref = oracle_attention(q[b:b + 1], k[b, :n], v[b, :n], hq=hq, hkv=hkv, d=d, off=n - 1)
        assert_parity(got[b:b + 1], ref, label=f"seq {b}")


@pytest.mark.parametrize("B", [1, 128, 600, 2048])
def test_batched_decode_counter_spacing(ctx, B):
    """The in-launch merge of the rows kernel at every arrival-counter
    spacing: 8 units (one 128-byte line per counter), 1024 (16 words apart),
    4800 (2 words) and 16,384 (the whole buffer, adjacent words). Sampled
    sequences match the oracle, and a second call, which needs every counter
    back at zero, is bit-identical."""
    hq, hkv, d, cap = 8, 8, 64, 40
    lengths = [40 - (b % 13) for b in range(B)]
    q, k, v, kt, vt, kview, vview, lt = _batched_case(ctx, 11 + B, B, hq, hkv, d, cap, lengths)
    qt = ctx.tensor(q)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    outs = []
    for _ in range(2):
        ctx.take_kernel_profiles()
        ctx.set_kernel_profiling(True)
        try:
            batch = ctx.begin_batch()
            out = batch.attention_decode_batched(qt, kview, vview, lt, cfg, 16)
            batch.finish()
            names = [name for name, _ in ctx.take_kernel_profiles()]
        finally:
            ctx.set_kernel_profiling(False)
        assert names == ["attn_rows_batched"], names  # merged inside the launch
        outs.append(ctx.download(out))
    assert np.array_equal(outs[0], outs[1])
    for b in sorted({0, B // 2, B - 1} | set(range(0, B, max(1, B // 16)))):
        n = lengths[b]
        ref = oracle_attention(q[b:b + 1], k[b, :n], v[b, :n], hq=hq, hkv=hkv, d=d, off=n - 1)
        assert_parity(outs[0][b:b + 1], ref, label=f"B={B} seq {b}")


def test_batched_decode_beyond_the_arrival_counters(ctx):
    """More (sequence, KV head) units than the context's arrival counters:
    the split partials are merged by a second launch instead (16,800 units
    against 16,384 counters)."""
    B, hq, hkv, d, cap = 2100, 8, 8, 64, 40
    lengths = [40 - (b % 13) for b in range(B)]
    q, k, v, kt, vt, kview, vview, lt = _batched_case(ctx, 5, B, hq, hkv, d, cap, lengths)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    ctx.take_kernel_profiles()
    ctx.set_kernel_profiling(True)
    try:
        batch = ctx.begin_batch()
        out = batch.attention_decode_batched(ctx.tensor(q), kview, vview, lt, cfg, 16)
        batch.finish()
        names = [name for name, _ in ctx.take_kernel_profiles()]
    finally:
        ctx.set_kernel_profiling(False)
    assert names == ["attn_rows_batched", "attn_merge"]
    got = ctx.download(out)
    for b in range(0, B, 37):
        n = lengths[b]
        ref = oracle_attention(q[b:b + 1], k[b, :n], v[b, :n], hq=hq, hkv=hkv, d=d, off=n - 1)
        assert_parity(got[b:b + 1], ref, label=f"seq {b}")


# --------------------------------------------------------- invariants -----

def test_masked_keys_do_not_influence_output(ctx):
    rng = np.random.default_rng(7)
    T, L, hq, hkv, d, off = 3, 300, 16, 8, 128, 200
    q = rng.standard_normal((T, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    geo = dict(hq=hq, hkv=hkv, d=d, off=off)
    k2, v2 = k.copy(), v.copy()
    k2[off + T:] = np.float16(30.0).view(np.uint16)
    v2[off + T:] = np.float16(-9.0).view(np.uint16)
    for kind in ("tiled", "flash-prefill", "reference"):
        a = run_attention(ctx, q, k, v, kind=kind, **geo)
        b = run_attention(ctx, q, k2, v2, kind=kind, **geo)
        assert (a == b).all(), kind
    a = run_attention(ctx, q[:1], k, v, kind="flash-decode", **geo)
    b = run_attention(ctx, q[:1], k2, v2, kind="flash-decode", **geo)
    assert (a == b).all()


def test_layouts_give_identical_bits(ctx):
    c = workloads.case(2)
    geo = dict(hq=c.q_heads, hkv=c.kv_heads, d=c.head_dim, off=c.query_offset)
    a = run_attention(ctx, c.q, c.k, c.v, kind="flash-decode", layout="head_major", **geo)
    b = run_attention(ctx, c.q, c.k, c.v, kind="flash-decode", layout="position_major", **geo)
    assert (a == b).all()


def test_decode_matches_last_prefill_row_and_chunked_prefill(ctx):
    rng = np.random.default_rng(9)
    T, hq, hkv, d = 96, 16, 8, 128
    q = rng.standard_normal((T, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((T, hkv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((T, hkv, d)).astype(np.float16).view(np.uint16)
    full = run_attention(ctx, q, k, v, kind="flash-prefill", hq=hq, hkv=hkv, d=d, off=0)
    dec = run_attention(ctx, q[-1:], k, v, kind="flash-decode", hq=hq, hkv=hkv, d=d, off=T - 1)
    assert max_abs(dec, f16(full[-1:])) <= 2 * TOL
    P = 40
    chunk = run_attention(ctx, q[P:], k, v, kind="flash-prefill", hq=hq, hkv=hkv, d=d, off=P)
    assert max_abs(chunk, f16(full[P:])) <= 2 * TOL


def test_gqa_equals_mha_with_repeated_heads(ctx):
    rng = np.random.default_rng(11)
    T, L, hq, hkv, d = 4, 500, 32, 8, 128
    q = rng.standard_normal((T, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    gqa = run_attention(ctx, q, k, v, kind="tiled", hq=hq, hkv=hkv, d=d, off=L - T)
    mha = run_attention(ctx, q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), kind="tiled",
                        hq=hq, hkv=hq, d=d, off=L - T)
    assert max_abs(gqa, f16(mha)) <= 2 * TOL


# ------------------------------------------- negative position strides ----

@pytest.mark.parametrize("kind", ["flash-prefill", "tiled", "flash-decode"])
def test_reversed_cache_views(ctx, kind):
    """K/V views whose position stride is negative (the last position first
    in memory): the MFMA kernels' 32-bit tile offsets cannot address them, so
    the plan takes the rows kernel (64-bit offsets); outputs match the
    oracle and the forward layout."""
    rng = np.random.default_rng(31)
    hq, hkv, d = 16, 8, 128
    T, off = (300, 37) if kind != "flash-decode" else (1, 700)
    L = off + T
    q = rng.standard_normal((T, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((L, hkv, d)).astype(np.float16).view(np.uint16)
    geo = dict(hq=hq, hkv=hkv, d=d, off=off)
    ko, kview = upload_kv(ctx, k, "reversed")
    assert kview.strides[0] < 0
    info = ctx.plan(ctx.tensor(q), kview, kview, mi_attn.AttentionConfig(hq, hkv, d, True, off),
                    KINDS[kind])
    assert info["kernel"] == "attn_rows", info
    out = run_attention(ctx, q, k, v, kind=kind, layout="reversed", **geo)
    ref = oracle_attention(q, k, v, **geo)
    assert_parity(out, ref, label=f"reversed/{kind}")


def test_batched_decode_reversed_cache_takes_the_rows_kernel(ctx):
    """A batched decode over caches with a negative position stride runs the
    rows kernel (the stream-K kernel's per-lane offsets are unsigned 32-bit)
    and matches the oracle for every sequence."""
    B, hq, hkv, d, cap = 3, 32, 8, 128, 600
    lengths = [600, 17, 333]
    rng = np.random.default_rng(41)
    q = rng.standard_normal((B, hq, d)).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((B, cap, hkv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((B, cap, hkv, d)).astype(np.float16).view(np.uint16)
    # storage [B, Hkv, cap, D] with positions reversed; view [B, cap, Hkv, D]
    kt = ctx.tensor(np.ascontiguousarray(k[:, ::-1].transpose(0, 2, 1, 3)))
    vt = ctx.tensor(np.ascontiguousarray(v[:, ::-1].transpose(0, 2, 1, 3)))
    strides = (hkv * cap * d, -d, cap * d, 1)
    kview = kt.view((B, cap, hkv, d), strides, offset=(cap - 1) * d)
    vview = vt.view((B, cap, hkv, d), strides, offset=(cap - 1) * d)
    lt = ctx.tensor(np.asarray(lengths, np.uint32), mi_attn.U32)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    ctx.take_kernel_profiles()
    ctx.set_kernel_profiling(True)
    try:
        batch = ctx.begin_batch()
        out = batch.attention_decode_batched(ctx.tensor(q), kview, vview, lt, cfg, 0)
        batch.finish()
        names = [name for name, _ in ctx.take_kernel_profiles()]
    finally:
        ctx.set_kernel_profiling(False)
    assert names == ["attn_rows_batched"], names
    got = ctx.download(out)
    for b in range(B):
        n = lengths[b]
        ref = oracle_attention(q[b:b + 1], k[b, :n], v[b, :n], hq=hq, hkv=hkv, d=d, off=n - 1)
        assert_parity(got[b:b + 1], ref, label=f"reversed seq {b} len {n}")
