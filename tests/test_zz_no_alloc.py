"""The entry point that allocates nothing (mi_attention_decode_batched_noalloc)
against the existing mi_attention_decode_batched, through the C ABI.

Its split partials live in the library's fixed per-GPU buffer instead of the
batch arena. Outputs must equal the arena entry point's bit for bit (same
kernels, same partial layout, same merge order) and meet the oracle bar, on
two calls in a row, the second smaller; the buffer keeps the first call's
contents, so the second call also shows that nothing stale leaks in.
"""
from __future__ import annotations

import numpy as np
import pytest

import mi_attn
import workloads
from helpers import assert_parity, oracle_attention

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nctx():
    # Its own context: the test runs the same alone or after the others.
    context = mi_attn.Context(0)
    yield context
    context.close()


def _cache(ctx, k, v, lengths, cap):
    """Per-sequence head-major caches [B, Hkv, cap, D] as [B, cap, Hkv, D] views."""
    B, hkv, d = len(k), k[0].shape[1], k[0].shape[2]
    kstore = np.zeros((B, hkv, cap, d), dtype=np.uint16)
    vstore = np.zeros((B, hkv, cap, d), dtype=np.uint16)
    for b in range(B):
        kstore[b, :, :lengths[b]] = k[b][:lengths[b]].transpose(1, 0, 2)
        vstore[b, :, :lengths[b]] = v[b][:lengths[b]].transpose(1, 0, 2)
    kt, vt = ctx.tensor(kstore), ctx.tensor(vstore)
    view = ((B, cap, hkv, d), (hkv * cap * d, d, cap * d, 1))
    return kt, vt, kt.view(*view), vt.view(*view)


def _both(ctx, q, kview, vview, lengths, cfg, block):
    """(arena entry point output, no-allocation entry point output, kernels run)."""
    qt = ctx.tensor(q)
    lt = ctx.tensor(np.asarray(lengths, np.uint32), mi_attn.U32)
    ref_out, out = ctx.empty(q.shape), ctx.empty(q.shape)
    batch = ctx.begin_batch()
    batch.attention_decode_batched(qt, kview, vview, lt, cfg, block, out=ref_out)
    batch.finish()
    ctx.take_kernel_profiles()
    ctx.set_kernel_profiling(True)
    try:
        batch = ctx.begin_batch()
        before = ctx.allocated_bytes()
        batch.attention_decode_batched_noalloc(qt, kview, vview, lt, cfg, block, out)
        assert ctx.allocated_bytes() == before, "the call allocated device memory"
        batch.finish()
        events = ctx.take_kernel_profiles()
    finally:
        ctx.set_kernel_profiling(False)
    assert events == [], "the no-allocation call creates no profiling events"
    return ctx.download(ref_out), ctx.download(out)


@pytest.mark.parametrize("block", [0, 512])
def test_no_alloc_matches_the_arena_entry_point_on_two_calls(nctx, block):
    """c4 (32 sequences, GQA 4) and then a smaller ragged batch (5 sequences,
    GQA 8, one of length zero): bit-identical to mi_attention_decode_batched
    and within 2e-3 of the oracle. block 0 runs the stream-K kernel, 512 the
    rows kernel with its in-launch merge."""
    c = workloads.case(4)
    kt, vt, kview, vview = _cache(nctx, c.k, c.v, c.lengths, c.kv_length)
    cfg = mi_attn.AttentionConfig(c.q_heads, c.kv_heads, c.head_dim, True, 0)
    ref, got = _both(nctx, c.q, kview, vview, c.lengths, cfg, block)
    assert (got == ref).all(), "first call differs from the arena entry point"
    for b in range(0, c.batch, 3):
        oracle = oracle_attention(c.q[b:b + 1], c.k[b], c.v[b], hq=c.q_heads, hkv=c.kv_heads,
                                  d=c.head_dim, off=int(c.lengths[b]) - 1)
        assert_parity(got[b:b + 1], oracle, label=f"c4 seq {b}")
    kt.free(), vt.free()

    rng = np.random.default_rng(3)
    B, hq, hkv, d, cap = 5, 64, 8, 128, 900
    lengths = [900, 0, 1, 517, 130]
    q = rng.standard_normal((B, hq, d)).astype(np.float16).view(np.uint16)
    k = [rng.standard_normal((cap, hkv, d)).astype(np.float16).view(np.uint16) for _ in range(B)]
    v = [rng.standard_normal((cap, hkv, d)).astype(np.float16).view(np.uint16) for _ in range(B)]
    kt, vt, kview, vview = _cache(nctx, k, v, lengths, cap)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    ref, got = _both(nctx, q, kview, vview, lengths, cfg, block)
    assert (got.view(np.uint16) == ref.view(np.uint16)).all(), "second call differs"
    for b in range(B):
        n = lengths[b]
        if n == 0:
            assert np.isnan(got[b].view(np.float16).astype(np.float32)).all()
            continue
        oracle = oracle_attention(q[b:b + 1], k[b][:n], v[b][:n], hq=hq, hkv=hkv, d=d, off=n - 1)
        assert_parity(got[b:b + 1], oracle, label=f"small seq {b}")
    kt.free(), vt.free()


def test_no_alloc_compact_layout_when_unit_slots_do_not_fit(nctx):
    """128 sequences x 8 KV heads (1024 units of 4 query heads): the fixed 8
    slots per unit would need 20 MB, so the no-allocation call takes the
    compact layout (every piece in an overflow slot, 3.2 MB). Bit-identical
    to the arena entry point (fixed slots, same merge order) on two calls,
    and within 2e-3 of the oracle on sampled sequences."""
    B, hq, hkv, d, cap = 128, 32, 8, 128, 600
    rng = np.random.default_rng(11)
    lengths = [int(x) for x in rng.integers(1, cap + 1, B)]
    lengths[5] = 0
    q = rng.standard_normal((B, hq, d)).astype(np.float16).view(np.uint16)
    k = [rng.standard_normal((cap, hkv, d)).astype(np.float16).view(np.uint16) for _ in range(B)]
    v = [rng.standard_normal((cap, hkv, d)).astype(np.float16).view(np.uint16) for _ in range(B)]
    kt, vt, kview, vview = _cache(nctx, k, v, lengths, cap)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    for rep in range(2):
        ref, got = _both(nctx, q, kview, vview, lengths, cfg, 0)
        assert (got.view(np.uint16) == ref.view(np.uint16)).all(), f"call {rep} differs"
    for b in (0, 5, 37, 127):
        n = lengths[b]
        if n == 0:
            assert np.isnan(got[b].view(np.float16).astype(np.float32)).all()
            continue
        oracle = oracle_attention(q[b:b + 1], k[b][:n], v[b][:n], hq=hq, hkv=hkv, d=d, off=n - 1)
        assert_parity(got[b:b + 1], oracle, label=f"compact seq {b}")
    kt.free(), vt.free()


def test_no_alloc_rejects_partials_beyond_its_buffer(nctx):
    """A call whose partials need more than the fixed 16 MiB fails before any
    launch, with the sizes in the message; the arena entry point runs it."""
    B, hq, hkv, d, cap = 1024, 64, 4, 128, 1
    # stream-K: (512 workgroups + 4096 units) x 16 heads x 130 floats = 38 MB, even
    # in the compact layout (no fixed slots per unit)
    rng = np.random.default_rng(9)
    q = rng.standard_normal((B, hq, d)).astype(np.float16).view(np.uint16)
    kv = rng.standard_normal((B, cap, hkv, d)).astype(np.float16).view(np.uint16)
    qt, kt = nctx.tensor(q), nctx.tensor(kv)
    lt = nctx.tensor(np.ones(B, np.uint32), mi_attn.U32)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    out = nctx.empty(q.shape)
    batch = nctx.begin_batch()
    with pytest.raises(mi_attn.MiError) as err:
        batch.attention_decode_batched_noalloc(qt, kt, kt, lt, cfg, 0, out)
    batch.abandon()
    assert err.value.name == "MI_ERR_RESOURCE"
    assert "exceeds the no-allocation buffer of 16777216 bytes" in err.value.message
    ok = nctx.empty(q.shape)
    batch = nctx.begin_batch()
    batch.attention_decode_batched(qt, kt, kt, lt, cfg, 0, out=ok)
    batch.finish()
    got = nctx.download(ok)
    # one key per sequence: the output is that key's value row, per head
    expect = np.repeat(kv[:, 0], hq // hkv, axis=1)
    assert (got == expect).all()


def test_no_alloc_two_contexts_alternating(nctx):
    """Two contexts on one GPU share the fixed buffer. Calls that alternate
    in stream order (each waited on before the other context calls) both
    succeed and equal the arena entry point bit for bit: the second context
    takes the buffer over once the first one's call has finished."""
    other = mi_attn.Context(0)
    try:
        rng = np.random.default_rng(17)
        B, hq, hkv, d, cap = 6, 32, 8, 128, 1500
        lengths = [1500, 3, 777, 1024, 64, 1299]
        q = rng.standard_normal((B, hq, d)).astype(np.float16).view(np.uint16)
        k = [rng.standard_normal((cap, hkv, d)).astype(np.float16).view(np.uint16)
             for _ in range(B)]
        v = [rng.standard_normal((cap, hkv, d)).astype(np.float16).view(np.uint16)
             for _ in range(B)]
        cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
        views = {id(c): _cache(c, k, v, lengths, cap) for c in (nctx, other)}
        for rep in range(2):
            for context in (nctx, other):
                _, _, kview, vview = views[id(context)]
                ref, got = _both(context, q, kview, vview, lengths, cfg, 0)
                assert (got == ref).all(), f"round {rep}: the two entry points differ"
        for context in (nctx, other):
            kt, vt, _, _ = views[id(context)]
            kt.free(), vt.free()
    finally:
        other.close()
