"""GPU tests of the head-major KV cache: append, fused Q/K norm + RoPE with
K-append, cache bookkeeping, and a decode loop in forward_layer's order
(crates/metal-infer-models/src/qwen3.rs:704-750)."""
from __future__ import annotations

import numpy as np
import pytest

import mi_attn
import oracle
from helpers import TOL, assert_parity, f16, oracle_attention

pytestmark = pytest.mark.gpu


def rand(seed, shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(
        np.float16).view(np.uint16)


def test_copy_into_cache_is_bit_exact_head_major(ctx):
    hkv, d, cap = 8, 128, 64
    cache = ctx.kv_cache(1, hkv, d, cap)
    key, value = cache.layer(0)
    assert key.shape == (cap, hkv, d) and key.strides == (d, cap * d, 1)
    sentinel = np.full((cap, hkv, d), 0x7bff, dtype=np.uint16)
    ctx.upload(key, sentinel)
    src = rand(1, (5, hkv, d))
    ctx.copy_into_cache(ctx.tensor(src), key, 17)
    got = ctx.download(key)
    expected = sentinel.copy()
    expected[17:22] = src
    assert (got == expected).all()
    # the storage really is head-major: [Hkv, cap, D]
    raw = ctx.download(key.view((hkv, cap, d), (cap * d, d, 1)))
    assert (raw[:, 17:22] == src.transpose(1, 0, 2)).all()
    cache.close()


def test_copy_into_cache_errors(ctx):
    cache = ctx.kv_cache(1, 2, 16, 8)
    key, _ = cache.layer(0)
    batch = ctx.begin_batch()
    with pytest.raises(mi_attn.MiError, match="KV cache capacity exceeded"):
        batch.copy_into_cache(ctx.tensor(rand(2, (3, 2, 16))), key, 6)
    with pytest.raises(mi_attn.MiError, match="incompatible"):
        batch.copy_into_cache(ctx.tensor(rand(2, (3, 4, 16))), key, 0)
    with pytest.raises(mi_attn.MiError) as err:
        batch.copy_into_cache(ctx.tensor(np.zeros((3, 2, 16), np.float32), mi_attn.F32), key, 0)
    assert err.value.name == "MI_ERR_DTYPE"
    batch.abandon()
    cache.close()


def test_kv_cache_bookkeeping(ctx):
    with pytest.raises(mi_attn.MiError, match="capacity must be non-zero"):
        ctx.kv_cache(2, 8, 128, 0)
    cache = ctx.kv_cache(28, 8, 128, 2048)
    assert len(cache) == 0 and cache.capacity == 2048
    cache.set_len(513)
    assert len(cache) == 513
    with pytest.raises(mi_attn.MiError) as err:
        cache.set_len(2049)
    assert err.value.name == "MI_ERR_CACHE_CAPACITY"
    cache.reset()
    assert len(cache) == 0
    k0, v0 = cache.layer(0)
    k27, _ = cache.layer(27)
    assert v0.data_ptr - k0.data_ptr == 8 * 2048 * 128 * 2
    assert k27.data_ptr - k0.data_ptr == 27 * 2 * 8 * 2048 * 128 * 2
    with pytest.raises(mi_attn.MiError, match="missing KV cache layer"):
        cache.layer(28)
    cache.close()


def _qk_case(ctx, q, k, qw, kw, offset, theta, eps, cap):
    T, hkv, d = k.shape
    cache = ctx.kv_cache(1, hkv, d, cap)
    key, _ = cache.layer(0)
    ctx.upload(key, np.zeros((cap, hkv, d), dtype=np.uint16))
    batch = ctx.begin_batch()
    q_out = batch.qk_norm_rope_cache(ctx.tensor(q), ctx.tensor(k), ctx.tensor(qw), ctx.tensor(kw),
                                     key, mi_attn.QkNormRopeCacheConfig(offset, theta, eps))
    batch.finish()
    got_q, got_cache = ctx.download(q_out), ctx.download(key)
    cache.close()
    return got_q, got_cache


def test_qk_norm_rope_cache_reference_case(ctx):
    """gpu.rs:540-576: Q = i/16 - 1, K = i/12 - 0.5, weights 0.75 + i/16,
    offset 1; K lands in cache rows 1..2 and nowhere else."""
    f = np.float32
    q = (np.arange(32, dtype=f) / f(16) - f(1)).astype(np.float16).view(np.uint16).reshape(2, 2, 8)
    k = (np.arange(16, dtype=f) / f(12) - f(0.5)).astype(np.float16).view(np.uint16).reshape(2, 1, 8)
    w = (f(0.75) + np.arange(8, dtype=f) / f(16)).astype(np.float16).view(np.uint16)
    got_q, got_cache = _qk_case(ctx, q, k, w, w, 1, 10_000.0, 1e-6, 4)
    want_q, want_k = oracle.qk_norm_rope(q, k, w, w, offset=1, theta=10_000.0, epsilon=1e-6)
    assert np.abs(got_q.astype(np.int32) - want_q.astype(np.int32)).max() <= 1
    assert np.abs(got_cache[1:3].astype(np.int32) - want_k.astype(np.int32)).max() <= 1
    assert (got_cache[0] == 0).all() and (got_cache[3] == 0).all()


@pytest.mark.parametrize("offset", [0, 300, 16384])
def test_qk_norm_rope_cache_seeded(ctx, offset):
    T, hq, hkv, d, theta, eps = 7, 16, 8, 128, 1_000_000.0, 1e-6
    q, k = rand(3, (T, hq, d)), rand(4, (T, hkv, d))
    qw = (1 + 0.1 * np.random.default_rng(5).standard_normal(d)).astype(np.float16).view(np.uint16)
    kw = (1 + 0.1 * np.random.default_rng(6).standard_normal(d)).astype(np.float16).view(np.uint16)
    got_q, got_cache = _qk_case(ctx, q, k, qw, kw, offset, theta, eps, offset + T)
    want_q, want_k = oracle.qk_norm_rope(q, k, qw, kw, offset=offset, theta=theta, epsilon=eps)
    # f32 sin/cos of the same f32 angle: at most one f16 ulp apart, except
    # where the rotation cancels (checked against the pair magnitude).
    for got, want in ((got_q, want_q), (got_cache[offset:], want_k)):
        diff = np.abs(f16(got).astype(np.float64) - f16(want))
        mag = np.abs(f16(want)).max()
        assert diff.max() <= max(2e-3, 2e-3 * mag), (offset, diff.max())


@pytest.mark.parametrize("T,hq,hkv,d,offset", [
    (37, 20, 3, 128, 11),   # 32 rows per wave: one ragged chunk, odd KV heads
    (17, 70, 8, 128, 3),    # 32 rows per wave: three Q chunks, the last of 6 rows
    (19, 8, 2, 256, 500),   # head_dim 256, 16 rows per wave
    (5, 6, 1, 256, 0),      # few tokens: four rows per wave
    (3, 5, 3, 128, 2),      # odd counts in the four-row steps
])
def test_qk_norm_rope_cache_row_layouts(ctx, T, hq, hkv, d, offset):
    theta, eps = 1_000_000.0, 1e-6
    q, k = rand(60 + T, (T, hq, d)), rand(61 + T, (T, hkv, d))
    qw = (1 + 0.1 * np.random.default_rng(62).standard_normal(d)).astype(np.float16).view(np.uint16)
    kw = (1 + 0.1 * np.random.default_rng(63).standard_normal(d)).astype(np.float16).view(np.uint16)
    got_q, got_cache = _qk_case(ctx, q, k, qw, kw, offset, theta, eps, offset + T + 2)
    want_q, want_k = oracle.qk_norm_rope(q, k, qw, kw, offset=offset, theta=theta, epsilon=eps)
    for got, want in ((got_q, want_q), (got_cache[offset:offset + T], want_k)):
        diff = np.abs(f16(got).astype(np.float64) - f16(want))
        mag = np.abs(f16(want)).max()
        assert diff.max() <= max(2e-3, 2e-3 * mag), (T, hq, hkv, d, diff.max())
    assert (got_cache[:offset] == 0).all() and (got_cache[offset + T:] == 0).all()


def test_decode_loop_in_forward_layer_order(ctx):
    """Per step: Q/K norm+RoPE with K into the cache, V appended, then
    attention over the cache prefix (qwen3.rs:704-750), all in one batch."""
    hq, hkv, d, cap, prompt, steps = 16, 8, 128, 512, 300, 4
    theta, eps = 1_000_000.0, 1e-6
    qw = np.full(d, np.float16(1.0).view(np.uint16), dtype=np.uint16)
    cache = ctx.kv_cache(1, hkv, d, cap)
    key, value = cache.layer(0)
    k_rows, v_rows = [], []
    qwt, kwt = ctx.tensor(qw), ctx.tensor(qw)
    for step in range(steps):
        T = prompt if step == 0 else 1
        offset = len(cache)
        q, k, v = rand(10 + step, (T, hq, d)), rand(20 + step, (T, hkv, d)), rand(30 + step, (T, hkv, d))
        batch = ctx.begin_batch()
        q_rot = batch.qk_norm_rope_cache(ctx.tensor(q), ctx.tensor(k), qwt, kwt, key,
                                         mi_attn.QkNormRopeCacheConfig(offset, theta, eps))
        batch.copy_into_cache(ctx.tensor(v), value, offset)
        active = offset + T
        kind = mi_attn.attention_kind_for_tokens(mi_attn.TILED, T, active, hq // hkv)
        cfg = mi_attn.AttentionConfig(hq, hkv, d, True, offset)
        out = batch.attention(q_rot, key.prefix(active), value.prefix(active), cfg, kind)
        batch.finish()
        cache.set_len(active)
        want_q, want_k = oracle.qk_norm_rope(q, k, qw, qw, offset=offset, theta=theta, epsilon=eps)
        k_rows.append(want_k)
        v_rows.append(v)
        got_q = ctx.download(q_rot)
        kk, vv = np.concatenate(k_rows), np.concatenate(v_rows)
        ref = oracle_attention(got_q, ctx.download(key.prefix(active)), vv, hq=hq, hkv=hkv, d=d,
                               off=offset)
        assert_parity(ctx.download(out), ref, label=f"step {step} kind {kind}")
        # RoPE may cancel to near zero, so compare absolutely, scaled by the
        # rows' magnitude (one f16 ulp at |x| < 4 is <= 2e-3).
        got_k = f16(ctx.download(key.prefix(active))).astype(np.float64)
        assert np.abs(got_k - f16(kk)).max() <= 2e-3 * max(1.0, np.abs(f16(kk)).max() / 4)
    cache.close()


# ------------------------------------- fused Q/K transform + value append --

def _fused_vs_pair(ctx, T, offset, capacity, hq=16, hkv=8, d=128):
    q, k, v = rand(80 + T, (T, hq, d)), rand(81 + T, (T, hkv, d)), rand(82 + T, (T, hkv, d))
    qw = (1 + 0.1 * np.random.default_rng(83).standard_normal(d)).astype(np.float16).view(np.uint16)
    kw = (1 + 0.1 * np.random.default_rng(84).standard_normal(d)).astype(np.float16).view(np.uint16)
    qt, kt, vt, qwt, kwt = (ctx.tensor(a) for a in (q, k, v, qw, kw))
    cfg = mi_attn.QkNormRopeCacheConfig(offset, 1_000_000.0, 1e-6)
    results = []
    for fused in (False, True):
        cache = ctx.kv_cache(1, hkv, d, capacity)
        key, value = cache.layer(0)
        # The cache starts uninitialised (like the reference's context.empty):
        # a sentinel shows which rows each path writes.
        ctx.upload(key, np.full((capacity, hkv, d), 0x7bff, dtype=np.uint16))
        ctx.upload(value, np.full((capacity, hkv, d), 0x7bfe, dtype=np.uint16))
        batch = ctx.begin_batch()
        if fused:
            q_out = batch.qk_norm_rope_cache_value(qt, kt, vt, qwt, kwt, key, value, cfg)
        else:
            q_out = batch.qk_norm_rope_cache(qt, kt, qwt, kwt, key, cfg)
            batch.copy_into_cache(vt, value, offset)
        batch.finish()
        results.append((ctx.download(q_out), ctx.download(key), ctx.download(value)))
        cache.close()
    return results, v


@pytest.mark.parametrize("T,offset,capacity,hq,hkv,d", [
    (1, 2047, 2048, 16, 8, 128), (5, 300, 512, 16, 8, 128), (3, 0, 3, 16, 8, 128),
    (5, 7, 16, 6, 3, 256),       # odd number of value rows
    (37, 100, 160, 20, 3, 128),  # 16 rows per wave
    (4, 1, 8, 4, 2, 64),         # head_dim 64: the generic kernel
])
def test_fused_value_append_matches_the_two_calls(ctx, T, offset, capacity, hq, hkv, d):
    """mi_qk_norm_rope_cache_value == qk_norm_rope_cache then
    copy_into_cache(value), bit for bit (qwen3.rs:704-728 order)."""
    (pair, fused), v = _fused_vs_pair(ctx, T, offset, capacity, hq, hkv, d)
    for a, b in zip(pair, fused):
        assert (a == b).all()
    assert (fused[2][offset:offset + T] == v).all()
    untouched = np.ones(capacity, bool)
    untouched[offset:offset + T] = False
    assert (fused[1][untouched] == 0x7bff).all() and (fused[2][untouched] == 0x7bfe).all()


def test_fused_value_append_errors(ctx):
    hq, hkv, d = 4, 2, 64
    cache = ctx.kv_cache(1, hkv, d, 8)
    key, value = cache.layer(0)
    q, k = ctx.tensor(rand(1, (2, hq, d))), ctx.tensor(rand(2, (2, hkv, d)))
    w = ctx.tensor(rand(3, (d,)))
    cfg = mi_attn.QkNormRopeCacheConfig(0, 1e4, 1e-6)
    batch = ctx.begin_batch()
    with pytest.raises(mi_attn.MiError, match="KV source/cache shapes are incompatible"):
        batch.qk_norm_rope_cache_value(q, k, ctx.tensor(rand(4, (2, 1, d))), w, w, key, value, cfg)
    with pytest.raises(mi_attn.MiError, match="value rows must have the key's shape"):
        batch.qk_norm_rope_cache_value(q, k, ctx.tensor(rand(5, (1, hkv, d))), w, w, key, value, cfg)
    with pytest.raises(mi_attn.MiError, match="KV cache capacity exceeded"):
        small = ctx.kv_cache(1, hkv, d, 16)
        _, small_value = small.layer(0)
        batch.qk_norm_rope_cache_value(q, k, ctx.tensor(rand(6, (2, hkv, d))), w, w, key,
                                       small_value.prefix(1), cfg)
    batch.abandon()
    small.close()
    cache.close()


@pytest.mark.parametrize("one_launch", [False, True])
def test_captured_fused_decode_step_replays_match_eager(ctx, one_launch):
    """Replays of a captured step (the two-kernel form, or
    mi_decode_step_attention) equal the eager step bit for bit, each replay
    after eager work of its own."""
    hq, hkv, d, cap, pos = 16, 8, 128, 1024, 600
    cache = ctx.kv_cache(1, hkv, d, cap)
    key, value = cache.layer(0)
    ctx.copy_into_cache(ctx.tensor(rand(90, (pos, hkv, d))), key, 0)
    ctx.copy_into_cache(ctx.tensor(rand(91, (pos, hkv, d))), value, 0)
    w = ctx.tensor(rand(92, (d,), scale=0.3))
    q_in, k_in, v_in = ctx.empty((1, hq, d)), ctx.empty((1, hkv, d)), ctx.empty((1, hkv, d))
    cfg = mi_attn.QkNormRopeCacheConfig(pos, 1_000_000.0, 1e-6)
    acfg = mi_attn.AttentionConfig(hq, hkv, d, True, pos)

    def step(batch, out=None):
        if one_launch:
            return batch.decode_step_attention(q_in, k_in, v_in, w, w, key, value, cfg, acfg,
                                               out=out)
        q_rot = batch.qk_norm_rope_cache_value(q_in, k_in, v_in, w, w, key, value, cfg)
        return batch.attention(q_rot, key.prefix(pos + 1), value.prefix(pos + 1), acfg,
                               mi_attn.FLASH_DECODE, out=out)

    o_graph = ctx.empty((1, hq, d))
    capture = ctx.begin_capture()
    step(capture, o_graph)
    graph = capture.end_capture()
    for rep in range(3):
        ctx.upload(q_in, rand(93 + rep, (1, hq, d)))
        ctx.upload(k_in, rand(96 + rep, (1, hkv, d)))
        ctx.upload(v_in, rand(99 + rep, (1, hkv, d)))
        graph.launch()
        ctx.synchronize()
        got = ctx.download(o_graph)
        batch = ctx.begin_batch()
        eager = step(batch)
        batch.finish()
        assert (got == ctx.download(eager)).all(), f"replay {rep}"
        assert (ctx.download(value.prefix(pos + 1))[pos] == ctx.download(v_in)[0]).all()
    graph.destroy()
    cache.close()


# ------------------------------------------- one-launch decode attention step --

@pytest.mark.parametrize("hq,hkv,d,pos", [
    (16, 8, 128, 2047),   # c2: 16 splits merged in the launch
    (32, 8, 128, 300),    # GQA 4
    (64, 8, 128, 100),    # GQA 8, one split
    (16, 8, 128, 0),      # the new token is the only key
    (8, 8, 128, 1000),    # MHA
    (8, 4, 64, 500),      # head_dim 64: the three calls' kernels
])
def test_decode_step_matches_the_three_calls(ctx, hq, hkv, d, pos):
    """mi_decode_step_attention == qk_norm_rope_cache_value then FlashDecode
    over the prefix [0, pos] (qwen3.rs:704-750), and both match the oracle."""
    cap, theta, eps = pos + 3, 1_000_000.0, 1e-6
    seed = 7 * pos + hq
    q, k, v = rand(seed, (1, hq, d)), rand(seed + 1, (1, hkv, d)), rand(seed + 2, (1, hkv, d))
    qw = (1 + 0.1 * np.random.default_rng(seed + 3).standard_normal(d)).astype(np.float16).view(np.uint16)
    kw = (1 + 0.1 * np.random.default_rng(seed + 4).standard_normal(d)).astype(np.float16).view(np.uint16)
    k_hist, v_hist = rand(seed + 5, (cap, hkv, d)), rand(seed + 6, (cap, hkv, d))
    qt, kt, vt, qwt, kwt = (ctx.tensor(a) for a in (q, k, v, qw, kw))
    qk_cfg = mi_attn.QkNormRopeCacheConfig(pos, theta, eps)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, pos)
    results = []
    for fused in (False, True):
        cache = ctx.kv_cache(1, hkv, d, cap)
        key, value = cache.layer(0)
        ctx.upload(key, k_hist)
        ctx.upload(value, v_hist)
        ctx.take_kernel_profiles()
        ctx.set_kernel_profiling(True)
        try:
            batch = ctx.begin_batch()
            if fused:
                out = batch.decode_step_attention(qt, kt, vt, qwt, kwt, key, value, qk_cfg, cfg)
            else:
                q_rot = batch.qk_norm_rope_cache_value(qt, kt, vt, qwt, kwt, key, value, qk_cfg)
                out = batch.attention(q_rot, key.prefix(pos + 1), value.prefix(pos + 1), cfg,
                                      mi_attn.FLASH_DECODE)
            batch.finish()
            names = [name for name, _ in ctx.take_kernel_profiles()]
        finally:
            ctx.set_kernel_profiling(False)
        if fused:
            want = ["attn_decode_step"] if d == 128 else ["qk_norm_rope_cache", "attn_rows"]
            assert names[:len(want)] == want, names
        results.append((ctx.download(out), ctx.download(key), ctx.download(value)))
        cache.close()
    (out_pair, key_pair, value_pair), (out_step, key_step, value_step) = results
    # Rows other than pos are untouched; the value row is copied bit for bit.
    others = np.ones(cap, bool)
    others[pos] = False
    assert (key_step[others] == k_hist[others]).all() and (value_step[others] == v_hist[others]).all()
    assert (value_step[pos] == v[0]).all() and (value_pair[pos] == v[0]).all()
    # The key transform sums the squares in another order: within one f16 ulp.
    assert np.abs(key_step[pos].astype(np.int32) - key_pair[pos].astype(np.int32)).max() <= 1
    want_q, want_k = oracle.qk_norm_rope(q, k, qw, kw, offset=pos, theta=theta, epsilon=eps)
    kk = key_step[:pos + 1].copy()
    ref = oracle_attention(want_q, kk, value_step[:pos + 1], hq=hq, hkv=hkv, d=d, off=pos)
    assert_parity(out_step, ref, label=f"step {hq}/{hkv}/{d} pos {pos}")
    assert np.abs(f16(out_step).astype(np.float64) - f16(out_pair)).max() <= TOL
    diff = np.abs(f16(key_step[pos]).astype(np.float64) - f16(want_k[0]))
    assert diff.max() <= max(2e-3, 2e-3 * np.abs(f16(want_k)).max())


def test_decode_step_errors(ctx):
    hq, hkv, d = 4, 2, 128
    cache = ctx.kv_cache(1, hkv, d, 8)
    key, value = cache.layer(0)
    q, k, v = (ctx.tensor(rand(i, (1, h, d))) for i, h in ((1, hq), (2, hkv), (3, hkv)))
    w = ctx.tensor(rand(4, (d,)))
    batch = ctx.begin_batch()
    with pytest.raises(mi_attn.MiError, match="query_offset must be the transform's offset"):
        batch.decode_step_attention(q, k, v, w, w, key, value, mi_attn.QkNormRopeCacheConfig(3, 1e4, 1e-6),
                                    mi_attn.AttentionConfig(hq, hkv, d, True, 2))
    with pytest.raises(mi_attn.MiError, match="cache offset"):
        batch.decode_step_attention(q, k, v, w, w, key, value, mi_attn.QkNormRopeCacheConfig(8, 1e4, 1e-6),
                                    mi_attn.AttentionConfig(hq, hkv, d, True, 8))
    q2 = ctx.tensor(rand(5, (2, hq, d)))
    with pytest.raises(mi_attn.MiError):
        batch.decode_step_attention(q2, k, v, w, w, key, value, mi_attn.QkNormRopeCacheConfig(3, 1e4, 1e-6),
                                    mi_attn.AttentionConfig(hq, hkv, d, True, 3))
    batch.abandon()
    cache.close()
