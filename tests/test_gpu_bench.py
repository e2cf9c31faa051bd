"""GPU checks of the benchmark's harnesses: the attention compare harness
(metal-infer-bench attention --kind compare, bench.rs:927-1108) and the
calibration kernels of libmi_probe.so that the floors entry times."""
from __future__ import annotations

import numpy as np
import pytest

import bench
import mi_attn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tokens,length", [(1, 640), (64, 640), (1, 100)])
def test_compare_harness_reports_every_kind(ctx, tokens, length):
    """Every kind the reference's harness times, on its closed-form inputs,
    with wall / GPU mean, median and p95 and the max-abs error against the
    Reference kind; every kind agrees with it well inside the reference's
    0.02 test tolerance (gpu.rs:6)."""
    report = bench.compare_attention(ctx, tokens, length, iterations=3, warmup=1)
    kinds = report["attention_comparison"]
    want = {"reference", "tiled"} | ({"flash_prefill"} if tokens > 1 else
                                     {"decode_split_kv", "flash_decode", "flash_decode_128",
                                      "flash_decode_default"})
    assert set(kinds) == want
    for key, entry in kinds.items():
        for field in ("wall_mean_ms", "wall_median_ms", "wall_p95_ms", "gpu_mean_ms",
                      "gpu_median_ms", "gpu_p95_ms"):
            assert entry[field] > 0, (key, field)
        assert entry["gpu_median_ms"] <= entry["gpu_p95_ms"]
        assert entry["max_abs_error"] <= 2e-3, (key, entry["max_abs_error"])
    assert report["benchmark"] == f"attention_f16[tokens={tokens},length={length}]"
    selected = ("flash-decode" if length >= 256 else "decode-split-kv") if tokens == 1 \
        else "flash-prefill"
    assert report["selected"] == selected


def test_probe_split_exchange_leaves_counters_zero(ctx):
    """The split-exchange probe runs the attention kernel's arrival protocol:
    the last split of each KV head resets its counter, so repeated calls
    (and graph replays) start from zero, and every output is finite."""
    probe = bench.probe_lib()
    hkv, group, d, L, block = 4, 2, 128, 1000, 128
    rng = np.random.default_rng(5)
    store = rng.standard_normal((hkv, L, d)).astype(np.float16).view(np.uint16)
    k, v = ctx.tensor(store), ctx.tensor(store[:, ::-1].copy())
    splits = (L + block - 1) // block
    partial = ctx.empty((hkv * splits * group * (d + 2),), mi_attn.F32)
    counters = ctx.tensor(np.zeros(32 * hkv, np.uint32), mi_attn.U32)  # one line per head
    words = ctx.empty((hkv * splits,), mi_attn.U32)
    out16 = ctx.empty((hkv * group * d,))
    for publish in (0, 1, 1):
        batch = ctx.begin_batch()
        rc = probe.mi_probe_split_decode(batch.stream, k.data_ptr, v.data_ptr, L * d, hkv, group,
                                         L, block, publish, partial.data_ptr, counters.data_ptr,
                                         words.data_ptr, out16.data_ptr)
        assert rc == 0
        batch.finish()
        assert (ctx.download(counters) == 0).all()
    assert np.isfinite(ctx.download(out16).view(np.float16)).all()
    # The data phase's word is the XOR of every K and V row it loaded: rows
    # k0 .. k0 + 127 of the split, those past its end clamped to its last
    # row (the attention kernel's load pattern), so a row may count twice.
    got = ctx.download(words).reshape(hkv, splits)
    kwords = store.view(np.uint32).reshape(hkv, L, d // 2)
    vwords = store[:, ::-1].copy().view(np.uint32).reshape(hkv, L, d // 2)
    for h in range(hkv):
        for s in range(splits):
            k0, k1 = s * block, min(L, (s + 1) * block)
            rows = [min(k0 + j, k1 - 1) for j in range(block)]
            want = np.bitwise_xor.reduce(kwords[h, rows].reshape(-1)) ^ \
                np.bitwise_xor.reduce(vwords[h, rows].reshape(-1))
            assert got[h, s] == want, (h, s)
    for t in (k, v, partial, counters, words, out16):
        t.free()


def test_dispatch_modes_report_every_mode(ctx):
    """The dispatch-mode comparison times one prefill config as a graph
    replay, an eager batch, per-dispatch events and isolated eager calls;
    every mode yields one positive duration per call."""
    report = bench.bench_dispatch_modes(ctx, bench.Hip(), 1, 3)
    assert report["workload"] == "c1" and report["calls"] == 3 and len(report["runs"]) == 2
    for run in report["runs"]:
        assert run["graph_us"] > 0 and run["eager_batch_us"] > 0
        assert len(run["dispatch_events_us"]) == 3 and min(run["dispatch_events_us"]) > 0
        assert len(run["isolated_us"]) == 3 and min(run["isolated_us"]) > 0


def test_kernel_profile_warm_calls_are_not_profiled(ctx):
    """kernel_profile's warm-up calls run before profiling starts: only the
    `count` calls' dispatches are reported."""
    c = bench.workloads.case(1)
    cache = ctx.kv_cache(1, c.kv_heads, c.head_dim, c.kv_length)
    key, value = cache.layer(0)
    ctx.upload(key, c.k)
    ctx.upload(value, c.v)
    q, out = ctx.tensor(c.q), ctx.empty(c.q.shape)
    cfg = mi_attn.AttentionConfig(c.q_heads, c.kv_heads, c.head_dim, True, c.query_offset)
    calls = []

    def enqueue(batch, i):
        calls.append(i)
        return batch.attention(q, key, value, cfg, mi_attn.FLASH_PREFILL, out=out)

    saved = bench.DISPATCH_EVENTS
    bench.DISPATCH_EVENTS = True
    try:
        name, median, kernels = bench.kernel_profile(ctx, enqueue, 4, "c1", warm=2)
    finally:
        bench.DISPATCH_EVENTS = saved
    assert len(calls) == 6 and name == "attn_prefill" and median > 0
    assert set(kernels) == {"attn_prefill"}
    q.free()
    out.free()
    cache.close()
