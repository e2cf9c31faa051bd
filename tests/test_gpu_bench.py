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
    counters = ctx.tensor(np.zeros(hkv, np.uint32), mi_attn.U32)
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
