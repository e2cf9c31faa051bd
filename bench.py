"""Benchmark of the MI355X causal GQA attention path (one GPU).

Headline (BASELINE.json metric, configs[1]): decode attention HBM GB/s at
Qwen3-0.6B geometry (16 Q / 8 KV heads, D 128, L 2048, fp16 head-major
cache). A step is one FlashDecode call; the timed steps rotate over 64
distinct caches (537 MB, larger than the 256 MB MALL) so every call reads
HBM, and are replayed from a HIP graph captured on the library's stream so
Python launch cost stays out of the GPU timeline. `value` is whole-job
algorithmic bytes / time over the timed region.

The same line carries the prefill half of the metric (TFLOP/s vs the fp16
MFMA peak, configs[2] and configs[4]) and the batched decode,
each with its own roofline, plus the CPU oracle baseline timed on this host.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "metal-infer-rs_amd"))

import mi_attn  # noqa: E402
import workloads  # noqa: E402

METRIC = "decode attn HBM GB/s (% peak) + prefill attn TFLOP/s (% MFMA peak), fp16"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
ROTATE = 64


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Hip:
    """The few HIP runtime calls bench.py needs (graph capture, events)."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        vp, P = ctypes.c_void_p, ctypes.POINTER
        for name, args in {
            "hipStreamBeginCapture": [vp, ctypes.c_int],
            "hipStreamEndCapture": [vp, P(vp)],
            "hipGraphInstantiate": [P(vp), vp, vp, ctypes.c_char_p, ctypes.c_size_t],
            "hipGraphLaunch": [vp, vp],
            "hipGraphExecDestroy": [vp],
            "hipGraphDestroy": [vp],
            "hipStreamSynchronize": [vp],
            "hipEventCreate": [P(vp)],
            "hipEventRecord": [vp, vp],
            "hipEventSynchronize": [vp],
            "hipEventElapsedTime": [P(ctypes.c_float), vp, vp],
            "hipEventDestroy": [vp],
        }.items():
            fn = getattr(self.lib, name)
            fn.argtypes, fn.restype = args, ctypes.c_int

    def check(self, rc: int, what: str) -> None:
        if rc != 0:
            raise RuntimeError(f"{what} failed with hipError {rc}")

    def event(self):
        ev = ctypes.c_void_p()
        self.check(self.lib.hipEventCreate(ctypes.byref(ev)), "hipEventCreate")
        return ev


def capture(hip: Hip, ctx: mi_attn.Context, enqueue, steps: int):
    """Capture `steps` calls of enqueue(batch, i) into one HIP graph."""
    batch = ctx.begin_batch()
    stream = ctypes.c_void_p(batch.stream)
    hip.check(hip.lib.hipStreamBeginCapture(stream, 2), "hipStreamBeginCapture")
    keep = []
    try:
        for i in range(steps):
            keep.append(enqueue(batch, i))
    finally:
        graph = ctypes.c_void_p()
        hip.check(hip.lib.hipStreamEndCapture(stream, ctypes.byref(graph)), "hipStreamEndCapture")
    exe = ctypes.c_void_p()
    hip.check(hip.lib.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0),
              "hipGraphInstantiate")
    batch.finish()
    return exe, graph, stream, keep


def time_graph(hip: Hip, exe, stream, reps: int) -> float:
    """Seconds per graph launch, bracketed by events on the capture stream."""
    start, end = hip.event(), hip.event()
    hip.check(hip.lib.hipStreamSynchronize(stream), "sync")
    hip.check(hip.lib.hipEventRecord(start, stream), "record")
    for _ in range(reps):
        hip.check(hip.lib.hipGraphLaunch(exe, stream), "hipGraphLaunch")
    hip.check(hip.lib.hipEventRecord(end, stream), "record")
    hip.check(hip.lib.hipEventSynchronize(end), "sync")
    ms = ctypes.c_float()
    hip.check(hip.lib.hipEventElapsedTime(ctypes.byref(ms), start, end), "elapsed")
    hip.lib.hipEventDestroy(start)
    hip.lib.hipEventDestroy(end)
    return ms.value / 1e3 / reps


def time_eager(ctx: mi_attn.Context, hip: Hip, enqueue, steps: int) -> float:
    """Seconds per call of `steps` eager calls in one batch, bracketed by
    events on the library stream (used under rocprofv3, which cannot trace
    graph launches here)."""
    batch = ctx.begin_batch()
    stream = ctypes.c_void_p(batch.stream)
    start, end = hip.event(), hip.event()
    hip.check(hip.lib.hipStreamSynchronize(stream), "sync")
    hip.check(hip.lib.hipEventRecord(start, stream), "record")
    keep = [enqueue(batch, i) for i in range(steps)]
    hip.check(hip.lib.hipEventRecord(end, stream), "record")
    batch.finish()
    hip.check(hip.lib.hipEventSynchronize(end), "sync")
    ms = ctypes.c_float()
    hip.check(hip.lib.hipEventElapsedTime(ctypes.byref(ms), start, end), "elapsed")
    hip.lib.hipEventDestroy(start)
    hip.lib.hipEventDestroy(end)
    del keep
    return ms.value / 1e3 / steps


def timed(ctx, hip, enqueue, steps: int, eager: bool, reps: int) -> tuple[int, float]:
    """(calls timed, seconds per call): a HIP graph of `steps` calls replayed
    `reps` times, or `steps * reps` eager calls."""
    if eager:
        return steps * reps, time_eager(ctx, hip, enqueue, steps * reps)
    exe, graph, stream, _ = capture(hip, ctx, enqueue, steps)
    time_graph(hip, exe, stream, 1)
    seconds = time_graph(hip, exe, stream, reps) / steps
    hip.lib.hipGraphExecDestroy(exe)
    hip.lib.hipGraphDestroy(graph)
    return steps * reps, seconds


def kernel_profile(ctx: mi_attn.Context, enqueue, count: int) -> tuple[str, float, dict]:
    """The dominant kernel (largest total time) of `count` eager calls, its
    median duration per launch (s), and every kernel's median, from the
    start / stop events the library binds to each dispatch on the batch's
    stream (hipExtLaunchKernelGGL)."""
    ctx.take_kernel_profiles()
    ctx.set_kernel_profiling(True)
    try:
        # Back to back in one batch, as in the timed region.
        batch = ctx.begin_batch()
        keep = [enqueue(batch, i) for i in range(count)]
        batch.finish()
        del keep
        profiles = ctx.take_kernel_profiles()
    finally:
        ctx.set_kernel_profiling(False)
    by_name: dict[str, list[float]] = {}
    for name, ns in profiles:
        by_name.setdefault(name, []).append(ns)
    # Median per kernel: a few launches that wait on the host or on a clock
    # change would otherwise skew a µs-scale kernel's mean.
    typical = {n: float(np.median(v)) * 1e-9 for n, v in by_name.items()}
    name = max(by_name, key=lambda n: sum(by_name[n]))
    return name, typical[name], typical


def measured_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` on `workload`, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (scaled by the copy-kernel
    calibration recorded there), or None when not measured."""
    path = ROOT / "profiles" / "pmc_traffic.json"
    if not path.exists():
        return None
    entry = json.loads(path.read_text()).get("workloads", {}).get(workload, {})
    if entry.get("kernel") != kernel:
        return None
    return entry.get("traffic_bytes")


# ----------------------------------------------------------------- decode --

def bench_decode(ctx, hip, steps, warmup, eager):
    c = workloads.case(2)
    hq, hkv, d, L = c.q_heads, c.kv_heads, c.head_dim, c.kv_length
    log(f"decode c2: {ROTATE} head-major caches of {L} positions")
    cache = ctx.kv_cache(ROTATE, hkv, d, L)
    layers = [cache.layer(i) for i in range(ROTATE)]
    for key, value in layers:
        ctx.upload(key, c.k)
        ctx.upload(value, c.v)
    q = ctx.tensor(c.q)
    out = ctx.empty(c.q.shape)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, c.query_offset)

    def enqueue(batch, i):
        key, value = layers[i % ROTATE]
        return batch.attention(q, key, value, cfg, mi_attn.FLASH_DECODE, out=out)

    for i in range(max(warmup, 1)):
        b = ctx.begin_batch()
        enqueue(b, i)
        b.finish()
    per_graph = max(ROTATE, (steps // ROTATE) * ROTATE)
    calls, seconds = timed(ctx, hip, enqueue, per_graph, eager, max(1, steps // per_graph))
    name, kernel_s, kernels = kernel_profile(ctx, enqueue, 4 * ROTATE)
    nbytes = c.algorithmic_bytes()
    cache.close()
    return c, dict(steps=calls, seconds=seconds, kernel=name, kernel_s=kernel_s,
                   kernels=kernels, bytes=nbytes)


def bench_decode_step(ctx, hip, steps):
    """One c2-sized decode step in qwen3.rs:704-750 order (Q/K norm + RoPE with
    K into the cache, V append, FlashDecode over the prefix: three kernels).
    PER_GRAPH consecutive steps are captured into one graph with the
    library's capture API and the graph is replayed, so the figure is the
    GPU's time per step (kernels plus the gaps between graph nodes), not the
    host's launch rate. The same steps enqueued eagerly from Python are
    reported beside it; that figure is bounded by the host's enqueue rate."""
    PER_GRAPH = 32
    c = workloads.case(2)
    hq, hkv, d, L = c.q_heads, c.kv_heads, c.head_dim, c.kv_length
    pos = L - 1
    cache = ctx.kv_cache(1, hkv, d, L)
    key, value = cache.layer(0)
    ctx.upload(key, c.k)
    ctx.upload(value, c.v)
    weights = ctx.tensor(np.full(d, np.float16(1.0).view(np.uint16), dtype=np.uint16))
    q_in = ctx.tensor(c.q)
    k_in = ctx.tensor(c.k[pos:pos + 1].copy())
    v_in = ctx.tensor(c.v[pos:pos + 1].copy())
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, pos)
    rope = mi_attn.QkNormRopeCacheConfig(pos, 1_000_000.0, 1e-6)
    out = ctx.empty(c.q.shape)

    def enqueue(batch, i):
        q_rot = batch.qk_norm_rope_cache(q_in, k_in, weights, weights, key, rope)
        batch.copy_into_cache(v_in, value, pos)
        return batch.attention(q_rot, key.prefix(L), value.prefix(L), cfg, mi_attn.FLASH_DECODE,
                               out=out)

    eager = time_eager(ctx, hip, enqueue, steps)
    capture = ctx.begin_capture()
    keep = [enqueue(capture, i) for i in range(PER_GRAPH)]
    graph = capture.end_capture()
    graph.launch()
    ctx.synchronize()
    reps = max(1, steps // PER_GRAPH)
    start, end = hip.event(), hip.event()
    batch = ctx.begin_batch()  # only for the stream handle; the replays run on it
    stream = ctypes.c_void_p(batch.stream)
    hip.check(hip.lib.hipEventRecord(start, stream), "record")
    for _ in range(reps):
        graph.launch()
    hip.check(hip.lib.hipEventRecord(end, stream), "record")
    hip.check(hip.lib.hipEventSynchronize(end), "sync")
    batch.finish()
    ms = ctypes.c_float()
    hip.check(hip.lib.hipEventElapsedTime(ctypes.byref(ms), start, end), "elapsed")
    graph.destroy()
    del keep
    graph_us = ms.value * 1e3 / (reps * PER_GRAPH)

    def graph_us_of(step):
        """GPU time per step of PER_GRAPH captured steps, replayed."""
        capture = ctx.begin_capture()
        kept = [step(capture, i) for i in range(PER_GRAPH)]
        g = capture.end_capture()
        g.launch()
        ctx.synchronize()
        b = ctx.begin_batch()
        s = ctypes.c_void_p(b.stream)
        hip.check(hip.lib.hipEventRecord(start, s), "record")
        for _ in range(reps):
            g.launch()
        hip.check(hip.lib.hipEventRecord(end, s), "record")
        hip.check(hip.lib.hipEventSynchronize(end), "sync")
        b.finish()
        elapsed = ctypes.c_float()
        hip.check(hip.lib.hipEventElapsedTime(ctypes.byref(elapsed), start, end), "elapsed")
        g.destroy()
        del kept
        return elapsed.value * 1e3 / (reps * PER_GRAPH)

    # The same step with the V append folded into the Q/K kernel
    # (mi_qk_norm_rope_cache_value): two kernels.
    def enqueue_fused(batch, i):
        q_rot = batch.qk_norm_rope_cache_value(q_in, k_in, v_in, weights, weights, key, value,
                                               rope)
        return batch.attention(q_rot, key.prefix(L), value.prefix(L), cfg, mi_attn.FLASH_DECODE,
                               out=out)

    # The whole step in one launch (mi_decode_step_attention): the Q/K
    # transforms run inside the attention kernel.
    def enqueue_step(batch, i):
        return batch.decode_step_attention(q_in, k_in, v_in, weights, weights, key, value, rope,
                                           cfg, out=out)

    fused_value_us = graph_us_of(enqueue_fused)
    one_launch_us = graph_us_of(enqueue_step)
    cache.close()
    return {"workload": "c2 decode step: qk_norm_rope_cache + copy_into_cache + FlashDecode "
                        f"(3 kernels), same cache slot every step; {PER_GRAPH} steps per "
                        "captured graph",
            "graph_us": round(graph_us, 3), "eager_us": round(eager * 1e6, 3),
            "graph_fused_value_us": round(fused_value_us, 3),
            "graph_one_launch_us": round(one_launch_us, 3)}


def bench_batched_decode(ctx, hip, steps, eager):
    c = workloads.case(4)
    B, hq, hkv, d, cap = c.batch, c.q_heads, c.kv_heads, c.head_dim, c.kv_length
    log(f"batched decode c4: B={B}, sum L={int(c.lengths.sum())}")
    kstore = np.zeros((B, hkv, cap, d), dtype=np.uint16)
    vstore = np.zeros((B, hkv, cap, d), dtype=np.uint16)
    for b in range(B):
        kstore[b, :, : c.lengths[b]] = c.k[b].transpose(1, 0, 2)
        vstore[b, :, : c.lengths[b]] = c.v[b].transpose(1, 0, 2)
    kt, vt = ctx.tensor(kstore), ctx.tensor(vstore)
    del kstore, vstore
    view = ((B, cap, hkv, d), (hkv * cap * d, d, cap * d, 1))
    kview, vview = kt.view(*view), vt.view(*view)
    q, lengths = ctx.tensor(c.q), ctx.tensor(c.lengths, mi_attn.U32)
    out = ctx.empty(c.q.shape)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)

    def enqueue(batch, i):
        return batch.attention_decode_batched(q, kview, vview, lengths, cfg, 0, out=out)

    for i in range(2):
        b = ctx.begin_batch()
        enqueue(b, i)
        b.finish()
    calls, seconds = timed(ctx, hip, enqueue, steps, eager, 3)
    name, kernel_s, kernels = kernel_profile(ctx, enqueue, 10)
    return c, dict(steps=calls, seconds=seconds, kernel=name, kernel_s=kernel_s,
                   kernels=kernels, bytes=c.algorithmic_bytes())


def bench_prefill(ctx, hip, config, steps, eager):
    c = workloads.case(config)
    hq, hkv, d = c.q_heads, c.kv_heads, c.head_dim
    log(f"prefill c{config}: T={c.tokens} L={c.kv_length} Hq={hq} Hkv={hkv}")
    cache = ctx.kv_cache(1, hkv, d, c.kv_length)
    key, value = cache.layer(0)
    ctx.upload(key, c.k)
    ctx.upload(value, c.v)
    q = ctx.tensor(c.q)
    out = ctx.empty(c.q.shape)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, c.query_offset)
    kind = mi_attn.FLASH_PREFILL

    def enqueue(batch, i):
        return batch.attention(q, key, value, cfg, kind, out=out)

    b = ctx.begin_batch()
    enqueue(b, 0)
    b.finish()
    calls, seconds = timed(ctx, hip, enqueue, steps, eager, 2)
    name, kernel_s, kernels = kernel_profile(ctx, enqueue, 10 if config == 3 else 3)
    cache.close()
    return c, dict(steps=calls, seconds=seconds, kernel=name, kernel_s=kernel_s,
                   kernels=kernels, flops=c.flops(),
                   plan=ctx.plan(q, key, value, cfg, kind)["kernel"])


# ---------------------------------------------------------------- o_proj --

# The matmul after attention (qwen3.rs:751-752): (label, m, n, k, distinct
# weights rotated so that the HBM-bound shapes read from HBM rather than the
# 256 MB MALL, roofline bound).
O_PROJ = (
    ("decode o_proj, Qwen3-0.6B: [1, 2048] x [1024, 2048]^T", 1, 1024, 2048, 128, "hbm"),
    ("batched decode o_proj, Qwen3-8B (c4): [32, 4096] x [4096, 4096]^T", 32, 4096, 4096, 16,
     "hbm"),
    ("prefill o_proj, c3 (Qwen3-0.6B): [2048, 2048] x [1024, 2048]^T", 2048, 1024, 2048, 1,
     "mfma"),
    ("prefill o_proj, c5 (Qwen3-32B): [4096, 8192] x [5120, 8192]^T", 4096, 5120, 8192, 1,
     "mfma"),
)


# The other neighbours of the attention (qwen3.rs:704-728 / 751-752): the
# standalone RMSNorm over the hidden size and the unfused RoPE over
# [tokens, heads, head_dim], at one decode token and at c5's prefill chunk.
# (label, op, shape, rotate); each is HBM-bound: read + write of the tensor
# (+ the norm weight).
NEIGHBOURS = (
    ("decode rms_norm, Qwen3-32B hidden: [1, 5120]", "rms_norm", (1, 5120), 64),
    ("prefill rms_norm, c5 (Qwen3-32B): [4096, 5120]", "rms_norm", (4096, 5120), 8),
    ("decode rope, Qwen3-32B q: [1, 64, 128]", "rope", (1, 64, 128), 64),
    ("prefill rope, c5 q (Qwen3-32B): [4096, 64, 128]", "rope", (4096, 64, 128), 8),
)


def bench_neighbours(ctx, hip, eager) -> list[dict]:
    rng = np.random.default_rng(1)
    results = []
    for label, op, shape, rotate in NEIGHBOURS:
        log(f"neighbour: {label}")
        host = rng.standard_normal(shape).astype(np.float16).view(np.uint16)
        xs = [ctx.tensor(host) for _ in range(rotate)]
        out = ctx.empty(shape)
        weight = ctx.tensor((1 + 0.1 * rng.standard_normal(shape[-1])).astype(np.float16)
                            .view(np.uint16))

        def enqueue(batch, i):
            x = xs[i % rotate]
            if op == "rms_norm":
                return batch.rms_norm(x, weight, 1e-6, out=out)
            return batch.rope(x, 3, 1_000_000.0, out=out)

        b = ctx.begin_batch()
        enqueue(b, 0)
        b.finish()
        calls, seconds = timed(ctx, hip, enqueue, max(rotate, 64), eager, 2)
        name, kernel_s, _ = kernel_profile(ctx, enqueue, max(rotate, 8))
        nbytes = 2 * 2 * int(np.prod(shape)) + (2 * shape[-1] if op == "rms_norm" else 0)
        achieved = nbytes / kernel_s / 1e9
        entry = {"workload": label, "ms_per_step": round(seconds * 1e3, 5), "kernel": name,
                 "kernel_us": round(kernel_s * 1e6, 3),
                 "value": round(nbytes / seconds / 1e9, 2), "unit": "GB/s",
                 "roofline": {"bound": "hbm", "achieved": round(achieved, 2),
                              "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                              "algorithmic_bytes": nbytes}}
        log(f"  {entry['value']} GB/s, {name} {entry['kernel_us']} us")
        results.append(entry)
        for x in xs:
            x.free()
        out.free()
        weight.free()
    results.append(bench_qk_norm_rope_prefill(ctx, hip, eager, rng))
    return results


def bench_qk_norm_rope_prefill(ctx, hip, eager, rng) -> dict:
    """The fused per-head Q/K RMSNorm + RoPE with K written into the cache
    (qk_norm_rope_cache, qwen3.rs:704-715) over c5's 4096-token chunk."""
    T, hq, hkv, d = 4096, 64, 8, 128
    label = f"prefill qk_norm_rope_cache, c5 (Qwen3-32B): Q [{T}, {hq}, {d}], K [{T}, {hkv}, {d}]"
    log(f"neighbour: {label}")
    rotate = 4
    qs = [ctx.tensor(rng.standard_normal((T, hq, d)).astype(np.float16).view(np.uint16))
          for _ in range(rotate)]
    ks = [ctx.tensor(rng.standard_normal((T, hkv, d)).astype(np.float16).view(np.uint16))
          for _ in range(rotate)]
    w = ctx.tensor((1 + 0.1 * rng.standard_normal(d)).astype(np.float16).view(np.uint16))
    cache = ctx.kv_cache(1, hkv, d, T)
    key, _ = cache.layer(0)
    q_out = ctx.empty((T, hq, d))
    cfg = mi_attn.QkNormRopeCacheConfig(0, 1_000_000.0, 1e-6)

    def enqueue(batch, i):
        return batch.qk_norm_rope_cache(qs[i % rotate], ks[i % rotate], w, w, key, cfg,
                                        out=q_out)

    b = ctx.begin_batch()
    enqueue(b, 0)
    b.finish()
    calls, seconds = timed(ctx, hip, enqueue, 16, eager, 2)
    name, kernel_s, _ = kernel_profile(ctx, enqueue, 8)
    nbytes = 2 * 2 * T * (hq + hkv) * d + 2 * 2 * d
    achieved = nbytes / kernel_s / 1e9
    entry = {"workload": label, "ms_per_step": round(seconds * 1e3, 5), "kernel": name,
             "kernel_us": round(kernel_s * 1e6, 3), "value": round(nbytes / seconds / 1e9, 2),
             "unit": "GB/s",
             "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                          "traffic": None, "algorithmic_bytes": nbytes}}
    log(f"  {entry['value']} GB/s, {name} {entry['kernel_us']} us")
    for t in qs + ks:
        t.free()
    w.free()
    q_out.free()
    cache.close()
    return entry


def bench_o_proj(ctx, hip, eager) -> list[dict]:
    rng = np.random.default_rng(0)
    results = []
    for label, m, n, k, rotate, bound in O_PROJ:
        log(f"o_proj: {label}")
        x = ctx.tensor((rng.standard_normal((m, k))).astype(np.float16).view(np.uint16))
        host_w = (rng.standard_normal((n, k)) * k ** -0.5).astype(np.float16).view(np.uint16)
        weights = [ctx.tensor(host_w) for _ in range(rotate)]
        out = ctx.empty((m, n))

        def enqueue(batch, i):
            return batch.matmul(x, weights[i % rotate], out=out)

        b = ctx.begin_batch()
        enqueue(b, 0)
        b.finish()
        steps = max(rotate, 64 if bound == "hbm" else 8)
        calls, seconds = timed(ctx, hip, enqueue, steps, eager, 2)
        name, kernel_s, kernels = kernel_profile(ctx, enqueue, max(rotate, 8))
        entry = {"workload": label, "ms_per_step": round(seconds * 1e3, 5), "kernel": name,
                 "kernel_us": round(kernel_s * 1e6, 3)}
        if bound == "hbm":
            nbytes = 2 * (n * k + m * k + m * n)
            value = nbytes / seconds / 1e9
            achieved = nbytes / kernel_s / 1e9
            entry.update({"value": round(value, 2), "unit": "GB/s", "roofline": {
                "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "algorithmic_bytes": nbytes}})
        else:
            flops = 2 * m * n * k
            value = flops / seconds / 1e12
            achieved = flops / kernel_s / 1e12
            entry.update({"value": round(value, 2), "unit": "TFLOP/s", "roofline": {
                "bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_F16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4),
                "traffic": None, "algorithmic_flops": flops}})
        log(f"  {entry['value']} {entry['unit']}, {name} {entry['kernel_us']} us")
        results.append(entry)
        for w in weights:
            w.free()
        x.free()
        out.free()
    return results


# -------------------------------------------------------------- CPU leg ---

def cpu_baseline(decode_case) -> dict:
    """The C oracle (attention_reference_f16 restated) on this host's cores,
    on a bounded sample: repeated c2 decodes for about 10 s."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    threads = oracle.default_threads()
    c = decode_case
    args = dict(q_heads=c.q_heads, kv_heads=c.kv_heads, head_dim=c.head_dim, causal=True,
                query_offset=c.query_offset, want=("f32",), threads=threads)
    oracle.attention(c.q, c.k, c.v, **args)
    calls, start = 0, time.perf_counter()
    while time.perf_counter() - start < 10.0:
        oracle.attention(c.q, c.k, c.v, **args)
        calls += 1
    seconds = (time.perf_counter() - start) / calls
    return {"value": round(c.algorithmic_bytes() / seconds / 1e9, 3), "unit": "GB/s",
            "cores": threads, "kind": "port",
            "sample": f"{calls} full c2 decode calls (L=2048, 16/8 heads) of the C oracle, "
                      f"{seconds * 1e3:.2f} ms each, {threads} OpenMP threads"}


def hbm_roofline(nbytes: int, run: dict, workload: str) -> dict:
    achieved = nbytes / run["kernel_s"] / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(workload, run["kernel"]), "kernel": run["kernel"],
            "kernel_us": round(run["kernel_s"] * 1e6, 3), "algorithmic_bytes": nbytes,
            "kernels_us": {n: round(t * 1e6, 3) for n, t in run["kernels"].items()}}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--workloads", default="c2,c4,c3,c5,o_proj",
                    help="comma list of c2 (headline decode), c4, c3, c5, o_proj; profiling "
                         "runs select one at a time")
    ap.add_argument("--eager", action="store_true",
                    help="time eager launches instead of HIP graph replays (for rocprofv3)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 256 MiB KV copy (PMC traffic calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the attention path has no multi-GPU "
              "component in this build; a multi-GPU layout is design-only here", file=sys.stderr)
        return 2
    chosen = [w.strip() for w in args.workloads.split(",") if w.strip()]
    unknown = set(chosen) - {"c2", "c3", "c4", "c5", "o_proj"}
    if unknown:
        print(f"unknown workloads {sorted(unknown)}", file=sys.stderr)
        return 2

    hip = Hip()
    ctx = mi_attn.Context(0)
    log(f"device: {ctx.device_name}, {ctx.compute_units} CUs")
    timing = "eager launches" if args.eager else "HIP graph replay"
    result = {"metric": METRIC, "value": None, "unit": "GB/s", "n_gpus": 1, "steps": 0,
              "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True,
              "scaling": "weak", "vs_baseline": None, "dtype": "f16",
              "data": "synthetic: seeded XorShift64/Box-Muller N(0,1) f16 (BASELINE configs)"}
    dc = None
    if "c2" in chosen:
        dc, dec = bench_decode(ctx, hip, args.steps, args.warmup, args.eager)
        value = dec["bytes"] / dec["seconds"] / 1e9
        roof = hbm_roofline(dec["bytes"], dec, "c2")
        log(f"decode: {value:.1f} GB/s whole-job, kernel {dec['kernel']} "
            f"{dec['kernel_s'] * 1e6:.2f} us -> {roof['achieved']:.1f} GB/s")
        result.update({
            "value": round(value, 2), "steps": dec["steps"],
            "ms_per_step": round(dec["seconds"] * 1e3, 6),
            "config": {"workload": "c2 single-token decode, L=2048, Hq=16, Hkv=8, D=128, "
                                   f"head-major fp16 cache, {ROTATE} rotated caches, {timing}",
                       "kv_length": dc.kv_length, "q_heads": dc.q_heads,
                       "kv_heads": dc.kv_heads, "head_dim": dc.head_dim},
            "roofline": roof})
    else:
        log("c2 not selected: the headline fields stay null (profiling run)")
    if "c2" in chosen and not args.eager:
        result["decode_step"] = bench_decode_step(ctx, hip, 256)
        log(f"decode step: graph {result['decode_step']['graph_us']} us "
            f"(fused value append {result['decode_step']['graph_fused_value_us']} us, "
            f"one launch {result['decode_step']['graph_one_launch_us']} us), "
            f"eager {result['decode_step']['eager_us']} us")
    if "c4" in chosen:
        bc, bat = bench_batched_decode(ctx, hip, 20, args.eager)
        bval = bat["bytes"] / bat["seconds"] / 1e9
        log(f"batched decode: {bval:.1f} GB/s, kernel {bat['kernel_s'] * 1e6:.1f} us")
        result["batched_decode"] = {
            "workload": "c4 batched decode B=32, L~U[1024,8192] seeded, Hq=32, Hkv=8, D=128",
            "value": round(bval, 2), "unit": "GB/s", "ms_per_step": round(bat["seconds"] * 1e3, 4),
            "roofline": hbm_roofline(bat["bytes"], bat, "c4")}
    prefill = []
    for config, steps in ((3, 10), (5, 2)):
        if f"c{config}" not in chosen:
            continue
        if config == 5 and not mi_attn_prefill_is_mfma(ctx):
            log("c5 skipped: FlashPrefill is not on the MFMA kernel in this build")
            continue
        pc, pre = bench_prefill(ctx, hip, config, steps, args.eager)
        tflops = pre["flops"] / pre["seconds"] / 1e12
        kt = pre["flops"] / pre["kernel_s"] / 1e12
        log(f"prefill c{config}: {tflops:.1f} TFLOP/s, kernel {pre['kernel_s'] * 1e3:.3f} ms")
        prefill.append({"workload": pc.description, "value": round(tflops, 2),
                        "unit": "TFLOP/s", "ms_per_step": round(pre["seconds"] * 1e3, 4),
                        "kernel_family": pre["plan"],
                        "roofline": {"bound": "mfma", "achieved": round(kt, 2),
                                     "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                     "frac": round(kt / MFMA_F16_PEAK_TFLOPS, 4),
                                     "traffic": measured_traffic(f"c{config}", pre["kernel"]),
                                     "kernel": pre["kernel"],
                                     "kernel_ms": round(pre["kernel_s"] * 1e3, 4),
                                     "algorithmic_flops": pre["flops"]}})
    if prefill:
        result["prefill"] = prefill
    if "o_proj" in chosen:
        result["o_proj"] = bench_o_proj(ctx, hip, args.eager)
        result["neighbours"] = bench_neighbours(ctx, hip, args.eager)
    if args.copy_calibration:
        result["copy_calibration"] = copy_calibration(ctx, hip)
    if not args.no_cpu and dc is not None:
        log("cpu baseline (oracle) ...")
        result["cpu_baseline"] = cpu_baseline(dc)
    print(json.dumps(result), flush=True)
    ctx.close()
    return 0


def copy_calibration(ctx, hip) -> dict:
    """A plain copy of known size (copy_kv_kernel: 256 MiB read, 256 MiB
    written), run three times; its FETCH_SIZE / WRITE_SIZE readings scale the
    counters of the attention kernels to bytes."""
    hkv, d, positions = 8, 128, 131072
    nbytes = positions * hkv * d * 2
    cache = ctx.kv_cache(1, hkv, d, positions)
    key, _ = cache.layer(0)
    source = ctx.empty((positions, hkv, d))
    calls, seconds = timed(ctx, hip, lambda b, i: b.copy_into_cache(source, key, 0), 3, True, 1)
    source.free()
    cache.close()
    log(f"copy calibration: {nbytes} B read + written, {seconds * 1e6:.1f} us per copy")
    return {"kernel": "copy_kv", "bytes_read": nbytes, "bytes_written": nbytes, "calls": calls,
            "us_per_copy": round(seconds * 1e6, 2)}


def mi_attn_prefill_is_mfma(ctx) -> bool:
    q = mi_attn.Tensor(mi_attn.describe(0x7F0000000000, (4096, 64, 128)))
    k = mi_attn.Tensor(mi_attn.describe(0x7F0000000000, (20480, 8, 128)))
    cfg = mi_attn.AttentionConfig(64, 8, 128, True, 16384)
    return mi_attn.plan(q, k, k, cfg, mi_attn.FLASH_PREFILL)["kernel"] == "attn_prefill"


if __name__ == "__main__":
    sys.exit(main())
