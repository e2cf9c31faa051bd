"""Benchmark of the MI355X causal GQA attention path (one GPU).

Headline (BASELINE.json metric, decode half): HBM GB/s of the largest
single-GPU decode configuration, configs[3] (c4: 32 sequences, Qwen3-8B
geometry, L ~ U[1024, 8192] seeded, fp16 head-major caches, 627 MB of K/V per
call, larger than the 256 MB MALL). A step is one batched-decode call over
all 32 sequences; exactly --steps calls are timed, replayed from a HIP graph
captured on the library's stream (Python launch cost stays out of the GPU
timeline), bracketed by HIP events on that stream after a synchronize.
`value` is algorithmic bytes x steps / timed seconds.

The prefill half of the metric (TFLOP/s against the fp16 MFMA peak) is
configs[4] (c5) in `prefill`, next to configs[2] (c3); configs[0] (c1) and
configs[1] (c2, 64 rotated caches) are sub-entries. Each entry carries its
roofline; `accuracy` is the max-abs error of the timed call's output against
the CPU oracle, computed in the cpu_baseline leg from the oracle runs it
times (null with --no-cpu).

`compare` holds the reference's attention compare harness
(`metal-infer-bench attention --kind compare`) at its default decode shape and
one prefill shape; `--compare` runs only that harness, at a chosen shape.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
       python bench.py --compare [--tokens 1] [--length 640] [--iterations 50]
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
ROTATE = 64                    # c2: distinct caches per graph (537 MB > MALL)
TOL = 2e-3                     # north_star max-abs bar against the oracle


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
    """Seconds per graph launch: the stream is synchronized, then `reps`
    launches are bracketed by events recorded on the same stream."""
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
    events on the library stream (used under rocprofv3, which does not trace
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


def timed(ctx, hip, enqueue, steps: int, warmup: int, eager: bool) -> float:
    """Seconds per call over exactly `steps` timed calls, after at least
    `warmup` untimed ones. Eager mode runs the warmup as eager calls. Graph
    mode runs two eager calls (they size the batch arena), captures the
    `steps` calls once, replays the graph untimed ceil(warmup / steps) times
    (at least once: the first launch uploads it) and then times one replay.
    Warmup replays keep the GPU busy back to back, so the timed replay runs
    at the clock a sustained load holds (a few eager calls from Python leave
    it idle between calls: c4 measured 107.2 us per call after 5 eager calls
    against 105.9 us after 300, same box)."""
    for i in range(warmup if eager else min(warmup, 2)):
        b = ctx.begin_batch()
        enqueue(b, i)
        b.finish()
    if eager:
        return time_eager(ctx, hip, enqueue, steps)
    exe, graph, stream, keep = capture(hip, ctx, enqueue, steps)
    for _ in range(max(1, -(-warmup // steps))):
        time_graph(hip, exe, stream, 1)
    seconds = time_graph(hip, exe, stream, 1) / steps
    hip.lib.hipGraphExecDestroy(exe)
    hip.lib.hipGraphDestroy(graph)
    del keep
    return seconds


# Launch record of each workload's dominant kernel (used when the eager
# per-dispatch pass is skipped).
DOMINANT = {"c1": "attn_prefill", "c2": "attn_rows", "c3": "attn_prefill",
            "c4": "attn_decode_stream", "c5": "attn_prefill"}
DISPATCH_EVENTS = True  # --no-dispatch-events clears it


def kernel_profile(ctx: mi_attn.Context, enqueue, count: int,
                   workload: str = "", warm: int = 0) -> tuple[str, float, dict]:
    """The dominant kernel (largest total time) of `count` eager calls, its
    median duration per launch (s), and every kernel's median, from the
    start / stop events the library binds to each dispatch on the batch's
    stream (hipExtLaunchKernelGGL). `warm` unprofiled calls run first: the
    first dispatches of a power-capped kernel after the GPU idled (c5 after
    its output's download) run up to ~10% slower than the steady state the
    timed replay sees. A diagnostic beside the timed region; skipped with
    --no-dispatch-events (so that a profiler's trace of the run holds only
    the timed calls)."""
    if not DISPATCH_EVENTS and workload in DOMINANT:
        return DOMINANT[workload], float("nan"), {}
    if warm:
        batch = ctx.begin_batch()
        keep = [enqueue(batch, i) for i in range(warm)]
        batch.finish()
        del keep
    ctx.take_kernel_profiles()
    ctx.set_kernel_profiling(True)
    try:
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


def roofline(run: dict, workload: str) -> dict:
    """Roofline of the step's kernels: one launch per attention call (split
    merges inside it), or for the batched decode the stream kernel and its
    merge launch, whose summed time is the call's kernel time (BASELINE's
    definition). The kernels' average time per call over the timed region
    is the timed seconds per step (HIP events on the launch stream); the
    per-dispatch event medians of a separate eager pass are kept as
    `dispatch_event_us`."""
    secs = run["seconds"]
    if "bytes" in run:
        achieved, peak, unit, work = run["bytes"] / secs / 1e9, HBM_PEAK_GBS, "GB/s", "bytes"
    else:
        achieved, peak, unit, work = run["flops"] / secs / 1e12, MFMA_F16_PEAK_TFLOPS, "TFLOP/s", "flops"
    return {"bound": "hbm" if unit == "GB/s" else "mfma", "achieved": round(achieved, 2),
            "peak": peak, "unit": unit, "frac": round(achieved / peak, 4),
            "traffic": measured_traffic(workload, run["kernel"]), "kernel": run["kernel"],
            "kernel_us": round(secs * 1e6, 3), f"algorithmic_{work}": run[work],
            "launches_per_step": run["launches"],
            "dispatch_event_us": {n: round(t * 1e6, 3) for n, t in run["kernels"].items()}}


# ---------------------------------------------------------------- decode --

def bench_batched_decode(ctx, hip, steps, warmup, eager):
    """c4 (the headline): one call decodes all 32 sequences."""
    c = workloads.case(4)
    B, hq, hkv, d, cap = c.batch, c.q_heads, c.kv_heads, c.head_dim, c.kv_length
    log(f"c4 batched decode: B={B}, sum L={int(c.lengths.sum())}")
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

    seconds = timed(ctx, hip, enqueue, steps, warmup, eager)
    got = ctx.download(out)
    name, _, kernels = kernel_profile(ctx, enqueue, 10, "c4")
    for t in (kt, vt, q, lengths, out):
        t.free()
    return c, dict(steps=steps, seconds=seconds, kernel=name, kernels=kernels,
                   launches=len(kernels) or None, bytes=c.algorithmic_bytes(), out=got)


def bench_decode(ctx, hip, steps, warmup, eager):
    """c2: single-sequence FlashDecode, rotating 64 caches per graph."""
    c = workloads.case(2)
    hq, hkv, d, L = c.q_heads, c.kv_heads, c.head_dim, c.kv_length
    log(f"c2 decode: {ROTATE} head-major caches of {L} positions")
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

    calls = max(ROTATE, (steps + ROTATE - 1) // ROTATE * ROTATE)
    seconds = timed(ctx, hip, enqueue, calls, warmup, eager)
    got = ctx.download(out)
    name, _, kernels = kernel_profile(ctx, enqueue, 4 * ROTATE, "c2")
    q.free()
    out.free()
    cache.close()
    return c, dict(steps=calls, seconds=seconds, kernel=name, kernels=kernels, launches=1,
                   bytes=c.algorithmic_bytes(), out=got)


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
    start, end = hip.event(), hip.event()
    reps = max(1, steps // PER_GRAPH)

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

    def enqueue(batch, i):
        q_rot = batch.qk_norm_rope_cache(q_in, k_in, weights, weights, key, rope)
        batch.copy_into_cache(v_in, value, pos)
        return batch.attention(q_rot, key.prefix(L), value.prefix(L), cfg, mi_attn.FLASH_DECODE,
                               out=out)

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

    eager = time_eager(ctx, hip, enqueue, steps)
    graph_us = graph_us_of(enqueue)
    fused_value_us = graph_us_of(enqueue_fused)
    one_launch_us = graph_us_of(enqueue_step)
    cache.close()
    return {"workload": "c2 decode step: qk_norm_rope_cache + copy_into_cache + FlashDecode "
                        f"(3 kernels), same cache slot every step; {PER_GRAPH} steps per "
                        "captured graph",
            "graph_us": round(graph_us, 3), "eager_us": round(eager * 1e6, 3),
            "graph_fused_value_us": round(fused_value_us, 3),
            "graph_one_launch_us": round(one_launch_us, 3)}


# --------------------------------------------------------------- prefill --

def bench_prefill(ctx, hip, config, steps, warmup, eager):
    c = workloads.case(config)
    hq, hkv, d = c.q_heads, c.kv_heads, c.head_dim
    log(f"c{config} prefill: T={c.tokens} L={c.kv_length} Hq={hq} Hkv={hkv}")
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

    plan = ctx.plan(q, key, value, cfg, kind)
    seconds = timed(ctx, hip, enqueue, steps, warmup, eager)
    got = ctx.download(out)
    name, _, kernels = kernel_profile(ctx, enqueue, 10 if config != 5 else 8, f"c{config}",
                                      warm=2)
    q.free()
    out.free()
    cache.close()
    return c, dict(steps=steps, seconds=seconds, kernel=name, kernels=kernels, launches=1,
                   flops=c.flops(), plan=plan, out=got)


def bench_dispatch_modes(ctx, hip, config: int, calls: int) -> dict:
    """One prefill config timed four ways in one process, in this order and
    twice over: a HIP graph replay of `calls` calls (the timed region's
    method), one eager batch of `calls` calls between two stream events,
    the per-dispatch events of an eager batch (every dispatch's duration),
    and `calls` isolated eager calls, each after a device synchronize."""
    c = workloads.case(config)
    cache = ctx.kv_cache(1, c.kv_heads, c.head_dim, c.kv_length)
    key, value = cache.layer(0)
    ctx.upload(key, c.k)
    ctx.upload(value, c.v)
    q = ctx.tensor(c.q)
    out = ctx.empty(c.q.shape)
    cfg = mi_attn.AttentionConfig(c.q_heads, c.kv_heads, c.head_dim, True, c.query_offset)

    def enqueue(batch, i):
        return batch.attention(q, key, value, cfg, mi_attn.FLASH_PREFILL, out=out)

    reps = []
    for _ in range(2):
        graph = timed(ctx, hip, enqueue, calls, 1, False)
        eager = timed(ctx, hip, enqueue, calls, 1, True)
        ctx.take_kernel_profiles()
        ctx.set_kernel_profiling(True)
        try:
            batch = ctx.begin_batch()
            keep = [enqueue(batch, i) for i in range(calls)]
            batch.finish()
            del keep
            each = [ns / 1e3 for _, ns in ctx.take_kernel_profiles()]
        finally:
            ctx.set_kernel_profiling(False)
        isolated = []
        for _ in range(calls):
            hip.check(hip.lib.hipDeviceSynchronize(), "sync")
            isolated.append(time_eager(ctx, hip, enqueue, 1) * 1e6)
        reps.append({"graph_us": round(graph * 1e6, 1), "eager_batch_us": round(eager * 1e6, 1),
                     "dispatch_events_us": [round(x, 1) for x in each],
                     "isolated_us": [round(x, 1) for x in isolated]})
        log(f"dispatch modes c{config}: {reps[-1]}")
    q.free()
    out.free()
    cache.close()
    return {"workload": f"c{config}", "calls": calls, "runs": reps}


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


def _hbm_entry(label, seconds, name, kernel_s, nbytes) -> dict:
    achieved = nbytes / kernel_s / 1e9
    return {"workload": label, "ms_per_step": round(seconds * 1e3, 5), "kernel": name,
            "kernel_us": round(kernel_s * 1e6, 3), "value": round(nbytes / seconds / 1e9, 2),
            "unit": "GB/s",
            "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "traffic": None, "algorithmic_bytes": nbytes}}


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

        seconds = timed(ctx, hip, enqueue, max(rotate, 64), 1, eager)
        name, kernel_s, _ = kernel_profile(ctx, enqueue, max(rotate, 8))
        nbytes = 2 * 2 * int(np.prod(shape)) + (2 * shape[-1] if op == "rms_norm" else 0)
        entry = _hbm_entry(label, seconds, name, kernel_s, nbytes)
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

    seconds = timed(ctx, hip, enqueue, 16, 1, eager)
    name, kernel_s, _ = kernel_profile(ctx, enqueue, 8)
    nbytes = 2 * 2 * T * (hq + hkv) * d + 2 * 2 * d
    entry = _hbm_entry(label, seconds, name, kernel_s, nbytes)
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

        steps = max(rotate, 64 if bound == "hbm" else 8)
        seconds = timed(ctx, hip, enqueue, steps, 1, eager)
        name, kernel_s, kernels = kernel_profile(ctx, enqueue, max(rotate, 8))
        if bound == "hbm":
            entry = _hbm_entry(label, seconds, name, kernel_s, 2 * (n * k + m * k + m * n))
        else:
            flops = 2 * m * n * k
            achieved = flops / kernel_s / 1e12
            entry = {"workload": label, "ms_per_step": round(seconds * 1e3, 5), "kernel": name,
                     "kernel_us": round(kernel_s * 1e6, 3),
                     "value": round(flops / seconds / 1e12, 2), "unit": "TFLOP/s",
                     "roofline": {"bound": "mfma", "achieved": round(achieved, 2),
                                  "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                  "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4),
                                  "traffic": None, "algorithmic_flops": flops}}
        log(f"  {entry['value']} {entry['unit']}, {name} {entry['kernel_us']} us")
        results.append(entry)
        for w in weights:
            w.free()
        x.free()
        out.free()
    return results


# ---------------------------------------------------------------- floors --

def probe_lib() -> ctypes.CDLL:
    """libmi_probe.so (include/mi_probe.h): calibration kernels."""
    lib = ctypes.CDLL(str(ROOT / "metal-infer-rs_amd" / "libmi_probe.so"))
    vp, u32, u64, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32
    lib.mi_probe_empty.argtypes = [vp, u32, u32, u32]
    lib.mi_probe_read.argtypes = [vp, vp, u64, u32, vp]
    lib.mi_probe_split_decode.argtypes = [vp, vp, vp, u64, u32, u32, u32, u32, i32, vp, vp, vp,
                                          vp]
    for fn in (lib.mi_probe_empty, lib.mi_probe_read, lib.mi_probe_split_decode):
        fn.restype = i32
    return lib


def bench_floors(ctx, hip, steps) -> dict:
    """What the decode kernels' time is made of, measured beside them in the
    same process with the same timing (HIP graph replays on the library's
    stream):
     - c2 (single-sequence FlashDecode, 64 rotated caches): an empty kernel
       on the attention kernel's grid (16 splits x 8 KV heads, 512 threads);
       the same grid loading exactly the attention kernel's K/V rows (the
       data phase); the data phase plus the split exchange (partials with
       device-scope stores, the arrival, the last arriver's acquire and merge,
       f16 output); and the attention call itself;
     - c4: a streaming read of c4's algorithmic bytes by 512 to 2048
       workgroups (the achievable HBM read rate at that size), beside the
       batched-decode call."""
    probe = probe_lib()
    out = {}
    c = workloads.case(2)
    hq, hkv, d, L = c.q_heads, c.kv_heads, c.head_dim, c.kv_length
    group, block = hq // hkv, 128
    splits = (L + block - 1) // block
    log(f"floors: c2 grid {splits} x {hkv}, {ROTATE} rotated caches")
    cache = ctx.kv_cache(ROTATE, hkv, d, L)
    layers = [cache.layer(i) for i in range(ROTATE)]
    for key, value in layers:
        ctx.upload(key, c.k)
        ctx.upload(value, c.v)
    head_stride = layers[0][0].strides[1]
    partial = ctx.empty((hkv * splits * group * (d + 2),), mi_attn.F32)
    counters = ctx.tensor(np.zeros(32 * hkv, np.uint32), mi_attn.U32)  # one line per head
    words = ctx.empty((hkv * splits,), mi_attn.U32)
    out16 = ctx.empty((hkv * group * d,))
    q = ctx.tensor(c.q)
    attn_out = ctx.empty(c.q.shape)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, c.query_offset)

    def split_probe(publish):
        def enqueue(batch, i):
            key, value = layers[i % ROTATE]
            rc = probe.mi_probe_split_decode(batch.stream, key.data_ptr, value.data_ptr,
                                             head_stride, hkv, group, L, block, publish,
                                             partial.data_ptr, counters.data_ptr,
                                             words.data_ptr, out16.data_ptr)
            hip.check(rc, "mi_probe_split_decode")
        return enqueue

    def empty(batch, i):
        hip.check(probe.mi_probe_empty(batch.stream, splits, hkv, 512), "mi_probe_empty")

    def attention(batch, i):
        key, value = layers[i % ROTATE]
        return batch.attention(q, key, value, cfg, mi_attn.FLASH_DECODE, out=attn_out)

    calls = max(ROTATE, (steps + ROTATE - 1) // ROTATE * ROTATE)
    c2 = {"grid": [splits, hkv], "threads": 512, "calls": calls}
    for label, enqueue in (("empty_kernel", empty), ("data_phase", split_probe(0)),
                           ("data_publish_merge", split_probe(1)), ("attention", attention)):
        reps = [timed(ctx, hip, enqueue, calls, 2, False) for _ in range(3)]
        c2[label + "_us"] = round(float(np.median(reps)) * 1e6, 3)
    assert (ctx.download(counters) == 0).all(), "the probe left a counter set"
    log("floors c2: " + ", ".join(f"{k} {v}" for k, v in c2.items() if k.endswith("_us")))
    out["c2"] = c2
    for t in (partial, counters, words, out16, q, attn_out):
        t.free()
    cache.close()

    c4 = workloads.case(4, generate=False)
    nbytes = c4.algorithmic_bytes()
    # per-workgroup shares are rounded up to 16 bytes: at most 16 B more per workgroup
    src = ctx.empty((nbytes // 2 + 32 * 1024,))
    sink = ctx.empty((2048 * 4,), mi_attn.U32)
    rates = {}
    for wgs in (512, 1024, 2048):
        per = (nbytes + wgs - 1) // wgs
        per = (per + 15) // 16 * 16

        def read(batch, i, per=per, wgs=wgs):
            hip.check(probe.mi_probe_read(batch.stream, src.data_ptr, per, wgs, sink.data_ptr),
                      "mi_probe_read")
        seconds = timed(ctx, hip, read, steps, 2, False)
        rates[str(wgs)] = round(per * wgs / seconds / 1e9, 1)
    out["c4_read"] = {"bytes": nbytes, "gb_per_s_by_workgroups": rates,
                      "best_gb_per_s": max(rates.values())}
    log(f"floors c4 read: {rates} GB/s")
    src.free()
    sink.free()
    return out


# ------------------------------------------------------ compare harness --

def duration_stats(samples_s: list[float]) -> tuple[float, float, float]:
    """(mean, median, p95) in ms, indexed as bench.rs:1995-2008 does
    (median = sorted[n / 2], p95 = sorted[round((n - 1) * 0.95)])."""
    s = sorted(samples_s)
    p95 = s[int(round((len(s) - 1) * 0.95))]
    return (sum(s) / len(s) * 1e3, s[len(s) // 2] * 1e3, p95 * 1e3)


def compare_attention(ctx, tokens=1, length=640, query_heads=16, kv_heads=8, head_dim=128,
                      iterations=50, warmup=10) -> dict:
    """`metal-infer-bench attention --kind compare`
    (crates/metal-infer-cli/src/bin/bench.rs:927-1108): every attention kind
    on the closed-form inputs (bench.rs:973-981), each timed as `iterations`
    one-dispatch batches after `warmup` (begin_batch, attention, finish:
    wall clock around the three calls, GPU time from the batch's events;
    bench.rs:823-836), reported as mean / median / p95 with the max-abs
    error of its output against the Reference kind's (bench.rs:1243-1252).
    FlashDecode appears as the reference's two explicit (64, 256) and
    (64, 128) configurations and as this library's default (what
    `attention(.., FlashDecode)` runs untuned); it is offered for every GQA
    ratio (the reference requires two query heads per KV head)."""
    if not (0 < tokens <= length) or min(query_heads, kv_heads, head_dim) <= 0:
        raise ValueError("attention dimensions must be non-zero and tokens must not exceed length")
    if query_heads % kv_heads:
        raise ValueError("attention query-heads must be divisible by kv-heads")
    qh, kh, vh = workloads.compare_inputs(tokens, length, query_heads, kv_heads, head_dim)
    q, k, v = ctx.tensor(qh), ctx.tensor(kh), ctx.tensor(vh)
    cfg = mi_attn.AttentionConfig(query_heads, kv_heads, head_dim, True, length - tokens)

    def f32(bits):
        return bits.view(np.float16).astype(np.float32)

    def variant(name, dispatch):
        batch = ctx.begin_batch()
        out = dispatch(batch)
        batch.finish()
        got = f32(ctx.download(out))
        del out
        for _ in range(warmup):
            batch = ctx.begin_batch()
            dispatch(batch)
            batch.finish()
        wall, gpu = [], []
        for _ in range(iterations):
            t0 = time.perf_counter()
            batch = ctx.begin_batch()
            dispatch(batch)
            stats = batch.finish()
            wall.append(time.perf_counter() - t0)
            gpu.append(stats.gpu_ns * 1e-9)
        w, g = duration_stats(wall), duration_stats(gpu)
        return got, {"kind": name, "wall_mean_ms": w[0], "wall_median_ms": w[1],
                     "wall_p95_ms": w[2], "gpu_mean_ms": g[0], "gpu_median_ms": g[1],
                     "gpu_p95_ms": g[2]}

    def kind(attention_kind):
        return lambda batch: batch.attention(q, k, v, cfg, attention_kind)

    reference_out, reference = variant("reference", kind(mi_attn.REFERENCE))
    reference["max_abs_error"] = 0.0
    comparison = {"reference": reference}

    def add(key, name, dispatch):
        out, report = variant(name, dispatch)
        report["max_abs_error"] = float(np.abs(out - reference_out).max())
        comparison[key] = report

    add("tiled", "tiled", kind(mi_attn.TILED))
    if tokens > 1:
        add("flash_prefill", "flash-prefill", kind(mi_attn.FLASH_PREFILL))
    else:
        add("decode_split_kv", "decode-split-kv", kind(mi_attn.DECODE_SPLIT_KV))
        add("flash_decode", "flash-decode-256t",
            lambda b: b.attention_flash_decode_with_configuration(q, k, v, cfg, 64, 256))
        add("flash_decode_128", "flash-decode-128t",
            lambda b: b.attention_flash_decode_with_configuration(q, k, v, cfg, 64, 128))
        add("flash_decode_default", "flash-decode", kind(mi_attn.FLASH_DECODE))
    # The variant the model's policy would pick (bench.rs:1050-1063, with this
    # library's default FlashDecode standing for the (64, 256) one).
    if tokens == 1:
        selected = comparison["flash_decode_default" if length >= 256 else "decode_split_kv"]
    else:
        selected = comparison["flash_prefill" if tokens >= 32 else "tiled"]
    for t in (q, k, v):
        t.free()
    return {"benchmark": f"attention_f16[tokens={tokens},length={length}]",
            "device": ctx.device_name, "iterations": iterations, "warmup": warmup,
            "shape": {"query_heads": query_heads, "kv_heads": kv_heads, "head_dim": head_dim,
                      "query_offset": length - tokens},
            "selected": selected["kind"],
            "mean_ms": selected["wall_mean_ms"], "median_ms": selected["wall_median_ms"],
            "p95_ms": selected["wall_p95_ms"], "gpu_mean_ms": selected["gpu_mean_ms"],
            "gpu_median_ms": selected["gpu_median_ms"], "gpu_p95_ms": selected["gpu_p95_ms"],
            "allocated_bytes": ctx.allocated_bytes(), "attention_comparison": comparison}


# The compare block of the default run: the harness's defaults (one decode
# token over 640 keys, Qwen3-0.6B heads) and one prefill shape.
COMPARE_SHAPES = ((1, 640), (640, 640))


# -------------------------------------------------------------- CPU leg ---

def host_cpu() -> dict:
    """The host's CPU model, its logical CPUs, and the threads the oracle
    uses: the CPUs this process may run on, capped by OMP_NUM_THREADS when
    set (the GPU box grants each GPU a 16-thread share and sets it to 16)."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(usable, int(cap)) if cap.isdigit() and int(cap) > 0 else usable
    return {"model": model, "nproc": usable, "threads": threads}


def cpu_baseline(entries: dict) -> dict:
    """The C oracle (attention_reference_f16 restated, oracle/) timed on this
    host's cores for every BASELINE config: one warm-up and the median of 5
    runs for c1-c4, and one run of the full call for c5 (~2.5 TFLOP, several
    seconds). The oracle's outputs from these runs are also the reference for
    each GPU entry's `accuracy` (max-abs of the timed call's output, every
    row)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    host = host_cpu()
    threads = host["threads"]
    configs = {}

    def f16(bits):
        return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)

    def timed_runs(fn, reps):
        fn()
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            result = fn()
            times.append(time.perf_counter() - t0)
        return float(np.median(times)), result

    for name, (c, run, entry) in entries.items():
        args = dict(q_heads=c.q_heads, kv_heads=c.kv_heads, head_dim=c.head_dim, causal=True,
                    want=("f32",), threads=threads)
        rows = None
        if c.kind == "batched_decode":
            def fn():
                return [oracle.attention(c.q[b:b + 1], c.k[b], c.v[b],
                                         query_offset=int(c.lengths[b]) - 1, **args)["f32"]
                        for b in range(c.batch)]
            seconds, ref = timed_runs(fn, 5)
            ref = np.concatenate(ref, axis=0)
            work, unit = c.algorithmic_bytes(), "GB/s"
            sample = f"all {c.batch} sequences, median of 5 runs"
        elif name == "c5":
            t0 = time.perf_counter()
            ref = oracle.attention(c.q, c.k, c.v, query_offset=c.query_offset, **args)["f32"]
            seconds = time.perf_counter() - t0
            work, unit = c.flops(), "GFLOP/s"
            sample = "the full call, one run"
        else:
            def fn():
                return oracle.attention(c.q, c.k, c.v, query_offset=c.query_offset,
                                        **args)["f32"]
            seconds, ref = timed_runs(fn, 5)
            if c.kind == "decode":
                work, unit = c.algorithmic_bytes(), "GB/s"
            else:
                work, unit = c.flops(), "GFLOP/s"
            sample = "the full call, median of 5 runs"
        rate = work / seconds / 1e9
        configs[name] = {"value": round(rate, 3), "unit": unit,
                         "ms_per_call": round(seconds * 1e3, 3), "threads": threads,
                         "sample": sample}
        got = f16(run["out"] if rows is None else run["out"][rows])
        diff = np.abs(got - np.asarray(ref, np.float64))
        err = float(diff.max())
        entry["accuracy"] = {"max_abs": err, "tol": TOL, "ok": bool(err <= TOL),
                             "rows_checked": int(got.shape[0] * got.shape[1]),
                             "against": "oracle f32 (unrounded), same seeded inputs"}
        log(f"cpu {name}: {rate:.3f} {unit} ({seconds * 1e3:.1f} ms per call), "
            f"GPU max-abs {err:.2e}")
    head = configs["c4"] if "c4" in configs else next(iter(configs.values()))
    return {"value": head["value"], "unit": head["unit"], "cores": threads, "kind": "port",
            "cpu_model": host["model"], "nproc": host["nproc"],
            "sample": f"c4: {head['sample']} of the C oracle, {threads} OpenMP threads on "
                      f"{host['model']}; every config in `configs`",
            "configs": configs}


# ------------------------------------------------------------------ main --

def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--workloads", default="c4,c5,c3,c2,c1,step,o_proj,compare",
                    help="comma list of c4 (headline), c5, c3, c2, c1, step (decode step "
                         "graphs), o_proj (with the other neighbours), compare (the "
                         "attention compare harness), floors (calibration kernels beside "
                         "the decodes), dispatch (c5 and c3 as graph replays, eager batches, "
                         "per-dispatch events and isolated calls); profiling runs select "
                         "one at a time")
    ap.add_argument("--eager", action="store_true",
                    help="time eager launches instead of HIP graph replays (for rocprofv3)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 256 MiB KV copy (PMC traffic calibration)")
    ap.add_argument("--compare", action="store_true",
                    help="only the attention compare harness (metal-infer-bench attention "
                         "--kind compare) at --tokens/--length/--query-heads/--kv-heads/"
                         "--head-dim, --iterations/--compare-warmup; prints its report")
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--length", type=int, default=640)
    ap.add_argument("--query-heads", type=int, default=16)
    ap.add_argument("--kv-heads", type=int, default=8)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--iterations", type=int, default=50)
    ap.add_argument("--compare-warmup", type=int, default=10)
    ap.add_argument("--no-dispatch-events", action="store_true",
                    help="skip the eager per-dispatch event pass beside each timed region "
                         "(for a profiler trace of the timed calls only)")
    args = ap.parse_args()
    global DISPATCH_EVENTS
    DISPATCH_EVENTS = not args.no_dispatch_events
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the attention path has no multi-GPU "
              "component in this build; a multi-GPU layout is design-only here", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2
    chosen = [w.strip() for w in args.workloads.split(",") if w.strip()]
    unknown = set(chosen) - {"c1", "c2", "c3", "c4", "c5", "step", "o_proj", "compare", "floors",
                             "dispatch"}
    if unknown:
        print(f"unknown workloads {sorted(unknown)}", file=sys.stderr)
        return 2

    hip = Hip()
    ctx = mi_attn.Context(0)
    log(f"device: {ctx.device_name}, {ctx.compute_units} CUs")
    if args.compare:
        if args.iterations < 1:
            print("--iterations must be >= 1", file=sys.stderr)
            return 2
        print(json.dumps(compare_attention(ctx, args.tokens, args.length, args.query_heads,
                                           args.kv_heads, args.head_dim, args.iterations,
                                           args.compare_warmup)), flush=True)
        ctx.close()
        return 0
    timing = "eager launches" if args.eager else "HIP graph replay"
    K, W = args.steps, args.warmup
    result = {"metric": METRIC, "value": None, "unit": "GB/s", "n_gpus": 1, "steps": K,
              "warmup": W, "ms_per_step": None, "higher_is_better": True,
              "scaling": "weak", "vs_baseline": None, "dtype": "f16",
              "data": "synthetic: seeded XorShift64/Box-Muller N(0,1) f16 (BASELINE configs)"}
    checked = {}  # config -> (case, run, entry) for the CPU leg's accuracy check
    if "c4" in chosen:
        c, run = bench_batched_decode(ctx, hip, K, W, args.eager)
        value = run["bytes"] / run["seconds"] / 1e9
        log(f"c4: {value:.1f} GB/s whole job, {run['seconds'] * 1e6:.2f} us per step")
        result.update({
            "value": round(value, 2), "ms_per_step": round(run["seconds"] * 1e3, 6),
            "config": {"workload": "c4 batched decode (BASELINE configs[3], the largest "
                                   "single-GPU decode config): B=32, L~U[1024,8192] seeded, "
                                   "Hq=32, Hkv=8, D=128, fp16 head-major caches, one "
                                   "call per step (the stream-K kernel and its merge "
                                   f"launch), {timing}; prefill half: c5 in prefill[]",
                       "batch": c.batch, "kv_lengths_sum": int(c.lengths.sum()),
                       "q_heads": c.q_heads, "kv_heads": c.kv_heads, "head_dim": c.head_dim},
            "roofline": roofline(run, "c4")})
        checked["c4"] = (c, run, result)
    else:
        log("c4 not selected: the headline fields stay null (profiling run)")
    prefill = []
    for config in (5, 3):
        if f"c{config}" not in chosen:
            continue
        c, run = bench_prefill(ctx, hip, config, K, W, args.eager)
        tflops = run["flops"] / run["seconds"] / 1e12
        log(f"c{config}: {tflops:.1f} TFLOP/s, {run['seconds'] * 1e3:.4f} ms per step")
        entry = {"workload": c.description, "value": round(tflops, 2), "unit": "TFLOP/s",
                 "steps": K, "ms_per_step": round(run["seconds"] * 1e3, 5),
                 "kernel_family": run["plan"]["kernel"],
                 "plan": {k: run["plan"][k] for k in ("grid", "block_threads", "splits")},
                 "roofline": roofline(run, f"c{config}")}
        prefill.append(entry)
        checked[f"c{config}"] = (c, run, entry)
    if prefill:
        result["prefill"] = prefill
    if "c2" in chosen:
        c, run = bench_decode(ctx, hip, K, W, args.eager)
        value = run["bytes"] / run["seconds"] / 1e9
        log(f"c2: {value:.1f} GB/s, {run['seconds'] * 1e6:.2f} us per step")
        entry = {"workload": f"c2 single-token FlashDecode, L=2048, Hq=16, Hkv=8, D=128, "
                             f"{ROTATE} rotated head-major caches, {timing}",
                 "value": round(value, 2), "unit": "GB/s", "steps": run["steps"],
                 "ms_per_step": round(run["seconds"] * 1e3, 6), "roofline": roofline(run, "c2")}
        result["decode_c2"] = entry
        checked["c2"] = (c, run, entry)
    if "c1" in chosen:
        c, run = bench_prefill(ctx, hip, 1, K, W, args.eager)
        entry = {"workload": c.description + " (parity config; launch-bound)",
                 "value": round(run["flops"] / run["seconds"] / 1e12, 3), "unit": "TFLOP/s",
                 "steps": K, "ms_per_step": round(run["seconds"] * 1e3, 6),
                 "roofline": roofline(run, "c1")}
        result["prefill_c1"] = entry
        checked["c1"] = (c, run, entry)
    if "step" in chosen and not args.eager:
        result["decode_step"] = bench_decode_step(ctx, hip, 256)
        log(f"decode step: graph {result['decode_step']['graph_us']} us "
            f"(fused value append {result['decode_step']['graph_fused_value_us']} us, "
            f"one launch {result['decode_step']['graph_one_launch_us']} us)")
    if "o_proj" in chosen:
        result["o_proj"] = bench_o_proj(ctx, hip, args.eager)
        result["neighbours"] = bench_neighbours(ctx, hip, args.eager)
    if "floors" in chosen and not args.eager:
        result["floors"] = bench_floors(ctx, hip, 64)
    if "dispatch" in chosen and not args.eager:
        result["dispatch_modes"] = [bench_dispatch_modes(ctx, hip, 5, 4),
                                    bench_dispatch_modes(ctx, hip, 3, 20)]
    if "compare" in chosen:
        result["compare"] = []
        for tokens, length in COMPARE_SHAPES:
            report = compare_attention(ctx, tokens, length)
            log(f"compare {report['benchmark']}: " + ", ".join(
                f"{r['kind']} {r['gpu_median_ms'] * 1e3:.1f} us (err {r['max_abs_error']:.1e})"
                for r in report["attention_comparison"].values()))
            result["compare"].append(report)
    if args.copy_calibration:
        result["copy_calibration"] = copy_calibration(ctx, hip)
    if not args.no_cpu and checked:
        log("cpu baseline (oracle) and accuracy ...")
        order = ["c1", "c2", "c3", "c4", "c5"]
        result["cpu_baseline"] = cpu_baseline({k: checked[k] for k in order if k in checked})
    for _, run, _ in checked.values():
        run.pop("out", None)
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
    seconds = timed(ctx, hip, lambda b, i: b.copy_into_cache(source, key, 0), 3, 0, True)
    source.free()
    cache.close()
    log(f"copy calibration: {nbytes} B read + written, {seconds * 1e6:.1f} us per copy")
    return {"kernel": "copy_kv", "bytes_read": nbytes, "bytes_written": nbytes, "calls": 3,
            "us_per_copy": round(seconds * 1e6, 2)}


if __name__ == "__main__":
    sys.exit(main())
