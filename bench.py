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


def kernel_profile(ctx: mi_attn.Context, enqueue, count: int) -> tuple[str, float]:
    """Average duration (s) of the dominant kernel over `count` eager calls,
    from HIP events placed around each launch on the batch's stream."""
    ctx.take_kernel_profiles()
    ctx.set_kernel_profiling(True)
    try:
        for i in range(count):
            batch = ctx.begin_batch()
            enqueue(batch, i)
            batch.finish()
        profiles = ctx.take_kernel_profiles()
    finally:
        ctx.set_kernel_profiling(False)
    by_name: dict[str, list[float]] = {}
    for name, ns in profiles:
        by_name.setdefault(name, []).append(ns)
    name = max(by_name, key=lambda n: sum(by_name[n]))
    per_call = sum(sum(v) for v in by_name.values()) / count
    return name, per_call * 1e-9


# ----------------------------------------------------------------- decode --

def bench_decode(ctx, hip, steps, warmup):
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
    exe, graph, stream, _ = capture(hip, ctx, enqueue, per_graph)
    time_graph(hip, exe, stream, 1)
    reps = max(1, steps // per_graph)
    seconds = time_graph(hip, exe, stream, reps) / per_graph
    hip.lib.hipGraphExecDestroy(exe)
    hip.lib.hipGraphDestroy(graph)
    name, kernel_s = kernel_profile(ctx, enqueue, ROTATE)
    nbytes = c.algorithmic_bytes()
    cache.close()
    return c, dict(steps=per_graph * reps, seconds=seconds, kernel=name, kernel_s=kernel_s,
                   bytes=nbytes)


def bench_batched_decode(ctx, hip, steps):
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
    exe, graph, stream, _ = capture(hip, ctx, enqueue, steps)
    time_graph(hip, exe, stream, 1)
    seconds = time_graph(hip, exe, stream, 3) / steps
    hip.lib.hipGraphExecDestroy(exe)
    hip.lib.hipGraphDestroy(graph)
    name, kernel_s = kernel_profile(ctx, enqueue, 5)
    return c, dict(steps=steps * 3, seconds=seconds, kernel=name, kernel_s=kernel_s,
                   bytes=c.algorithmic_bytes())


def bench_prefill(ctx, hip, config, steps):
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
    exe, graph, stream, _ = capture(hip, ctx, enqueue, steps)
    time_graph(hip, exe, stream, 1)
    seconds = time_graph(hip, exe, stream, 2) / steps
    hip.lib.hipGraphExecDestroy(exe)
    hip.lib.hipGraphDestroy(graph)
    name, kernel_s = kernel_profile(ctx, enqueue, 3)
    cache.close()
    return c, dict(steps=steps * 2, seconds=seconds, kernel=name, kernel_s=kernel_s,
                   flops=c.flops(), plan=ctx.plan(q, key, value, cfg, kind)["kernel"])


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-only", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the attention path has no multi-GPU "
              "component in this build (see DESIGN.md for how it would shard)", file=sys.stderr)
        return 2

    hip = Hip()
    ctx = mi_attn.Context(0)
    log(f"device: {ctx.device_name}, {ctx.compute_units} CUs")
    dc, dec = bench_decode(ctx, hip, args.steps, args.warmup)
    value = dec["bytes"] / dec["seconds"] / 1e9
    achieved = dec["bytes"] / dec["kernel_s"] / 1e9
    log(f"decode: {value:.1f} GB/s whole-job, kernel {dec['kernel']} "
        f"{dec['kernel_s'] * 1e6:.2f} us -> {achieved:.1f} GB/s")
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": dec["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(dec["seconds"] * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: seeded XorShift64/Box-Muller N(0,1) f16 (BASELINE configs)",
        "config": {"workload": "c2 single-token decode, L=2048, Hq=16, Hkv=8, D=128, "
                               f"head-major fp16 cache, {ROTATE} rotated caches, HIP graph",
                   "kv_length": dc.kv_length, "q_heads": dc.q_heads, "kv_heads": dc.kv_heads,
                   "head_dim": dc.head_dim},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None, "kernel": dec["kernel"],
                     "kernel_us": round(dec["kernel_s"] * 1e6, 3),
                     "algorithmic_bytes": dec["bytes"]},
    }
    if not args.decode_only:
        bc, bat = bench_batched_decode(ctx, hip, 20)
        bval = bat["bytes"] / bat["seconds"] / 1e9
        bach = bat["bytes"] / bat["kernel_s"] / 1e9
        log(f"batched decode: {bval:.1f} GB/s, kernel {bat['kernel_s'] * 1e6:.1f} us")
        result["batched_decode"] = {
            "workload": "c4 batched decode B=32, L~U[1024,8192] seeded, Hq=32, Hkv=8, D=128",
            "value": round(bval, 2), "unit": "GB/s", "ms_per_step": round(bat["seconds"] * 1e3, 4),
            "roofline": {"bound": "hbm", "achieved": round(bach, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(bach / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": bat["kernel"], "algorithmic_bytes": bat["bytes"]}}
        prefill = []
        for config, steps in ((3, 10), (5, 2)):
            if config == 5 and not mi_attn_prefill_is_mfma(ctx):
                log("c5 skipped: FlashPrefill is not on the MFMA kernel in this build")
                continue
            pc, pre = bench_prefill(ctx, hip, config, steps)
            tflops = pre["flops"] / pre["seconds"] / 1e12
            kt = pre["flops"] / pre["kernel_s"] / 1e12
            log(f"prefill c{config}: {tflops:.1f} TFLOP/s, kernel {pre['kernel_s'] * 1e3:.3f} ms")
            prefill.append({"workload": pc.description, "value": round(tflops, 2),
                            "unit": "TFLOP/s", "ms_per_step": round(pre["seconds"] * 1e3, 4),
                            "kernel_family": pre["plan"],
                            "roofline": {"bound": "mfma", "achieved": round(kt, 2),
                                         "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                         "frac": round(kt / MFMA_F16_PEAK_TFLOPS, 4),
                                         "traffic": None, "kernel": pre["kernel"],
                                         "algorithmic_flops": pre["flops"]}})
        result["prefill"] = prefill
    if not args.no_cpu:
        log("cpu baseline (oracle) ...")
        result["cpu_baseline"] = cpu_baseline(dc)
    print(json.dumps(result), flush=True)
    ctx.close()
    return 0


def mi_attn_prefill_is_mfma(ctx) -> bool:
    q = mi_attn.Tensor(mi_attn.describe(0x7F0000000000, (4096, 64, 128)))
    k = mi_attn.Tensor(mi_attn.describe(0x7F0000000000, (20480, 8, 128)))
    cfg = mi_attn.AttentionConfig(64, 8, 128, True, 16384)
    return mi_attn.plan(q, k, k, cfg, mi_attn.FLASH_PREFILL)["kernel"] == "attn_prefill"


if __name__ == "__main__":
    sys.exit(main())
