"""Per-workgroup timelines of the c4 batched decode, the c3 prefill and the
c2 single-sequence decode.

    python3 metal-infer-rs_amd/timeline.py [--workloads c4,c3,c2] [--replays 3]
        [--json PATH]

Loads the timeline build of the library (libmi_attn_timeline.so: the same
sources as libmi_attn.so compiled with MI_TIMELINE; include/mi_timeline.h),
replays one call of each workload as a HIP graph, reads the kernels'
per-workgroup stamps (s_memrealtime, 100 MHz) after each replay and prints a
summary per replay:

 - c4 (attn_decode_stream_kernel): the span, the prologue before each
   workgroup's first piece, how the workgroups pair on CUs (w and w + CUs)
   and which of a pair finishes first, the duration of each slot, and the
   number of workgroups still running in 5 us bins;
 - c3 (attn_prefill_kernel): the first K/V tile's arrival, the key loop's
   end, the split epilogue (publish, arrival, the last arriver's merge), the
   per-key-tile time of the CUs' first and second slots, and the span;
 - c2 (attn_rows_kernel, FlashDecode): the spread of the workgroups' starts,
   the first K/V batch's arrival (this build waits for it before the
   arithmetic), the arithmetic, the wave merge with the partial's stores and
   their completion, the arrival, the last arriver's merge, and the span.

A measurement aid, not part of the attention path; nothing else imports it.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import sys
from pathlib import Path

import numpy as np

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(PACKAGE))

import mi_attn  # noqa: E402

mi_attn.LIB_PATH = PACKAGE / "libmi_attn_timeline.so"

import bench  # noqa: E402
import workloads  # noqa: E402

FIELDS = 8   # u64 words per workgroup row (include/mi_timeline.h)
TICK_US = 0.01  # s_memrealtime runs at 100 MHz


def read_rows(reader, count: int) -> np.ndarray:
    buf = np.zeros(count * FIELDS, np.uint64)
    rc = reader(buf.ctypes.data, buf.nbytes)
    if rc != 0:
        raise RuntimeError(f"timeline read failed: hipError_t {rc}")
    return buf.reshape(count, FIELDS)


def place(rows: np.ndarray) -> np.ndarray:
    """A CU's identity from word 1: XCC_ID and HW_ID's SE / SH / CU fields."""
    xcc = rows[:, 1] & 0xFF
    hw = rows[:, 1] >> 8
    cu, sh, se = (hw >> 8) & 0xF, (hw >> 12) & 1, (hw >> 13) & 7
    return (xcc * 1000 + se * 100 + sh * 16 + cu).astype(np.int64)


def running(start: np.ndarray, end: np.ndarray, step: float) -> list[int]:
    edges = np.arange(0.0, float(end.max()) + step, step)
    return [int(((start <= e) & (end > e)).sum()) for e in edges]


def replay(hip, ctx, enqueue, replays: int, read):
    exe, graph, stream, keep = bench.capture(hip, ctx, enqueue, 1)
    bench.time_graph(hip, exe, stream, 1)
    out = []
    for _ in range(replays):
        seconds = bench.time_graph(hip, exe, stream, 1)
        out.append((seconds, read()))
    hip.lib.hipGraphExecDestroy(exe)
    hip.lib.hipGraphDestroy(graph)
    del keep
    return out


def c4_timeline(hip, ctx, lib, replays: int) -> list[dict]:
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
    q, lengths = ctx.tensor(c.q), ctx.tensor(c.lengths, mi_attn.U32)
    out = ctx.empty(c.q.shape)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, 0)
    cus = ctx.compute_units
    wgs = 2 * cus

    def enqueue(batch, i):
        return batch.attention_decode_batched(q, kview, vview, lengths, cfg, 0, out=out)

    reports = []
    for seconds, rows in replay(hip, ctx, enqueue, replays,
                                lambda: read_rows(lib.mi_timeline_read_stream, wgs)):
        rows = rows.astype(np.int64)
        t0 = rows[:, 0].min()
        start = (rows[:, 0] - t0) * TICK_US
        end = (rows[:, 2] - t0) * TICK_US
        first = (rows[:, 3] - t0) * TICK_US
        pieces = rows[:, 4] & 0xFFFF
        epilogue = rows[:, 5] * TICK_US
        key = place(rows)
        slot1, slot2 = np.arange(cus), np.arange(cus, wgs)
        same_cu = float(np.mean(key[slot1] == key[slot2]))
        dur = end - start
        first_done_first = float(np.mean(end[slot1] < end[slot2]))
        reports.append({
            "workload": "c4", "graph_us": round(seconds * 1e6, 2),
            "span_us": round(float(end.max()), 2),
            "prologue_us_median": round(float(np.median(first - start)), 2),
            "pieces_per_workgroup": {int(k): int(v) for k, v in
                                     zip(*np.unique(pieces, return_counts=True))},
            "epilogue_share_of_workgroup_time": round(float(epilogue.sum() / dur.sum()), 4),
            "pairs_w_and_w_plus_cus_share_a_cu": round(same_cu, 4),
            "first_of_pair_finishes_first": round(first_done_first, 4),
            "duration_us_median": {"first_slot": round(float(np.median(dur[slot1])), 2),
                                   "second_slot": round(float(np.median(dur[slot2])), 2)},
            "running_every_5us": running(start, end, 5.0)})
    for t in (kt, vt, q, lengths, out):
        t.free()
    return reports


def c3_timeline(hip, ctx, lib, replays: int) -> list[dict]:
    c = workloads.case(3)
    cache = ctx.kv_cache(1, c.kv_heads, c.head_dim, c.kv_length)
    key, value = cache.layer(0)
    ctx.upload(key, c.k)
    ctx.upload(value, c.v)
    q, out = ctx.tensor(c.q), ctx.empty(c.q.shape)
    cfg = mi_attn.AttentionConfig(c.q_heads, c.kv_heads, c.head_dim, True, c.query_offset)
    plan = ctx.plan(q, key, value, cfg, mi_attn.FLASH_PREFILL)
    wgs = int(np.prod(plan["grid"]))
    cus = ctx.compute_units

    def enqueue(batch, i):
        return batch.attention(q, key, value, cfg, mi_attn.FLASH_PREFILL, out=out)

    reports = []
    for seconds, rows in replay(hip, ctx, enqueue, replays,
                                lambda: read_rows(lib.mi_timeline_read_prefill, wgs)):
        desc = rows[:, 7]
        merged = (desc >> np.uint64(63)) == 1
        begin = ((desc >> np.uint64(20)) & np.uint64(0xFFFFF)).astype(np.int64)
        end_tile = ((desc >> np.uint64(40)) & np.uint64(0xFFFFF)).astype(np.int64)
        rows = rows.astype(np.int64)
        real = rows[:, 3] > 0  # pieces that ran a key loop
        t0 = rows[:, 0].min()
        us = lambda f: (rows[:, f] - t0) * TICK_US  # noqa: E731
        start, end, ready, loop = us(0), us(2), us(3), us(4)
        published = rows[:, 5] > 0
        tiles = np.maximum(end_tile - begin, 1)
        per_tile = (loop - ready) / tiles
        slot1 = real & (np.arange(wgs) < cus)
        slot2 = real & (np.arange(wgs) >= cus)
        pub, arr = us(5), us(6)
        reports.append({
            "workload": "c3", "plan_grid": list(plan["grid"]), "splits": plan["splits"],
            "graph_us": round(seconds * 1e6, 2), "span_us": round(float(end.max()), 2),
            "pieces": int(real.sum()),
            "first_tile_ready_us_median": round(float(np.median((ready - start)[real])), 2),
            "loop_end_us": {"median": round(float(np.median(loop[real])), 2),
                            "max": round(float(loop[real].max()), 2)},
            "us_per_key_tile_median": {
                "first_slot": round(float(np.median(per_tile[slot1])), 2) if slot1.any() else None,
                "second_slot": round(float(np.median(per_tile[slot2])), 2) if slot2.any() else None},
            "publish_us_median": round(float(np.median((pub - loop)[published])), 2)
            if published.any() else None,
            "arrival_us_median": round(float(np.median((arr - pub)[published])), 2)
            if published.any() else None,
            "merge_us_median": round(float(np.median((end - arr)[published & merged])), 2)
            if (published & merged).any() else None,
            "running_every_2us": running(start[real], end[real], 2.0)})
    q.free()
    out.free()
    cache.close()
    return reports


def c2_timeline(hip, ctx, lib, replays: int) -> list[dict]:
    c = workloads.case(2)
    cache = ctx.kv_cache(1, c.kv_heads, c.head_dim, c.kv_length)
    key, value = cache.layer(0)
    ctx.upload(key, c.k)
    ctx.upload(value, c.v)
    q, out = ctx.tensor(c.q), ctx.empty(c.q.shape)
    cfg = mi_attn.AttentionConfig(c.q_heads, c.kv_heads, c.head_dim, True, c.query_offset)
    plan = ctx.plan(q, key, value, cfg, mi_attn.FLASH_DECODE)
    wgs = int(np.prod(plan["grid"]))

    def enqueue(batch, i):
        return batch.attention(q, key, value, cfg, mi_attn.FLASH_DECODE, out=out)

    def med(x):
        return round(float(np.median(x)), 2) if len(x) else None

    reports = []
    for seconds, rows in replay(hip, ctx, enqueue, replays,
                                lambda: read_rows(lib.mi_timeline_read_rows, wgs)):
        merged = (rows[:, 7] >> np.uint64(63)) == 1
        rows = rows.astype(np.int64)
        t0 = rows[:, 0].min()
        us = lambda f: (rows[:, f] - t0) * TICK_US  # noqa: E731
        start, end, ready, loop, pub, arr = us(0), us(2), us(3), us(4), us(5), us(6)
        published = rows[:, 5] > 0
        last = int(np.argmax(end))
        reports.append({
            "workload": "c2", "plan_grid": list(plan["grid"]), "splits": plan["splits"],
            "graph_us": round(seconds * 1e6, 2), "span_us": round(float(end.max()), 2),
            "start_spread_us": round(float(start.max()), 2),
            "first_batch_ready_us_median": med(ready - start),
            "arithmetic_us_median": med(loop - ready),
            "wave_merge_and_publish_us_median": med((pub - loop)[published]),
            "arrival_us_median": med((arr - pub)[published]),
            "merge_us_median": med((end - arr)[published & merged]),
            "last_workgroup_us": {k: round(float(v[last]), 2) for k, v in
                                  (("start", start), ("ready", ready), ("loop_end", loop),
                                   ("published", pub), ("arrived", arr), ("end", end))}})
    q.free()
    out.free()
    cache.close()
    return reports


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workloads", default="c4,c3,c2")
    ap.add_argument("--replays", type=int, default=3)
    ap.add_argument("--json", default="")
    args = ap.parse_args()
    chosen = [w.strip() for w in args.workloads.split(",") if w.strip()]
    if set(chosen) - {"c4", "c3", "c2"} or args.replays < 1:
        print("workloads: c4, c3, c2; replays >= 1", file=sys.stderr)
        return 2
    hip = bench.Hip()
    ctx = mi_attn.Context(0)
    lib = mi_attn.lib()
    for name in ("mi_timeline_read_stream", "mi_timeline_read_prefill", "mi_timeline_read_rows"):
        getattr(lib, name).argtypes = [ctypes.c_void_p, ctypes.c_uint64]
        getattr(lib, name).restype = ctypes.c_int32
    result = {"device": ctx.device_name, "compute_units": ctx.compute_units, "replays": []}
    if "c4" in chosen:
        result["replays"] += c4_timeline(hip, ctx, lib, args.replays)
    if "c3" in chosen:
        result["replays"] += c3_timeline(hip, ctx, lib, args.replays)
    if "c2" in chosen:
        result["replays"] += c2_timeline(hip, ctx, lib, args.replays)
    for r in result["replays"]:
        print(json.dumps(r), flush=True)
    if args.json:
        Path(args.json).write_text(json.dumps(result, indent=1) + "\n")
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
