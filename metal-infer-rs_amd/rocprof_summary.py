"""Summaries of rocprofv3 output for the committed profile records.

  stats DIR --command CMD [--last N]
      Markdown table of a `rocprofv3 --kernel-trace --stats --output-format csv`
      run: calls and average / min / max duration per kernel (and, with --last,
      the average of each kernel's last N dispatches, in trace order).
  counters --run WORKLOAD=DIR[,DIR...] ... --command CMD [--skip N]
      SQ / GRBM counters of each workload's dominant kernel from
      `rocprofv3 --pmc` passes (per-dispatch means after the first N dispatches)
      and what they imply: the shader clock (GRBM_GUI_ACTIVE over the XCDs and
      the dispatch's duration), the MFMA pipes' busy share of SIMD cycles
      (SQ_VALU_MFMA_BUSY_CYCLES over SIMDs x GRBM cycles), and the same against
      the 2.4 GHz peak clock.
  traffic --copy-bytes N --run WORKLOAD=FETCH_DIR,WRITE_DIR ... --command CMD
      HBM bytes per dispatch of each workload's dominant kernel from two
      `rocprofv3 --pmc` passes (FETCH_SIZE, then WRITE_SIZE; KiB per
      dispatch), each scaled by what the same counter reads for the copy
      kernel (copy_kv_kernel, N bytes read and N written) that ran in the same
      process. Writes a JSON record and a markdown table.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import re
import sys
from collections import defaultdict
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent))

# Each workload's dominant launch record and the rocprof kernels of one call
# (the batched decode is its stream kernel plus the merge launch; the other
# calls are one kernel).
DOMINANT = {
    "c2": ("attn_rows", ("attn_rows_kernel",)),
    "c4": ("attn_decode_stream", ("attn_decode_stream_kernel", "attn_stream_merge_kernel")),
    "c3": ("attn_prefill", ("attn_prefill_kernel",)),
    "c5": ("attn_prefill", ("attn_prefill_kernel",)),
}
COPY_KERNEL = "copy_kv_kernel"


def short(name: str) -> str:
    """'void mi::kernels::(anonymous namespace)::attn_rows_kernel<128, 4, 8>(...)'
    -> 'attn_rows_kernel<128, 4, 8>'."""
    m = re.search(r"(\w+_kernel(?:<[^>]*>)?)\(", name)
    return m.group(1) if m else name


def base(name: str) -> str:
    return short(name).split("<")[0]


def one_file(directory: str, suffix: str) -> Path:
    found = sorted(glob.glob(f"{directory}/**/*{suffix}", recursive=True))
    if not found:
        raise SystemExit(f"no *{suffix} under {directory}")
    return Path(found[0])


def stats(args) -> None:
    """Per (kernel, grid) durations from the kernel trace (one kernel serves
    several workloads, told apart by grid), then rocprofv3's own --stats
    table."""
    trace: dict[tuple[str, str], list[float]] = defaultdict(list)
    rows = sorted(csv.DictReader(one_file(args.dir, "kernel_trace.csv").open()),
                  key=lambda r: int(r["Start_Timestamp"]))
    for r in rows:
        grid = "x".join(str(int(r[f"Grid_Size_{a}"]) // int(r[f"Workgroup_Size_{a}"]))
                        for a in "XYZ")
        ns = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        trace[(short(r["Kernel_Name"]), grid)].append(ns / 1e3)
    print(f"# Kernel durations: {args.title}\n" if args.title else "# Kernel durations\n")
    print(f"Command (from the repository root on the GPU box):\n\n    {args.command}\n")
    print("## Per kernel and workgroup grid (kernel trace)\n")
    last = args.last
    if last:
        print(f"`timed average` is over each row's last {last} dispatches, which lie in "
              f"bench.py's timed region: one replay of a graph of the workload's calls ({last}; "
              "c2 rounds up to whole rotations of its 64 caches). The earlier dispatches are "
              "the eager calls before capture and the untimed warmup replays.\n")
    print("| kernel | workgroups | calls | average (us) | timed average (us) | median (us) | "
          "min (us) | max (us) |")
    print("|---|---|---:|---:|---:|---:|---:|---:|")
    for (name, grid), us in sorted(trace.items(), key=lambda kv: -sum(kv[1])):
        tail = us[-last:] if last and len(us) >= last else []
        timed = f"{sum(tail) / len(tail):.2f}" if tail else "—"
        us = sorted(us)
        print(f"| `{name}` | {grid} | {len(us)} | {sum(us) / len(us):.2f} | {timed} | "
              f"{us[len(us) // 2]:.2f} | {us[0]:.2f} | {us[-1]:.2f} |")
    rows = list(csv.DictReader(one_file(args.dir, "kernel_stats.csv").open()))
    print("\n## rocprofv3 --stats\n")
    print("| kernel | calls | average (us) | min (us) | max (us) | share of GPU time |")
    print("|---|---:|---:|---:|---:|---:|")
    for r in rows:
        print(f"| `{short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
              f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
              f"{float(r['Percentage']):.1f}% |")


def counter_means(directory: str, counter: str) -> dict[str, tuple[float, int]]:
    """Mean value per dispatch of `counter` for every kernel base name."""
    values: dict[str, list[float]] = defaultdict(list)
    for r in csv.DictReader(one_file(directory, "counter_collection.csv").open()):
        if r["Counter_Name"] == counter:
            values[base(r["Kernel_Name"])].append(float(r["Counter_Value"]))
    return {k: (sum(v) / len(v), len(v)) for k, v in values.items()}


def traffic(args) -> None:
    import workloads

    out = {"source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, KiB per dispatch",
           "command": args.command, "copy_bytes": args.copy_bytes, "workloads": {}}
    lines = []
    for spec in args.run:
        workload, dirs = spec.split("=", 1)
        fetch_dir, write_dir = dirs.split(",")
        record, kernels = DOMINANT[workload]
        fetch = counter_means(fetch_dir, "FETCH_SIZE")
        write = counter_means(write_dir, "WRITE_SIZE")
        copy_kib = args.copy_bytes / 1024
        f_scale = copy_kib / fetch[COPY_KERNEL][0]
        w_scale = copy_kib / write[COPY_KERNEL][0]
        # One dispatch of each of the call's kernels.
        fetch_kib = sum(fetch[k][0] for k in kernels)
        write_kib = sum(write[k][0] for k in kernels)
        fetch_b = fetch_kib * f_scale * 1024
        write_b = write_kib * w_scale * 1024
        case = workloads.case(int(workload[1:]), generate=False)
        algorithmic = case.algorithmic_bytes()
        out["workloads"][workload] = {
            "kernel": record, "rocprof_kernels": list(kernels),
            "dispatches": fetch[kernels[0]][1],
            "fetch_kib_raw": round(fetch_kib, 1), "write_kib_raw": round(write_kib, 1),
            "copy_fetch_kib_raw": round(fetch[COPY_KERNEL][0], 1),
            "copy_write_kib_raw": round(write[COPY_KERNEL][0], 1),
            "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
            "fetch_bytes": int(fetch_b), "write_bytes": int(write_b),
            "traffic_bytes": int(fetch_b + write_b), "algorithmic_bytes": algorithmic,
            "traffic_over_algorithmic": round((fetch_b + write_b) / algorithmic, 3)}
        kernel = " + ".join(kernels)
        e = out["workloads"][workload]
        lines.append(f"| {workload} | `{kernel}` | {e['dispatches']} | {e['fetch_kib_raw']:.0f} | "
                     f"{e['write_kib_raw']:.0f} | {e['fetch_scale']:.3f} / {e['write_scale']:.3f} | "
                     f"{e['traffic_bytes'] / 1e6:.2f} | {algorithmic / 1e6:.2f} | "
                     f"{e['traffic_over_algorithmic']:.2f} |")
    Path(args.json).write_text(json.dumps(out, indent=1) + "\n")
    with open(args.md, "w") as f:
        f.write("# HBM traffic per dispatch (rocprofv3 PMC)\n\n")
        f.write("Two counter passes per workload, FETCH_SIZE then WRITE_SIZE (KiB per "
                "dispatch), each scaled by the reading of the same counter for "
                f"copy_kv_kernel copying {args.copy_bytes} bytes (read and written once) "
                "in the same process.\n\nCommands (from the repository root on the GPU box):\n\n")
        for c in args.command.split(" ;; "):
            f.write(f"    {c}\n")
        f.write("\n| workload | kernel | dispatches | FETCH KiB raw | WRITE KiB raw | "
                "scale fetch / write | traffic MB | algorithmic MB | ratio |\n")
        f.write("|---|---|---:|---:|---:|---:|---:|---:|---:|\n")
        f.write("\n".join(lines) + "\n")


# MI355X: 256 CUs of 4 SIMDs in 8 XCDs; GRBM_GUI_ACTIVE is summed over the
# XCDs. Peak clock of the dense MFMA rating (2.5 PFLOP/s f16).
XCDS, SIMDS, PEAK_HZ = 8, 1024, 2.4e9


def counters(args) -> None:
    out = {"source": "rocprofv3 --pmc, per-dispatch means", "command": args.command,
           "workloads": {}}
    lines = []
    for spec in args.run:
        workload, dirs = spec.split("=", 1)
        record, kernels = DOMINANT[workload]
        values: dict[str, list[float]] = defaultdict(list)
        durations: list[float] = []
        for directory in dirs.split(","):
            seen: dict[str, int] = defaultdict(int)
            rows = sorted(csv.DictReader(one_file(directory, "counter_collection.csv").open()),
                          key=lambda r: int(r["Dispatch_Id"]))
            for r in rows:
                if base(r["Kernel_Name"]) != kernels[0]:
                    continue
                seen[r["Counter_Name"]] += 1
                if seen[r["Counter_Name"]] <= args.skip:
                    continue
                values[r["Counter_Name"]].append(float(r["Counter_Value"]))
                if r["Counter_Name"] == "GRBM_GUI_ACTIVE":
                    durations.append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e9)
        mean = {k: sum(v) / len(v) for k, v in values.items()}
        entry = {"kernel": kernels[0], "dispatches": len(durations),
                 "counters": {k: round(v, 1) for k, v in sorted(mean.items())}}
        if "GRBM_GUI_ACTIVE" in mean and durations:
            seconds = sum(durations) / len(durations)
            cycles = mean["GRBM_GUI_ACTIVE"] / XCDS
            entry["duration_us"] = round(seconds * 1e6, 2)
            entry["clock_ghz"] = round(cycles / seconds / 1e9, 3)
            if "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
                busy = mean["SQ_VALU_MFMA_BUSY_CYCLES"] / SIMDS
                entry["mfma_busy_of_cycles"] = round(busy / cycles, 4)
                entry["mfma_busy_of_peak_clock"] = round(busy / (seconds * PEAK_HZ), 4)
        if "SQ_INSTS_MFMA" in mean and "SQ_INSTS_VALU" in mean:
            entry["valu_per_mfma"] = round(mean["SQ_INSTS_VALU"] / mean["SQ_INSTS_MFMA"], 3)
            if "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
                entry["busy_cycles_per_mfma"] = round(
                    mean["SQ_VALU_MFMA_BUSY_CYCLES"] / mean["SQ_INSTS_MFMA"], 2)
        out["workloads"][workload] = entry
        lines.append(f"| {workload} | `{kernels[0]}` | {entry['dispatches']} | "
                     f"{entry.get('duration_us', '—')} | {entry.get('clock_ghz', '—')} | "
                     f"{entry.get('mfma_busy_of_cycles', '—')} | "
                     f"{entry.get('mfma_busy_of_peak_clock', '—')} | "
                     f"{entry.get('valu_per_mfma', '—')} |")
    Path(args.json).write_text(json.dumps(out, indent=1) + "\n")
    with open(args.md, "w") as f:
        f.write(f"# {args.title}\n\n" if args.title else "# SQ / GRBM counters\n\n")
        f.write("Per-dispatch means of `rocprofv3 --pmc` passes (the first "
                f"{args.skip} dispatches of each counter skipped as warmup). MI355X: "
                f"{SIMDS} SIMDs in {XCDS} XCDs; GRBM_GUI_ACTIVE is summed over the XCDs, so "
                "clock = GRBM_GUI_ACTIVE / 8 / duration, and the MFMA busy share = "
                "SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs / (GRBM_GUI_ACTIVE / 8). Against "
                "the 2.4 GHz clock of the 2.5 PFLOP/s rating the same busy cycles are "
                "divided by duration x 2.4 GHz.\n\nCommands (from the repository root on "
                "the GPU box):\n\n")
        for c in args.command.split(" ;; "):
            f.write(f"    {c}\n")
        f.write("\n| workload | kernel | dispatches | duration (us) | clock (GHz) | "
                "MFMA busy / cycles | MFMA busy / peak-clock cycles | VALU per MFMA |\n")
        f.write("|---|---|---:|---:|---:|---:|---:|---:|\n")
        f.write("\n".join(lines) + "\n\n## Counter means per dispatch\n\n")
        names = sorted({k for e in out["workloads"].values() for k in e["counters"]})
        f.write("| counter | " + " | ".join(out["workloads"]) + " |\n")
        f.write("|---|" + "---:|" * len(out["workloads"]) + "\n")
        for n in names:
            f.write(f"| {n} | " + " | ".join(
                f"{e['counters'].get(n, float('nan')):.4g}" for e in out["workloads"].values())
                + " |\n")


def main() -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--title", default="")
    s.add_argument("--last", type=int, default=0,
                   help="also average each kernel's last N dispatches (the timed replay)")
    s.add_argument("--command", required=True)
    t = sub.add_parser("traffic")
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--run", action="append", required=True)
    t.add_argument("--command", required=True)
    t.add_argument("--json", required=True)
    t.add_argument("--md", required=True)
    c = sub.add_parser("counters")
    c.add_argument("--run", action="append", required=True)
    c.add_argument("--command", required=True)
    c.add_argument("--skip", type=int, default=2)
    c.add_argument("--title", default="")
    c.add_argument("--json", required=True)
    c.add_argument("--md", required=True)
    args = ap.parse_args()
    {"stats": stats, "traffic": traffic, "counters": counters}[args.cmd](args)


if __name__ == "__main__":
    main()
