"""GPU check of the timeline build (libmi_attn_timeline.so,
include/mi_timeline.h): metal-infer-rs_amd/timeline.py replays c4, c3 and
c2 once in its own process and reports per-workgroup timelines whose stamps are
ordered and complete."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def test_timeline_reports_ordered_stamps(tmp_path):
    out = tmp_path / "timeline.json"
    subprocess.run([sys.executable, str(ROOT / "metal-infer-rs_amd" / "timeline.py"),
                    "--replays", "1", "--json", str(out)], check=True, timeout=300)
    result = json.loads(out.read_text())
    by = {r["workload"]: r for r in result["replays"]}
    c4, c3, c2 = by["c4"], by["c3"], by["c2"]
    # c4: every workgroup of the stream-K grid ran (two per CU) and ended
    # after its prologue; pieces are 1 to 3 per workgroup.
    assert 0 < c4["prologue_us_median"] < c4["span_us"] <= c4["graph_us"]
    assert sum(c4["pieces_per_workgroup"].values()) == 2 * result["compute_units"]
    assert set(c4["pieces_per_workgroup"]) <= {"1", "2", "3"}  # JSON keys
    assert 0 < c4["epilogue_share_of_workgroup_time"] < 0.5
    assert c4["running_every_5us"][-1] == 0
    # c3: the ordered split plan's 504 pieces all ran a key loop; the loops
    # end after the first tile and before the span; splits publish, arrive
    # and one of them merges.
    assert c3["pieces"] == 504 and c3["splits"] == 3
    assert 0 < c3["first_tile_ready_us_median"] < c3["loop_end_us"]["median"] <= c3["span_us"]
    assert c3["publish_us_median"] > 0 and c3["arrival_us_median"] > 0
    assert c3["merge_us_median"] > 0
    assert c3["span_us"] <= c3["graph_us"]
    # c2: the (split, KV head) grid of FlashDecode; every split but the
    # merger's publishes, arrives, and the last arriver of each head merges.
    assert c2["splits"] > 1 and c2["plan_grid"][1] == 8
    last = c2["last_workgroup_us"]
    assert (last["start"] <= last["ready"] <= last["loop_end"] <= last["published"]
            <= last["arrived"] <= last["end"] == c2["span_us"])
    assert c2["first_batch_ready_us_median"] > 0 and c2["merge_us_median"] > 0
    assert c2["span_us"] <= c2["graph_us"]
