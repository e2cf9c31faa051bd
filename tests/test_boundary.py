"""CPU tests of the C-ABI boundary: loading, exports, host-side validation.

No GPU work happens here. mi_attention_plan runs the same validation and
kernel choice as mi_attention without touching device memory, so every
error path of ops.rs:1065-1150 is forced from the host.
"""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

import mi_attn
from mi_attn import (DECODE_SPLIT_KV, FLASH_DECODE, FLASH_PREFILL, REFERENCE, TILED, F16, F32,
                     AttentionConfig, MiError, describe)

ROOT = Path(__file__).resolve().parent.parent
FAKE = 0x7F0000000000  # 256-B aligned address; plan() never dereferences it


def tensor(shape, dtype=F16, strides=None, offset=0):
    return mi_attn.Tensor(describe(FAKE + offset, shape, strides, dtype))


def plan(q, k, v, cfg, kind, block=0, threads=0):
    return mi_attn.plan(q, k, v, cfg, kind, block, threads)


def declared(header: str) -> list[str]:
    text = (ROOT / "include" / header).read_text()
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))


def exported(lib: Path) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], check=True,
                         capture_output=True, text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


@pytest.mark.parametrize("header,lib", [("mi_attn.h", "libmi_attn.so"),
                                        ("mi_bench.h", "libmi_bench.so")])
def test_library_exports_every_declared_symbol(header, lib):
    path = ROOT / "metal-infer-rs_amd" / lib
    names = declared(header)
    assert len(names) > 0
    missing = set(names) - exported(path)
    assert not missing, f"{lib} lacks {sorted(missing)}"
    handle = ctypes.CDLL(str(path))
    for name in names:
        getattr(handle, name)


def test_abi_version_and_status_names():
    assert mi_attn.lib().mi_abi_version() == 1
    assert mi_attn.lib().mi_status_name(8) == b"invalid tensor shape"
    assert mi_attn.lib().mi_status_name(9) == b"unsupported dtype"


def test_product_library_does_not_link_the_oracle():
    out = subprocess.run(["ldd", str(ROOT / "metal-infer-rs_amd" / "libmi_attn.so")],
                         capture_output=True, text=True).stdout
    assert "oracle" not in out
    assert "orc_" not in " ".join(exported(ROOT / "metal-infer-rs_amd" / "libmi_attn.so"))


# ------------------------------------------- validation (ops.rs:1065-1150) --

def _decode(hq=16, hkv=8, d=128, L=2048):
    return (tensor((1, hq, d)), tensor((L, hkv, d)), tensor((L, hkv, d)),
            AttentionConfig(hq, hkv, d, True, L - 1))


def expect(status, fragment, fn, *args):
    with pytest.raises(MiError) as err:
        fn(*args)
    assert err.value.name == status
    assert fragment in err.value.message


def test_dtype_and_rank_errors():
    q, k, v, cfg = _decode()
    expect("MI_ERR_DTYPE", "expected f16, got f32", plan, tensor((1, 16, 128), F32), k, v, cfg,
           TILED)
    expect("MI_ERR_SHAPE", "query must have rank 3", plan, tensor((16, 128)), k, v, cfg, TILED)
    expect("MI_ERR_SHAPE", "key must have rank 3", plan, q, tensor((2048, 1024)), v, cfg, TILED)
    expect("MI_ERR_SHAPE", "value must have rank 3", plan, q, k, tensor((2048, 1024)), cfg, TILED)


def test_shape_config_and_ratio_errors():
    q, k, v, cfg = _decode()
    expect("MI_ERR_SHAPE", "do not match config", plan, q, k, v,
           AttentionConfig(16, 4, 128, True, 0), TILED)
    expect("MI_ERR_SHAPE", "do not match config", plan, q, k, tensor((2047, 8, 128)), cfg, TILED)
    q3, k3 = tensor((1, 12, 128)), tensor((4, 8, 128))
    expect("MI_ERR_SHAPE", "divisible by kv_heads", plan, q3, k3, k3,
           AttentionConfig(12, 8, 128, True, 3), TILED)
    expect("MI_ERR_SHAPE", "do not match config", plan, q3, k3, k3,
           AttentionConfig(12, 0, 128, True, 3), TILED)


def test_head_dim_rules():
    q, k = tensor((2, 4, 96)), tensor((2, 2, 96))
    cfg = AttentionConfig(4, 2, 96, True, 0)
    expect("MI_ERR_SHAPE", "power-of-two head_dim <= 256", plan, q, k, k, cfg, FLASH_PREFILL)
    assert plan(q, k, k, cfg, REFERENCE)["kernel"] == "attn_naive"  # Reference takes any D
    q5, k5 = tensor((2, 4, 512)), tensor((2, 2, 512))
    expect("MI_ERR_SHAPE", "power-of-two head_dim <= 256", plan, q5, k5, k5,
           AttentionConfig(4, 2, 512, True, 0), TILED)


def test_decode_kinds_need_one_token():
    q, k = tensor((2, 2, 128)), tensor((8, 1, 128))
    cfg = AttentionConfig(2, 1, 128, True, 6)
    for kind in (DECODE_SPLIT_KV, FLASH_DECODE):
        expect("MI_ERR_SHAPE", "exactly one query token", plan, q, k, k, cfg, kind)


def test_flash_decode_configuration_is_validated():
    q, k, v, cfg = _decode()
    expect("MI_ERR_SHAPE", "block size must be 32, 64, 128, or 256", plan, q, k, v, cfg,
           FLASH_DECODE, 48, 256)
    expect("MI_ERR_SHAPE", "threadgroup size must be 128 or 256", plan, q, k, v, cfg,
           FLASH_DECODE, 64, 64)
    for block in (32, 64, 128, 256):
        for threads in (128, 256):
            p = plan(q, k, v, cfg, FLASH_DECODE, block, threads)
            assert p["block_keys"] == block and p["block_threads"] == threads
            assert p["splits"] == -(-2048 // block)
    # untuned default (context.rs:258-267 keeps (64, 256) for Apple GPUs):
    # 128-key splits, 8 waves per workgroup, merge inside the launch
    # (measured fastest on MI355X); the configuration query still reports
    # the nearest reference configuration, (128, 256)
    p = plan(q, k, v, cfg, FLASH_DECODE)
    assert (p["block_keys"], p["block_threads"]) == (128, 512)
    p = plan(q, k, v, cfg, DECODE_SPLIT_KV)
    assert p["block_threads"] == 512


def test_flash_decode_accepts_every_gqa_ratio():
    # Deliberate extension: the reference requires Hq == 2 * Hkv (ops.rs:1141).
    for hq, hkv in ((16, 8), (32, 8), (64, 8), (8, 8), (24, 8)):
        q, k, v, cfg = _decode(hq, hkv)
        p = plan(q, k, v, cfg, FLASH_DECODE)
        assert p["kernel"] == "attn_rows"
        group = hq // hkv
        chunk = max(c for c in (8, 4, 2, 1) if group % c == 0)
        assert p["grid"][1] == hkv * (group // chunk)  # each KV row read once per chunk


def test_causal_window_bounds_the_splits():
    # Keys past query_offset are never visited: 65 keys, offset 62 -> 63 visible.
    q, k, v = tensor((1, 16, 128)), tensor((65, 8, 128)), tensor((65, 8, 128))
    p = plan(q, k, v, AttentionConfig(16, 8, 128, True, 62), FLASH_DECODE, 32, 128)
    assert p["splits"] == 2
    p = plan(q, k, v, AttentionConfig(16, 8, 128, False, 62), FLASH_DECODE, 32, 128)
    assert p["splits"] == 3


def test_kernel_choice_and_layout_fallback():
    q, k, v, cfg = _decode()
    assert plan(q, k, v, cfg, REFERENCE)["kernel"] == "attn_naive"
    assert plan(q, k, v, cfg, DECODE_SPLIT_KV)["kernel"] == "attn_rows"
    # head-major cache view [L, Hkv, D] with strides (D, cap * D, 1)
    kh = tensor((2048, 8, 128), strides=(128, 4096 * 128, 1))
    assert plan(q, kh, kh, cfg, FLASH_DECODE)["kernel"] == "attn_rows"
    # rows that are not 16-byte aligned cannot feed 128-bit loads
    odd = tensor((2048, 8, 128), strides=(1028, 128, 1))
    assert plan(q, odd, odd, cfg, FLASH_DECODE)["kernel"] == "attn_naive"


def test_split_k_sizes_cover_the_window():
    for L in (1, 63, 64, 65, 256, 640, 2048, 8192, 20480):
        q, k, v, cfg = _decode(L=L)
        p = plan(q, k, v, cfg, DECODE_SPLIT_KV)
        assert p["splits"] * p["block_keys"] >= L
        assert (p["splits"] - 1) * p["block_keys"] < L
        if p["splits"] > 1:
            assert p["scratch_bytes"] == 8 * p["splits"] * 2 * 130 * 4


# ---------------------------------------- policy (qwen3.rs:799-822) -------

def test_kind_policy_matches_reference_cases():
    kind = mi_attn.attention_kind_for_tokens
    # qwen3.rs:1044-1081
    assert kind(TILED, 1, 640, 2) == FLASH_DECODE
    assert kind(TILED, 1, 255, 2) == DECODE_SPLIT_KV
    assert kind(TILED, 31, 31, 2) == TILED
    assert kind(TILED, 32, 32, 2) == FLASH_PREFILL
    assert kind(TILED, 512, 512, 2) == FLASH_PREFILL
    assert kind(REFERENCE, 1, 640, 2) == REFERENCE
    # generalised: the split-K kernel serves ratio 4 too (reference: DecodeSplitKv)
    assert kind(TILED, 1, 640, 4) == FLASH_DECODE
    assert kind(FLASH_DECODE, 8, 640, 2) == TILED
    assert kind(DECODE_SPLIT_KV, 1, 640, 2) == DECODE_SPLIT_KV
    assert kind(FLASH_PREFILL, 1, 300, 8) == FLASH_DECODE
    assert kind(FLASH_PREFILL, 1, 100, 8) == DECODE_SPLIT_KV


# ---------------------------------------------- tensor views ---------------

def test_prefix_and_reshape():
    t = tensor((4096, 8, 128), strides=(128, 4096 * 128, 1))
    p = t.prefix(2048)
    assert p.shape == (2048, 8, 128) and p.strides == t.strides and p.data_ptr == t.data_ptr
    with pytest.raises(MiError, match="outside capacity"):
        t.prefix(0)
    with pytest.raises(MiError, match="outside capacity"):
        t.prefix(4097)
    c = tensor((4, 6))
    assert c.reshape((2, 12)).shape == (2, 12)
    with pytest.raises(MiError):
        c.reshape((5, 5))
    with pytest.raises(MiError, match="contiguous"):
        t.reshape((4096, 1024))


def test_flash_prefill_routes_to_mfma_kernel():
    for d, expected in ((128, "attn_prefill"), (64, "attn_prefill"), (32, "attn_prefill"),
                        (16, "attn_rows"), (256, "attn_prefill")):
        q, k = tensor((2048, 16, d)), tensor((2048, 8, d))
        p = plan(q, k, k, AttentionConfig(16, 8, d, True, 0), FLASH_PREFILL)
        assert p["kernel"] == expected, d
    # c5: 4096 tokens x 8 heads per KV head = 128 row tiles of 256 (8 waves),
    # 1024 workgroups: at least four per CU
    q, k = tensor((4096, 64, 128)), tensor((20480, 8, 128))
    p = plan(q, k, k, AttentionConfig(64, 8, 128, True, 16384), FLASH_PREFILL)
    assert p["kernel"] == "attn_prefill" and p["grid"][:2] == (128, 8) and p["block_threads"] == 512
    # half of c5's rows: 512 such workgroups, so 128-row tiles
    q = tensor((2048, 64, 128))
    p = plan(q, k, k, AttentionConfig(64, 8, 128, True, 16384), FLASH_PREFILL)
    assert p["grid"][:2] == (128, 8) and p["block_threads"] == 256
    # c3: 2048 x 2 = 4096 packed rows. It takes key splits, which keep the
    # 128-row tile at two workgroups per CU (256 threads).
    q, k = tensor((2048, 16, 128)), tensor((2048, 8, 128))
    p = plan(q, k, k, AttentionConfig(16, 8, 128, True, 0), FLASH_PREFILL)
    assert p["splits"] > 1 and p["block_threads"] == 256, p


def _pieces(T, G, L, off, per_split_keys, block_m=128):
    """Non-empty (row tile, key split) pieces of one KV head."""
    tiles = []
    for t in range(-(-T * G // block_m)):
        t_last = (min(T * G, (t + 1) * block_m) - 1) // G
        tiles.append(-(-min(L, off + t_last + 1) // 64))
    per = per_split_keys // 64
    return sum(-(-n // per) for n in tiles), max(tiles)


def test_small_prefill_grids_split_the_keys():
    # c3: 256 workgroups of 128 rows on 256 CUs. The split count is the largest
    # whose non-empty pieces all fit at two workgroups per CU: at most 3 splits
    # of at most 11 key tiles, 63 pieces per KV head, launched as an ordered
    # grid of exactly those pieces (63 x 8).
    q, k = tensor((2048, 16, 128)), tensor((2048, 8, 128))
    p = plan(q, k, k, AttentionConfig(16, 8, 128, True, 0), FLASH_PREFILL)
    assert p["grid"] == (63, 8, 1) and p["splits"] == 3 and p["block_keys"] == 11 * 64
    assert p["block_threads"] == 256
    # per row (m, l) as f32 + 128 O values as f16 (8-byte slots of 64 lanes),
    # for 128 rows (4 waves) per row tile
    assert p["scratch_bytes"] == 3 * 32 * 8 * 4 * (1 + 128 // 8) * 64 * 8
    pieces, max_tiles = _pieces(2048, 2, 2048, 0, p["block_keys"])
    assert pieces == 63 and pieces * 8 <= 2 * 256
    finer = -(-max_tiles // 4) * 64  # one more split would not fit
    assert _pieces(2048, 2, 2048, 0, finer)[0] * 8 > 2 * 256
    # more pieces per KV head than the ordered grid holds (64): the
    # (row tile, KV head, split) grid, splits past a row tile's window empty
    q, k = tensor((333, 16, 128)), tensor((633, 1, 128))
    p = plan(q, k, k, AttentionConfig(16, 1, 128, True, 300), FLASH_PREFILL)
    assert p["splits"] > 1 and p["grid"] == (42, 1, p["splits"]), p
    assert _pieces(333, 16, 633, 300, p["block_keys"])[0] > 64
    # c5 fills the chip on its own: no split, no scratch
    q, k = tensor((4096, 64, 128)), tensor((20480, 8, 128))
    p = plan(q, k, k, AttentionConfig(64, 8, 128, True, 16384), FLASH_PREFILL)
    assert p["splits"] == 1 and p["scratch_bytes"] == 0
    # fewer than 8 key tiles: not split
    q, k = tensor((128, 16, 128)), tensor((128, 8, 128))
    assert plan(q, k, k, AttentionConfig(16, 8, 128, True, 0), FLASH_PREFILL)["splits"] == 1
    # every split is a whole number of 64-key tiles, together covering the window
    q, k = tensor((1024, 16, 128)), tensor((1024, 8, 128))
    p = plan(q, k, k, AttentionConfig(16, 8, 128, True, 0), FLASH_PREFILL)
    assert 2 <= p["splits"] <= 8 and p["block_keys"] % 64 == 0
    assert p["splits"] * p["block_keys"] >= 1024 > (p["splits"] - 1) * p["block_keys"]
    rows = 256 if p["block_threads"] == 512 else 128
    per_cu = 1 if rows == 256 else 2
    assert _pieces(1024, 2, 1024, 0, p["block_keys"], block_m=rows)[0] * 8 <= per_cu * 256


def test_prefill_needs_non_negative_position_strides():
    """The MFMA prefill kernel addresses a key tile with unsigned 32-bit byte
    offsets from the tile base, so K or V views whose position stride is
    negative (a reversed cache) or spans 4 GiB per tile take the rows kernel,
    which uses 64-bit offsets."""
    L, hkv, d = 2048, 8, 128
    q = tensor((L, 16, d))
    cfg = AttentionConfig(16, 8, d, True, 0)
    fwd = tensor((L, hkv, d))
    # the same rows, last position first: element 0 is the last row in memory
    rev = tensor((L, hkv, d), strides=(-hkv * d, d, 1), offset=(L - 1) * hkv * d * 2)
    assert plan(q, fwd, fwd, cfg, FLASH_PREFILL)["kernel"] == "attn_prefill"
    for k, v in ((rev, fwd), (fwd, rev), (rev, rev)):
        p = plan(q, k, v, cfg, FLASH_PREFILL)
        assert p["kernel"] == "attn_rows", (k.strides, v.strides, p)
    # 64 rows at a stride of 2^25 halves span 4 GiB
    huge = tensor((L, hkv, d), strides=(1 << 25, d, 1))
    assert plan(q, huge, fwd, cfg, FLASH_PREFILL)["kernel"] == "attn_rows"
    near = tensor((L, hkv, d), strides=((1 << 25) - 1024, d, 1))
    assert plan(q, near, fwd, cfg, FLASH_PREFILL)["kernel"] == "attn_prefill"


def test_probe_library_exports_its_header():
    """libmi_probe.so (calibration kernels, include/mi_probe.h) is separate
    from the attention library, which exports none of its symbols."""
    path = ROOT / "metal-infer-rs_amd" / "libmi_probe.so"
    names = declared("mi_probe.h")
    assert names == ["mi_probe_empty", "mi_probe_read", "mi_probe_split_decode"]
    assert set(names) <= exported(path)
    assert not set(names) & exported(ROOT / "metal-infer-rs_amd" / "libmi_attn.so")


def test_timeline_library_is_the_attention_library_plus_its_readers():
    """libmi_attn_timeline.so (include/mi_timeline.h) is built from the same
    sources with per-workgroup timestamps: it exports every attention entry
    point and the two readers; the product library exports no reader."""
    pkg = ROOT / "metal-infer-rs_amd"
    names = declared("mi_timeline.h")
    assert sorted(names) == ["mi_timeline_read_prefill", "mi_timeline_read_rows",
                             "mi_timeline_read_stream"]
    timeline = exported(pkg / "libmi_attn_timeline.so")
    assert set(names) <= timeline
    assert set(declared("mi_attn.h")) <= timeline
    assert not set(names) & exported(pkg / "libmi_attn.so")


def test_compare_statistics_follow_the_reference_indexing():
    """bench.rs:1995-2008: median = sorted[n / 2], p95 = sorted[round((n - 1)
    * 0.95)], mean over all samples, in ms."""
    import bench

    samples = [i * 1e-3 for i in (5, 1, 4, 2, 3, 10, 9, 8, 7, 6)]
    mean, median, p95 = bench.duration_stats(samples)
    assert mean == pytest.approx(5.5)
    assert median == pytest.approx(6.0)   # sorted[5]
    assert p95 == pytest.approx(10.0)     # sorted[round(8.55)] = sorted[9]
    assert bench.duration_stats([2e-3])[1:] == pytest.approx((2.0, 2.0))
