"""The reference's own attention test cases, regenerated exactly.

Inputs are the closed-form patterns of crates/metal-infer-core/tests/gpu.rs
(f32 arithmetic, then f16 round-to-nearest-even as MetalContext::tensor_f16
does, context.rs:756-774). Each case records where it comes from.
"""
from __future__ import annotations

import numpy as np


def _f32_to_f16_bits(values: np.ndarray) -> np.ndarray:
    # numpy's float32 -> float16 cast rounds to nearest even, like
    # half::f16::from_f32; tests/test_oracle.py pins both against each other.
    return values.astype(np.float32).astype(np.float16).view(np.uint16)


def pattern(n: int, kind: str) -> np.ndarray:
    """f16 bits of one of the reference's input formulas over 0..n-1."""
    i = np.arange(n, dtype=np.int64)
    f = np.float32
    if kind == "mod41":      # gpu.rs:619-621, 775-777
        x = (i % 41).astype(f) / f(41.0) - f(0.5)
    elif kind == "mod43":    # gpu.rs:648-650, 700-702, bench.rs:973-975
        x = (i % 43).astype(f) / f(43.0) - f(0.5)
    elif kind == "mod37":    # gpu.rs:622-624, 651-653, 703-705; bench.rs:976-978
        x = (i % 37).astype(f) / f(37.0) - f(0.25)
    elif kind == "mod37h":   # gpu.rs:778-780 (mod 37 minus 0.5), 741-743
        x = (i % 37).astype(f) / f(37.0) - f(0.5)
    elif kind == "mod29":    # gpu.rs:625-627, 654-656, 781-783; bench.rs:979-981
        x = (i % 29).astype(f) / f(29.0)
    elif kind == "mod29h":   # gpu.rs:706-708
        x = (i % 29).astype(f) / f(29.0) - f(0.5)
    elif kind == "pm2_q":    # gpu.rs:734-736: 2 if i % 3 == 0 else -2
        x = np.where(i % 3 == 0, f(2.0), f(-2.0))
    elif kind == "pm2_k":    # gpu.rs:738-740: 2 if i % 7 < 3 else -2
        x = np.where(i % 7 < 3, f(2.0), f(-2.0))
    elif kind == "opt_q":    # ops.rs:1424-1426
        x = ((i * 17 % 101).astype(f) - f(50.0)) / f(101.0)
    elif kind == "opt_k":    # ops.rs:1436-1438
        x = ((i * 29 % 127).astype(f) - f(63.0)) / f(127.0)
    elif kind == "opt_v":    # ops.rs:1439-1441
        x = ((i * 13 % 89).astype(f) - f(44.0)) / f(89.0)
    else:
        raise KeyError(kind)
    return _f32_to_f16_bits(x)


def build(case: dict) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(q [T,Hq,D], k [L,Hkv,D], v [L,Hkv,D]) f16 bits for a case."""
    T, L, hq, hkv, d = case["T"], case["L"], case["hq"], case["hkv"], case["d"]
    q = pattern(T * hq * d, case["q"]).reshape(T, hq, d)
    k = pattern(L * hkv * d, case["k"]).reshape(L, hkv, d)
    v = pattern(L * hkv * d, case["v"]).reshape(L, hkv, d)
    return q, k, v


def attention_cases() -> list[dict]:
    cases = []
    # tiled_attention_matches_reference (gpu.rs:613-679)
    cases.append(dict(name="tiled_T2_L2", src="gpu.rs:617-645", T=2, L=2, hq=2, hkv=1, d=128,
                      off=0, q="mod41", k="mod37", v="mod29",
                      kinds=("reference", "tiled")))
    cases.append(dict(name="tiled_T1_L17", src="gpu.rs:647-677", T=1, L=17, hq=2, hkv=1, d=128,
                      off=16, q="mod43", k="mod37", v="mod29",
                      kinds=("reference", "tiled", "decode-split-kv", "flash-decode")))
    # flash_prefill_matches_reference_at_tile_edges (gpu.rs:681-727)
    for d in (1, 2, 4, 8, 16, 32, 64, 128, 256):
        for T, L in ((1, 1), (31, 31), (32, 32), (33, 33), (63, 63), (64, 64), (65, 65),
                     (33, 65)):
            cases.append(dict(name=f"prefill_d{d}_T{T}_L{L}", src="gpu.rs:681-727", T=T, L=L,
                              hq=4, hkv=2, d=d, off=L - T, q="mod43", k="mod37", v="mod29h",
                              kinds=("reference", "flash-prefill", "tiled")))
    # flash_decode_matches_reference_across_block_boundaries (gpu.rs:729-768)
    for L in (1, 63, 64, 65, 256, 640, 8192):
        cases.append(dict(name=f"decode_blocks_L{L}", src="gpu.rs:729-768", T=1, L=L, hq=2,
                          hkv=1, d=128, off=L - 1, q="pm2_q", k="pm2_k", v="mod37h",
                          kinds=("reference", "flash-decode", "decode-split-kv")))
    # flash_decode_..._multiple_gqa_groups_and_causal_limit (gpu.rs:770-808)
    for off in (62, 64):
        cases.append(dict(name=f"decode_gqa_off{off}", src="gpu.rs:770-808", T=1, L=65, hq=16,
                          hkv=8, d=128, off=off, q="mod41", k="mod37h", v="mod29",
                          kinds=("reference", "flash-decode", "decode-split-kv")))
    # flash_decode_128_is_bit_exact_to_legacy inputs (ops.rs:1416-1476)
    for L in (256, 511, 576, 1024, 2048):
        cases.append(dict(name=f"decode_opt_L{L}", src="ops.rs:1416-1476", T=1, L=L, hq=2,
                          hkv=1, d=128, off=L - 1, q="opt_q", k="opt_k", v="opt_v",
                          kinds=("flash-decode", "decode-split-kv")))
    return cases
