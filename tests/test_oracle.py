"""CPU tests that pin the oracle (oracle/attn_oracle.c) before it judges the GPU.

Each oracle function is checked against something that does not share its
code: numpy's IEEE conversions, torch's float64 SDPA (the golden fixtures),
transformers' Qwen3 RMSNorm/RoPE, closed forms, invariants and brute force.
A final group plants plausible mistakes (a transposed operand, an
off-by-one causal window, a dropped key, a wrong scale) and checks that the
pins catch each one.
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
import ref_cases
import workloads
from helpers import f16

GOLDEN = Path(__file__).resolve().parent / "golden" / "attention_golden.npz"


@pytest.fixture(scope="module")
def golden():
    data = np.load(GOLDEN, allow_pickle=False)
    return {name: data[name] for name in data["__names__"].tolist()}


def rand_f16(seed, shape, scale=1.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape) * scale).astype(np.float16).view(np.uint16)


# ------------------------------------------------------------ f16 --------

def test_f16_to_f32_matches_numpy_exhaustively():
    bits = np.arange(65536, dtype=np.uint16)
    ours = oracle.f16_to_f32(bits)
    numpy = bits.view(np.float16).astype(np.float32)
    same = (ours.view(np.uint32) == numpy.view(np.uint32)) | (np.isnan(ours) & np.isnan(numpy))
    assert same.all()


def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(1)
    pieces = [
        rng.standard_normal(2_000_000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(200_000) * 1e-5).astype(np.float32),   # subnormal range
        (rng.standard_normal(200_000) * 6e4).astype(np.float32),    # near overflow
        np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65520.0, 65519.996, 2.0**-24,
                  2.0**-25, 2.0**-25 * 1.0000001, 3 * 2.0**-26, 1.0 + 2.0**-11,
                  1.0 + 3 * 2.0**-11], dtype=np.float32),
    ]
    # every f32 whose low mantissa bits sit exactly on an f16 tie
    halves = np.arange(0x3800, 0x3c00, dtype=np.uint32) << 13 | 0x1000
    pieces.append(halves.view(np.float32))
    x = np.concatenate(pieces)
    ours = oracle.f32_to_f16(x)
    numpy = x.astype(np.float16).view(np.uint16)
    assert (ours == numpy).all()
    nan = oracle.f32_to_f16(np.array([np.nan], dtype=np.float32))
    assert np.isnan(nan.view(np.float16)).all()


# ------------------------------------------------------ generator --------

def test_xorshift_matches_marsaglias_published_xor64():
    """qwen3.rs:1011-1034 is Marsaglia's xor64 (shifts 13, 7, 17; "Xorshift
    RNGs", Journal of Statistical Software 8(14), 2003), whose published seed
    88172645463325252 gives 8748534153485358512, 3040900993826735515,
    3453997556048239312. A wrong shift triple or order fails this; the
    draw is that state over 2^64 (u64::MAX as f64 + 1.0)."""
    import ctypes

    state = ctypes.c_uint64(oracle.lib().orc_xorshift_seed(88172645463325252))
    for expected in (8748534153485358512, 3040900993826735515, 3453997556048239312):
        draw = oracle.lib().orc_xorshift_next_f64(ctypes.byref(state))
        assert state.value == expected
        assert draw == expected / 2.0**64
    # seed 0 is replaced by the golden-ratio word (qwen3.rs:1016-1023)
    assert oracle.lib().orc_xorshift_seed(0) == 0x9E3779B97F4A7C15
    # the package's native generator walks the same stream: its first
    # uniform draw from this seed, scaled to [0, 2^32), is the top word
    first = workloads.uniform_u32(88172645463325252, 0, 0xFFFFFFFE, 1)[0]
    assert first == (8748534153485358512 * 0xFFFFFFFF) >> 64


def test_box_muller_known_answers_from_marsaglias_seed():
    """The normal generator's Box-Muller step as the input spec states it
    (cos branch, u1 replaced by 1 - u1, f64 -> f32 -> f16 RNE), from
    Marsaglia's published xor64 states: draw 0 uses the published first two
    states exactly, later draws the states a Python xor64 gives (checked
    against the third published state). numpy's float64 log/cos and its
    float16 cast are independent of the oracle's C. The sin branch, u1 in
    place of 1 - u1, and swapped uniforms each give different bits here."""
    mask = (1 << 64) - 1

    def step(x):
        x ^= (x << 13) & mask
        x ^= x >> 7
        x ^= (x << 17) & mask
        return x

    states, x = [], 88172645463325252
    for _ in range(16):
        x = step(x)
        states.append(x)
    assert states[:3] == [8748534153485358512, 3040900993826735515, 3453997556048239312]
    u = np.array(states, dtype=np.float64) / 2.0**64
    u1, u2 = u[0::2], u[1::2]

    def spec(a, b, trig=np.cos, flip=True):
        radius = np.sqrt(-2.0 * np.log(1.0 - a if flip else a))
        return (radius * trig(2.0 * np.pi * b)).astype(np.float32).astype(np.float16)

    expected = spec(u1, u2).view(np.uint16)
    got = oracle.normal_f16(88172645463325252, (8,), threads=1)
    assert (got == expected).all(), (got, expected)
    assert (workloads.normal_f16(88172645463325252, 8, threads=1) == expected).all()
    for wrong in (spec(u1, u2, trig=np.sin), spec(u1, u2, flip=False), spec(u2, u1)):
        assert (wrong.view(np.uint16) != expected).any()


def test_xorshift_jump_composes():
    s = oracle.lib().orc_xorshift_seed(12345)
    assert oracle.xorshift_jump(s, 1000 + 2345) == oracle.xorshift_jump(
        oracle.xorshift_jump(s, 1000), 2345)
    draws = oracle.xorshift_draws(12345, 10)
    state = oracle.xorshift_jump(s, 9)
    assert state / 2.0**64 == pytest.approx(draws[8], rel=0, abs=0)


def test_generator_is_thread_count_independent_and_matches_package():
    a = oracle.normal_f16(0x4D490010, (300_001,), threads=1)
    b = oracle.normal_f16(0x4D490010, (300_001,), threads=8)
    c = workloads.normal_f16(0x4D490010, 300_001, threads=3)
    assert (a == b).all() and (a == c).all()
    x = f16(a).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    lengths = oracle.uniform_u32(0x4D490043, 1024, 8192, 32)
    assert (lengths == workloads.uniform_u32(0x4D490043, 1024, 8192, 32)).all()
    assert lengths.min() >= 1024 and lengths.max() <= 8192


# ------------------------------------------------------ golden -----------

@pytest.mark.parametrize("case", ref_cases.attention_cases(), ids=lambda c: c["name"])
def test_oracle_matches_torch_sdpa_golden(case, golden):
    q, k, v = ref_cases.build(case)
    out = oracle.attention(q, k, v, q_heads=case["hq"], kv_heads=case["hkv"],
                           head_dim=case["d"], causal=True, query_offset=case["off"],
                           want=("f16", "f32", "f64"))
    expected = golden[case["name"]]
    assert np.abs(out["f64"] - expected).max() <= 1e-12
    assert np.abs(out["f32"] - expected).max() <= 2e-5
    # f16 output is the f32 result rounded: at most half an ulp away.
    ulp = np.spacing(np.abs(expected).astype(np.float16)).astype(np.float64)
    assert (np.abs(f16(out["f16"]) - expected) <= 0.5 * ulp + 2e-5).all()


# ------------------------------------------------ closed forms -----------

def test_first_causal_row_is_first_value_row():
    T, hq, hkv, d = 9, 6, 2, 64
    q, k, v = rand_f16(1, (T, hq, d)), rand_f16(2, (T, hkv, d)), rand_f16(3, (T, hkv, d))
    out = oracle.attention(q, k, v, q_heads=hq, kv_heads=hkv, head_dim=d, causal=True,
                           query_offset=0, want=("f16",))["f16"]
    for h in range(hq):
        assert (out[0, h] == v[0, h // 3]).all()


def test_identical_keys_give_prefix_mean():
    T, L, hq, hkv, d = 5, 12, 4, 4, 32
    q = rand_f16(4, (T, hq, d))
    k = np.repeat(rand_f16(5, (1, hkv, d)), L, axis=0)
    v = rand_f16(6, (L, hkv, d))
    off = L - T
    out = oracle.attention(q, k, v, q_heads=hq, kv_heads=hkv, head_dim=d, causal=True,
                           query_offset=off, want=("f64", "f32"))
    vf = f16(v).astype(np.float64)
    for t in range(T):
        expected = vf[: off + t + 1].mean(axis=0)
        assert np.abs(out["f64"][t] - expected).max() < 1e-12
        assert np.abs(out["f32"][t] - expected).max() < 1e-5


def test_constant_values_and_single_key():
    T, L, hq, hkv, d = 4, 20, 2, 1, 16
    q, k = rand_f16(7, (T, hq, d)), rand_f16(8, (L, hkv, d))
    v = np.full((L, hkv, d), np.float16(0.75).view(np.uint16), dtype=np.uint16)
    out = oracle.attention(q, k, v, q_heads=hq, kv_heads=hkv, head_dim=d, causal=False,
                           want=("f16", "f64"))
    assert np.abs(out["f64"] - 0.75).max() < 1e-14
    assert (f16(out["f16"]) == 0.75).all()
    one = oracle.attention(q[:1], k[:1], rand_f16(9, (1, hkv, d)), q_heads=hq, kv_heads=hkv,
                           head_dim=d, causal=True, want=("f16",))
    assert (one["f16"][0, 0] == rand_f16(9, (1, hkv, d))[0, 0]).all()


def test_one_hot_values_expose_softmax_weights():
    L, hq, d = 16, 2, 16
    q, k = rand_f16(10, (1, hq, d), 2.0), rand_f16(11, (L, 1, d), 2.0)
    v = np.zeros((L, 1, d), dtype=np.uint16)
    v[np.arange(L), 0, np.arange(L)] = np.float16(1.0).view(np.uint16)
    out = oracle.attention(q, k, v, q_heads=hq, kv_heads=1, head_dim=d, causal=False,
                           want=("f64",))["f64"]
    scores = f16(q)[0].astype(np.float64) @ f16(k)[:, 0].astype(np.float64).T / math.sqrt(d)
    weights = np.exp(scores - scores.max(axis=1, keepdims=True))
    weights /= weights.sum(axis=1, keepdims=True)
    assert np.abs(out[0] - weights).max() < 1e-12


def test_brute_force_tiny_python_loops():
    T, L, hq, hkv, d, off = 3, 5, 4, 2, 4, 2
    q, k, v = rand_f16(12, (T, hq, d)), rand_f16(13, (L, hkv, d)), rand_f16(14, (L, hkv, d))
    out = oracle.attention(q, k, v, q_heads=hq, kv_heads=hkv, head_dim=d, causal=True,
                           query_offset=off, want=("f32", "f64"))
    qf, kf, vf = f16(q).tolist(), f16(k).tolist(), f16(v).tolist()
    for t in range(T):
        for h in range(hq):
            g = h // (hq // hkv)
            window = min(L, off + t + 1)
            s = [sum(qf[t][h][x] * kf[j][g][x] for x in range(d)) / math.sqrt(d)
                 for j in range(window)]
            m = max(s)
            p = [math.exp(x - m) for x in s]
            for x in range(d):
                want = sum(p[j] * vf[j][g][x] for j in range(window)) / sum(p)
                assert abs(out["f64"][t, h, x] - want) < 1e-13
                assert abs(out["f32"][t, h, x] - want) < 1e-5


# --------------------------------------------------- invariants ----------

def test_decode_equals_last_prefill_row_and_chunking():
    T, hq, hkv, d = 40, 8, 2, 64
    q, k, v = rand_f16(15, (T, hq, d)), rand_f16(16, (T, hkv, d)), rand_f16(17, (T, hkv, d))
    full = oracle.attention(q, k, v, q_heads=hq, kv_heads=hkv, head_dim=d, causal=True,
                            query_offset=0, want=("f16", "f32"))
    dec = oracle.attention(q[-1:], k, v, q_heads=hq, kv_heads=hkv, head_dim=d, causal=True,
                           query_offset=T - 1, want=("f16", "f32"))
    assert (dec["f32"][0] == full["f32"][-1]).all()
    P = 25
    chunk = oracle.attention(q[P:], k, v, q_heads=hq, kv_heads=hkv, head_dim=d, causal=True,
                             query_offset=P, want=("f32",))
    assert (chunk["f32"] == full["f32"][P:]).all()
    rows = oracle.attention(q, k, v, q_heads=hq, kv_heads=hkv, head_dim=d, causal=True,
                            rows=[0, 7, 39], want=("f32",))
    assert (rows["f32"] == full["f32"][[0, 7, 39]]).all()


def test_gqa_equals_repeated_mha_and_strided_views():
    T, L, hq, hkv, d = 6, 30, 8, 2, 32
    q, k, v = rand_f16(18, (T, hq, d)), rand_f16(19, (L, hkv, d)), rand_f16(20, (L, hkv, d))
    gqa = oracle.attention(q, k, v, q_heads=hq, kv_heads=hkv, head_dim=d, query_offset=L - T,
                           want=("f32",))["f32"]
    mha = oracle.attention(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), q_heads=hq,
                           kv_heads=hq, head_dim=d, query_offset=L - T, want=("f32",))["f32"]
    assert (gqa == mha).all()
    kh = workloads.head_major(k, 64)            # [Hkv, cap, D] storage
    kview = kh.transpose(1, 0, 2)[:L]           # logical [L, Hkv, D] view
    vview = workloads.head_major(v, 64).transpose(1, 0, 2)[:L]
    strided = oracle.attention(q, kview, vview, q_heads=hq, kv_heads=hkv, head_dim=d,
                               query_offset=L - T, want=("f32",))["f32"]
    assert (strided == gqa).all()


def test_masked_keys_have_no_influence_and_permutation_invariance():
    T, L, hq, hkv, d, off = 4, 50, 2, 1, 16, 20
    q, k, v = rand_f16(21, (T, hq, d)), rand_f16(22, (L, hkv, d)), rand_f16(23, (L, hkv, d))
    a = oracle.attention(q, k, v, q_heads=hq, kv_heads=hkv, head_dim=d, query_offset=off,
                         want=("f32",))["f32"]
    k2, v2 = k.copy(), v.copy()
    k2[off + T:] = rand_f16(24, k2[off + T:].shape, 5.0)
    v2[off + T:] = rand_f16(25, v2[off + T:].shape, 5.0)
    b = oracle.attention(q, k2, v2, q_heads=hq, kv_heads=hkv, head_dim=d, query_offset=off,
                         want=("f32",))["f32"]
    assert (a == b).all()
    perm = np.random.default_rng(3).permutation(L)
    nc = oracle.attention(q, k, v, q_heads=hq, kv_heads=hkv, head_dim=d, causal=False,
                          want=("f64",))["f64"]
    pc = oracle.attention(q, k[perm], v[perm], q_heads=hq, kv_heads=hkv, head_dim=d,
                          causal=False, want=("f64",))["f64"]
    assert np.abs(nc - pc).max() < 1e-13


def test_empty_window_is_nan_like_reference():
    q, k, v = rand_f16(26, (1, 2, 8)), rand_f16(27, (0, 1, 8)), rand_f16(28, (0, 1, 8))
    out = oracle.attention(q, k.reshape(0, 1, 8), v.reshape(0, 1, 8), q_heads=2, kv_heads=1,
                           head_dim=8, causal=True, want=("f32",))["f32"]
    assert np.isnan(out).all()


def test_torch_sdpa_cross_check_seeded_gqa():
    T, L, hq, hkv, d = 37, 53, 8, 2, 128
    q, k, v = (oracle.normal_f16(s, shape) for s, shape in
               ((1, (T, hq, d)), (2, (L, hkv, d)), (3, (L, hkv, d))))
    out = oracle.attention(q, k, v, q_heads=hq, kv_heads=hkv, head_dim=d, query_offset=L - T,
                           want=("f32", "f64"))
    qt = torch.from_numpy(f16(q)).double().permute(1, 0, 2)
    kt = torch.from_numpy(f16(k)).double().permute(1, 0, 2)
    vt = torch.from_numpy(f16(v)).double().permute(1, 0, 2)
    ref = torch.nn.functional.scaled_dot_product_attention(
        qt, kt, vt, is_causal=False, enable_gqa=True,
        attn_mask=torch.arange(L)[None, :] <= (L - T + torch.arange(T))[:, None])
    ref = ref.permute(1, 0, 2).numpy()
    assert np.abs(out["f64"] - ref).max() < 1e-12
    assert np.abs(out["f32"] - ref).max() < 5e-6


# ---------------------------------------------- planted mistakes ---------

def _golden_error(q, k, v, case, expected, **override):
    args = dict(q_heads=case["hq"], kv_heads=case["hkv"], head_dim=case["d"], causal=True,
                query_offset=case["off"], want=("f64",))
    args.update(override)
    return np.abs(oracle.attention(q, k, v, **args)["f64"] - expected).max()


def test_pins_catch_planted_mistakes(golden):
    case = next(c for c in ref_cases.attention_cases() if c["name"] == "prefill_d64_T33_L65")
    q, k, v = ref_cases.build(case)
    expected = golden[case["name"]]
    assert _golden_error(q, k, v, case, expected) < 1e-12
    # transposed operands: K and V swapped
    assert _golden_error(q, v, k, case, expected) > 1e-3
    # off-by-one causal window
    assert _golden_error(q, k, v, case, expected, query_offset=case["off"] + 1) > 1e-3
    # a dropped term: the last query row sees its window minus the final key
    err_drop = np.abs(oracle.attention(q[-1:], k[:-1], v[:-1], q_heads=case["hq"],
                                       kv_heads=case["hkv"], head_dim=case["d"],
                                       causal=False, want=("f64",))["f64"]
                      - expected[-1:]).max()
    assert err_drop > 1e-4
    # wrong scale: scores not divided by sqrt(D) (emulated by scaling Q)
    q_unscaled = (f16(q) * np.float32(math.sqrt(case["d"]))).astype(np.float16).view(np.uint16)
    assert _golden_error(q_unscaled, k, v, case, expected) > 1e-3
    # wrong GQA head mapping: kv head h % Hkv instead of h // G
    q_perm = q[:, [0, 2, 1, 3]]
    assert np.abs(oracle.attention(q_perm, k, v, q_heads=4, kv_heads=2, head_dim=case["d"],
                                   causal=True, query_offset=case["off"], want=("f64",))["f64"]
                  [:, [0, 2, 1, 3]] - expected).max() > 1e-3


# -------------------------------------------------- QK norm + RoPE -------

def _hf_qk_norm_rope(x_bits, weight_bits, positions, theta, eps):
    """transformers' Qwen3RMSNorm + apply_rotary_pos_emb in float64."""
    from transformers.models.qwen3 import modeling_qwen3 as m

    x = torch.from_numpy(f16(x_bits)).double()          # [T, H, D]
    w = torch.from_numpy(f16(weight_bits)).double()
    norm = m.Qwen3RMSNorm(x.shape[-1], eps=eps).double()
    with torch.no_grad():
        norm.weight.copy_(w)
        y = norm(x)
    d = x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    ang = torch.tensor(positions, dtype=torch.float64)[:, None] * inv[None, :]
    emb = torch.cat((ang, ang), dim=-1)
    cos, sin = emb.cos()[:, None, :], emb.sin()[:, None, :]
    rot, _ = m.apply_rotary_pos_emb(y.transpose(0, 1)[None], y.transpose(0, 1)[None],
                                    cos.transpose(0, 1), sin.transpose(0, 1), unsqueeze_dim=0)
    return rot[0].transpose(0, 1).numpy()


def rope_tolerance(ref: np.ndarray, positions) -> np.ndarray:
    """Error model of an f32 RMSNorm + RoPE rounded to f16, per element.

    Half an f16 ulp for the final rounding, plus f32 rounding of the rotation,
    which scales with the magnitude of the (i, i + D/2) pair rather than the
    (possibly cancelled) output, plus the f32 angle's rounding, which grows
    with the position.
    """
    half = ref.shape[-1] // 2
    pair = np.sqrt(ref[..., :half] ** 2 + ref[..., half:] ** 2)
    pair = np.concatenate((pair, pair), axis=-1)
    pos = np.asarray(positions, dtype=np.float64).reshape(-1, *([1] * (ref.ndim - 1)))
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    return 0.5 * ulp + pair * (2e-6 + 2.4e-7 * (pos + 1))


@pytest.mark.parametrize("offset", [0, 1, 37, 2000])
def test_qk_norm_rope_matches_transformers_qwen3(offset):
    T, hq, hkv, d, theta, eps = 5, 4, 2, 128, 1_000_000.0, 1e-6
    q, k = rand_f16(30, (T, hq, d)), rand_f16(31, (T, hkv, d))
    qw = (1.0 + 0.1 * np.random.default_rng(32).standard_normal(d)).astype(np.float16).view(np.uint16)
    kw = (1.0 + 0.1 * np.random.default_rng(33).standard_normal(d)).astype(np.float16).view(np.uint16)
    q_out, k_out = oracle.qk_norm_rope(q, k, qw, kw, offset=offset, theta=theta, epsilon=eps)
    pos = [offset + t for t in range(T)]
    for got, x, w in ((q_out, q, qw), (k_out, k, kw)):
        ref = _hf_qk_norm_rope(x, w, pos, theta, eps)
        assert (np.abs(f16(got) - ref) <= rope_tolerance(ref, pos)).all()


def test_qk_norm_rope_reference_case_and_rotation_invariant():
    # gpu.rs:540-576 inputs: Q = i/16 - 1, K = i/12 - 0.5, weights 0.75 + i/16, offset 1.
    f = np.float32
    q = (np.arange(32, dtype=f) / f(16.0) - f(1.0)).astype(np.float16).view(np.uint16)
    k = (np.arange(16, dtype=f) / f(12.0) - f(0.5)).astype(np.float16).view(np.uint16)
    w = (f(0.75) + np.arange(8, dtype=f) / f(16.0)).astype(np.float16).view(np.uint16)
    q_out, k_out = oracle.qk_norm_rope(q.reshape(2, 2, 8), k.reshape(2, 1, 8), w, w, offset=1,
                                       theta=10_000.0, epsilon=1e-6)
    for got, x in ((q_out, q.reshape(2, 2, 8)), (k_out, k.reshape(2, 1, 8))):
        ref = _hf_qk_norm_rope(x, w, [1, 2], 10_000.0, 1e-6)
        assert np.abs(f16(got) - ref).max() <= 2e-3
        # RoPE is a rotation of each (i, i + D/2) pair: norms are unchanged.
        xf = f16(x).astype(np.float64)
        normed = xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-6) * f16(w)
        pair_in = normed[..., :4] ** 2 + normed[..., 4:] ** 2
        gf = f16(got).astype(np.float64)
        pair_out = gf[..., :4] ** 2 + gf[..., 4:] ** 2
        assert np.abs(pair_out - pair_in).max() < 2e-2
