"""CPU tests that pin the oracle's RMSNorm, RoPE and matmul (the attention
block's neighbours) before they judge the GPU.

Checks share no code with the oracle: numpy float64 products, transformers'
Qwen3 RMSNorm and rotary embedding, the reference's own test cases with the
closed-form expectations they state, invariants, and the fused Q/K kernel's
restatement. A final group plants plausible mistakes and shows the pins
catch them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from helpers import f16

EPS_F32 = 2.0 ** -24
# crates/metal-infer-core/tests/gpu.rs:6
REFERENCE_TOLERANCE = 0.02


def bits(values) -> np.ndarray:
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def rand_f16(seed, shape, scale=1.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape) * scale).astype(np.float16).view(np.uint16)


def matmul_bound(x_bits, w_bits) -> np.ndarray:
    """Worst-case error of any f32 summation order of the k products (each
    exact in f32): gamma_k * sum |x * w| per output."""
    k = x_bits.shape[1]
    gamma = k * EPS_F32 / (1 - k * EPS_F32)
    return gamma * (np.abs(f16(x_bits)).astype(np.float64) @ np.abs(f16(w_bits)).astype(np.float64).T)


def exact_matmul(x_bits, w_bits) -> np.ndarray:
    return f16(x_bits).astype(np.float64) @ f16(w_bits).astype(np.float64).T


# ----------------------------------------------------------- matmul -------

def test_matmul_reference_closed_forms():
    # gpu.rs:79-87 and gpu.rs:132-140
    out, out32 = oracle.matmul(bits([[1, 2], [3, 4]]), bits([[5, 6], [7, 8]]))
    assert out32.tolist() == [[17.0, 23.0], [39.0, 53.0]]
    assert f16(out).tolist() == [[17.0, 23.0], [39.0, 53.0]]
    _, out32 = oracle.matmul(bits([[1, 2, 3]]), bits([[4, 5, 6], [7, 8, 9]]))
    assert out32.tolist() == [[32.0, 50.0]]


def test_matmul_reference_vectorized_matvec_case():
    # gpu.rs:163-184: expectation in f32 from the unrounded formula values.
    x = np.arange(128, dtype=np.float32) / 128.0 - 0.5
    w = (np.arange(257 * 128) % 31).astype(np.float32).reshape(257, 128) / 31.0 - 0.5
    expected = (w * x).sum(axis=1, dtype=np.float32)
    out, _ = oracle.matmul(bits(x[None]), bits(w))
    assert np.abs(f16(out)[0] - expected).max() <= REFERENCE_TOLERANCE


@pytest.mark.parametrize("m,n,k", [(32, 32, 32), (64, 96, 64), (31, 35, 37), (17, 29, 33),
                                   (3, 1024, 2048), (2, 65, 4096)])
def test_matmul_matches_float64_within_summation_bound(m, n, k):
    x, w = rand_f16(m * 7 + k, (m, k)), rand_f16(n * 11 + k, (n, k))
    out, out32 = oracle.matmul(x, w)
    ref = exact_matmul(x, w)
    assert (np.abs(out32 - ref) <= matmul_bound(x, w) + 1e-30).all()
    # f16 output is the RNE rounding of the f32 sum
    assert (out == out32.astype(np.float16).view(np.uint16)).all()


def test_matmul_rows_are_independent_and_thread_count_free():
    x, w = rand_f16(1, (9, 300)), rand_f16(2, (40, 300))
    full, full32 = oracle.matmul(x, w, threads=1)
    part, part32 = oracle.matmul(x[[2, 7]], w, threads=4)
    assert (full[[2, 7]] == part).all() and (full32[[2, 7]] == part32).all()
    again, _ = oracle.matmul(x, w, threads=8)
    assert (again == full).all()


# ---------------------------------------------------------- RMSNorm -------

def _hf_rms_norm(x_bits, w_bits, eps):
    from transformers.models.qwen3 import modeling_qwen3 as m

    x = torch.from_numpy(f16(x_bits)).double()
    norm = m.Qwen3RMSNorm(x.shape[-1], eps=eps).double()
    with torch.no_grad():
        norm.weight.copy_(torch.from_numpy(f16(w_bits)).double())
        return norm(x).numpy()


def rms_bound(ref: np.ndarray, width: int) -> np.ndarray:
    """f32 error of the oracle's RMSNorm: the sequential sum of squares
    (gamma_width relative), halved by the square root, plus a few roundings
    of the scale and the two products."""
    return np.abs(ref) * (0.5 * width * EPS_F32 + 8 * EPS_F32) + 1e-30


@pytest.mark.parametrize("shape", [(3, 65), (4, 1024), (2, 16, 128), (5, 8, 64), (1, 4096)])
def test_rms_norm_matches_transformers_qwen3(shape):
    x = rand_f16(sum(shape), shape)
    w = (1.0 + 0.1 * np.random.default_rng(7).standard_normal(shape[-1])).astype(np.float16)
    w = w.view(np.uint16)
    out, out32 = oracle.rms_norm(x, w, epsilon=1e-6)
    ref = _hf_rms_norm(x, w, 1e-6)
    assert (np.abs(out32 - ref) <= rms_bound(ref, shape[-1])).all()
    assert (out == out32.astype(np.float16).view(np.uint16)).all()


def test_rms_norm_reference_case_and_closed_forms():
    # gpu.rs:273-296 (simd_rms_norm_matches_cpu): expectation in f32.
    x = ((np.arange(3 * 65) % 23).astype(np.float32) / 11.0 - 1.0).reshape(3, 65)
    w = 0.5 + np.arange(65, dtype=np.float32) / 130.0
    scale = 1.0 / np.sqrt((x * x).sum(axis=1, dtype=np.float32) / np.float32(65) + np.float32(1e-6))
    expected = x * scale[:, None] * w
    out, _ = oracle.rms_norm(bits(x), bits(w), epsilon=1e-6)
    assert np.abs(f16(out) - expected).max() <= REFERENCE_TOLERANCE
    # a constant row c: out = c / sqrt(c^2 + eps) * w
    c = np.float32(0.75)
    _, out32 = oracle.rms_norm(bits(np.full((1, 64), c)), bits(np.ones(64)), epsilon=1e-3)
    assert np.allclose(out32, c / np.sqrt(c * c + 1e-3), rtol=1e-6)
    # a zero row stays zero
    out, _ = oracle.rms_norm(bits(np.zeros((1, 16))), bits(np.ones(16)), epsilon=1e-6)
    assert (f16(out) == 0).all()


# ------------------------------------------------------------- RoPE -------

def _hf_rope(x_bits, positions, theta):
    from transformers.models.qwen3 import modeling_qwen3 as m

    x = torch.from_numpy(f16(x_bits)).double()              # [T, H, D]
    d = x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    ang = torch.tensor(positions, dtype=torch.float64)[:, None] * inv[None, :]
    emb = torch.cat((ang, ang), dim=-1)
    cos, sin = emb.cos()[:, None, :], emb.sin()[:, None, :]
    xt = x.transpose(0, 1)[None]
    rot, _ = m.apply_rotary_pos_emb(xt, xt, cos.transpose(0, 1), sin.transpose(0, 1),
                                    unsqueeze_dim=0)
    return rot[0].transpose(0, 1).numpy()


def rope_bound(ref: np.ndarray, x_bits, positions) -> np.ndarray:
    """Half an f16 ulp for the final rounding, plus f32 rounding of the
    rotation (relative to the pair's magnitude) and of the f32 angle, which
    grows with the position."""
    x = f16(x_bits).astype(np.float64)
    half = x.shape[-1] // 2
    pair = np.sqrt(x[..., :half] ** 2 + x[..., half:] ** 2)
    pair = np.concatenate((pair, pair), axis=-1)
    pos = np.asarray(positions, dtype=np.float64).reshape(-1, 1, 1)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    return 0.5 * ulp + pair * (2e-6 + 2.4e-7 * (pos + 1))


@pytest.mark.parametrize("offset,theta,d", [(0, 10_000.0, 8), (1, 10_000.0, 128),
                                            (2047, 1_000_000.0, 128), (16384, 1_000_000.0, 64)])
def test_rope_matches_transformers(offset, theta, d):
    x = rand_f16(offset + d, (6, 3, d))
    out = oracle.rope(x, offset=offset, theta=theta)
    positions = [offset + t for t in range(6)]
    ref = _hf_rope(x, positions, theta)
    assert (np.abs(f16(out) - ref) <= rope_bound(ref, x, positions)).all()


def test_rope_identity_at_position_zero_and_pair_norms():
    x = rand_f16(3, (1, 4, 128))
    assert (oracle.rope(x, offset=0, theta=1e6) == x).all()
    y = rand_f16(4, (5, 2, 64))
    out = f16(oracle.rope(y, offset=100, theta=1e4)).astype(np.float64)
    yf = f16(y).astype(np.float64)
    norm_in = yf[..., :32] ** 2 + yf[..., 32:] ** 2
    norm_out = out[..., :32] ** 2 + out[..., 32:] ** 2
    assert np.abs(norm_out - norm_in).max() < 2e-2


def test_unfused_qk_path_matches_fused_restatement():
    """gpu.rs:540-576 on the oracle: rms_norm then rope equals the fused
    qk_norm_rope_cache, up to the f16 rounding between the two steps."""
    q = bits((np.arange(32, dtype=np.float32) / 16.0 - 1.0).reshape(2, 2, 8))
    k = bits((np.arange(16, dtype=np.float32) / 12.0 - 0.5).reshape(2, 1, 8))
    w = bits(0.75 + np.arange(8, dtype=np.float32) / 16.0)
    fused_q, fused_k = oracle.qk_norm_rope(q, k, w, w, offset=1, theta=10_000.0, epsilon=1e-6)
    unfused_q = oracle.rope(oracle.rms_norm(q, w, epsilon=1e-6)[0], offset=1, theta=10_000.0)
    unfused_k = oracle.rope(oracle.rms_norm(k, w, epsilon=1e-6)[0], offset=1, theta=10_000.0)
    for a, b in ((fused_q, unfused_q), (fused_k, unfused_k)):
        assert np.abs(f16(a) - f16(b)).max() <= REFERENCE_TOLERANCE
    # seeded, Qwen3 head size: the unfused path rounds the normalised pair
    # to f16 before rotating it (relative error 2^-11 of the pair's
    # magnitude), and each path rounds its output once.
    q = rand_f16(5, (4, 16, 128))
    k = rand_f16(6, (4, 8, 128))
    w = (1.0 + 0.1 * np.random.default_rng(8).standard_normal(128)).astype(np.float16).view(np.uint16)
    fused_q, _ = oracle.qk_norm_rope(q, k, w, w, offset=37, theta=1e6, epsilon=1e-6)
    unfused_q = oracle.rope(oracle.rms_norm(q, w, epsilon=1e-6)[0], offset=37, theta=1e6)
    a = f16(fused_q).astype(np.float64)
    pair = np.sqrt(a[..., :64] ** 2 + a[..., 64:] ** 2)
    pair = np.concatenate((pair, pair), axis=-1)
    ulp = np.spacing(np.abs(a).astype(np.float16)).astype(np.float64)
    assert (np.abs(a - f16(unfused_q)) <= ulp + 2.0 ** -11 * pair * 1.01).all()


# ------------------------------------------------- planted mistakes -------

def test_pins_catch_planted_mistakes():
    # the pins accept the oracle itself on the planted cases' inputs
    x = rand_f16(24, (3, 65))
    _, out32 = oracle.rms_norm(x, bits(np.ones(65)), epsilon=0.1)
    ref = _hf_rms_norm(x, bits(np.ones(65)), 0.1)
    assert (np.abs(out32 - ref) <= rms_bound(ref, 65)).all()
    # matmul: the weight read transposed ([k, n] instead of [n, k])
    x, w = rand_f16(20, (4, 48)), rand_f16(21, (48, 48))
    wrong = exact_matmul(x, w.T.copy())
    assert not (np.abs(wrong - exact_matmul(x, w)) <= matmul_bound(x, w)).all()
    # matmul: a dropped last term of the sum
    x, w = rand_f16(22, (4, 64)), rand_f16(23, (32, 64))
    dropped = exact_matmul(x[:, :-1], w[:, :-1])
    assert not (np.abs(dropped - exact_matmul(x, w)) <= matmul_bound(x, w)).all()
    # RMSNorm: mean over width - 1, or epsilon outside the square root
    x = rand_f16(24, (3, 65))
    w = bits(np.ones(65))
    ref = _hf_rms_norm(x, w, 0.1)
    xf = f16(x).astype(np.float64)
    for wrong in (xf / np.sqrt((xf ** 2).sum(-1, keepdims=True) / 64 + 0.1),
                  xf / (np.sqrt((xf ** 2).mean(-1, keepdims=True)) + 0.1)):
        assert not (np.abs(wrong - ref) <= rms_bound(ref, 65)).all()
    # RoPE: rotation sign flipped, or positions without the offset
    x = rand_f16(25, (3, 2, 16))
    positions = [5, 6, 7]
    ref = _hf_rope(x, positions, 1e4)
    flipped = _hf_rope(x, [-p for p in positions], 1e4)
    no_offset = _hf_rope(x, [0, 1, 2], 1e4)
    for wrong in (flipped, no_offset):
        assert not (np.abs(wrong - ref) <= rope_bound(ref, x, positions)).all()
