"""GPU parity of the attention block's neighbours through the C ABI:
rms_norm, rope and matmul (the o_proj), the unfused Q/K path of
forward_layer (crates/metal-infer-models/src/qwen3.rs:717-752) and its
captured replay. Each result is checked against the oracle (oracle/) on the
same inputs, and the reference's own test cases
(crates/metal-infer-core/tests/gpu.rs) against the expectations they state.
"""
from __future__ import annotations

import numpy as np
import pytest

import mi_attn
import oracle
from helpers import f16

pytestmark = pytest.mark.gpu

EPS_F32 = 2.0 ** -24
REFERENCE_TOLERANCE = 0.02  # gpu.rs:6


def bits(values) -> np.ndarray:
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def rand(seed, shape, scale=1.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape) * scale).astype(np.float16).view(np.uint16)


def half_spacing(values) -> np.ndarray:
    """Half the f16 spacing at each value: the most RNE rounding can move it."""
    return 0.5 * np.spacing(np.abs(np.asarray(values, dtype=np.float64)).astype(np.float16)
                            ).astype(np.float64)


def check_matmul(got_bits, x_bits, w_bits, label=""):
    """GPU f16 output vs the exact product of the f16 inputs: within RNE
    rounding plus the worst case of an f32 sum in any order (gamma_k times
    sum |x w|), and on average within a third of an f16 spacing (rounding
    alone averages a quarter), which a dropped or misplaced term breaks."""
    x = f16(x_bits).astype(np.float64)
    w = f16(w_bits).astype(np.float64)
    exact = x @ w.T
    k = x.shape[1]
    gamma = k * EPS_F32 / (1 - k * EPS_F32)
    bound = half_spacing(exact) + gamma * (np.abs(x) @ np.abs(w).T) + 1e-30
    got = f16(got_bits).astype(np.float64)
    err = np.abs(got - exact)
    assert (err <= bound).all(), f"{label}: max excess {(err - bound).max():.3e}"
    mean_ulps = float(np.mean(err / (2 * half_spacing(exact) + 1e-30)))
    assert mean_ulps <= 0.34, f"{label}: mean error {mean_ulps:.3f} f16 spacings"
    return exact


def run_matmul(ctx, x_bits, w_bits):
    x, w = ctx.tensor(np.ascontiguousarray(x_bits)), ctx.tensor(np.ascontiguousarray(w_bits))
    out = ctx.empty((x_bits.shape[0], w_bits.shape[0]))
    batch = ctx.begin_batch()
    batch.matmul(x, w, out=out)
    batch.finish()
    return ctx.download(out)


# ----------------------------------------------------------- matmul -------

def test_matmul_reference_closed_forms(ctx):
    # gpu.rs:79-87, gpu.rs:132-140
    got = run_matmul(ctx, bits([[1, 2], [3, 4]]), bits([[5, 6], [7, 8]]))
    assert f16(got).tolist() == [[17.0, 23.0], [39.0, 53.0]]
    got = run_matmul(ctx, bits([[1, 2, 3]]), bits([[4, 5, 6], [7, 8, 9]]))
    assert f16(got).tolist() == [[32.0, 50.0]]


def test_matmul_reference_matvec_cases(ctx):
    # gpu.rs:163-184 (vectorized matvec, 257 x 128)
    x = np.arange(128, dtype=np.float32) / 128.0 - 0.5
    w = ((np.arange(257 * 128) % 31).astype(np.float32) / 31.0 - 0.5).reshape(257, 128)
    got = run_matmul(ctx, bits(x[None]), bits(w))
    assert np.abs(f16(got)[0] - (w * x).sum(axis=1, dtype=np.float32)).max() <= REFERENCE_TOLERANCE
    check_matmul(got, bits(x[None]), bits(w), "257x128")
    # gpu.rs:189-221 (one row, k = 1024, n = 33)
    x = (np.arange(1024) % 41).astype(np.float32) / 41.0 - 0.5
    w = ((np.arange(33 * 1024) % 37).astype(np.float32) / 37.0 - 0.5).reshape(33, 1024)
    got = run_matmul(ctx, bits(x[None]), bits(w))
    check_matmul(got, bits(x[None]), bits(w), "33x1024")
    assert np.abs(f16(got) - f16(oracle.matmul(bits(x[None]), bits(w))[0])).max() <= REFERENCE_TOLERANCE
    # gpu.rs:224-250 (Qwen shapes, including a 65537-row vocabulary)
    for n, k in ((1024, 1024), (1024, 3072), (65_537, 256)):
        x = (np.arange(k) % 17).astype(np.float32) / 34.0 - 0.25
        w = ((np.arange(n * k) % 29).astype(np.float32) / 58.0 - 0.25).reshape(n, k)
        got = run_matmul(ctx, bits(x[None]), bits(w))
        check_matmul(got, bits(x[None]), bits(w), f"{n}x{k}")
        expected = oracle.matmul(bits(x[None]), bits(w))[1]
        assert np.abs(f16(got) - expected).max() <= REFERENCE_TOLERANCE


@pytest.mark.parametrize("m,n,k", [(32, 32, 32), (64, 96, 64), (31, 35, 37)])
def test_matmul_reference_simdgroup_shapes(ctx, m, n, k):
    # gpu.rs:110-129 inputs; the reference compares two of its kernels, here
    # the expectation is the oracle and the exact product.
    x = ((np.arange(m * k) % 19).astype(np.float32) / 19.0 - 0.5).reshape(m, k)
    w = ((np.arange(n * k) % 23).astype(np.float32) / 23.0 - 0.5).reshape(n, k)
    got = run_matmul(ctx, bits(x), bits(w))
    check_matmul(got, bits(x), bits(w), f"{m}x{n}x{k}")
    assert np.abs(f16(got) - oracle.matmul(bits(x), bits(w))[1]).max() <= REFERENCE_TOLERANCE


@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 9, 16, 128])
def test_matmul_o_proj_rows(ctx, m):
    """Qwen3-0.6B o_proj: [m, 16 * 128] x [1024, 2048]^T; up to 8 rows take
    the few-row kernel, more take the GEMM."""
    x = rand(100 + m, (m, 2048))
    w = rand(200 + m, (1024, 2048), scale=2048 ** -0.5)
    got = run_matmul(ctx, x, w)
    check_matmul(got, x, w, f"m={m}")
    ref = oracle.matmul(x, w)[1]
    assert np.abs(f16(got) - ref).max() <= 4 * half_spacing(ref).max() + 1e-3


def matmul_kernels(ctx, x_bits, w_bits):
    """Launch records of one matmul call, and its output."""
    ctx.take_kernel_profiles()
    ctx.set_kernel_profiling(True)
    try:
        got = run_matmul(ctx, x_bits, w_bits)
        names = [name for name, _ in ctx.take_kernel_profiles()]
    finally:
        ctx.set_kernel_profiling(False)
    return names, got


@pytest.mark.parametrize("m,n,k", [(9, 1024, 2048), (13, 1024, 2048), (17, 1024, 2048),
                                   (24, 1024, 2048), (31, 1024, 2048), (32, 1024, 2048),
                                   (32, 4096, 4096), (16, 16, 1024), (25, 48, 3072),
                                   (20, 5120, 8192)])
def test_matmul_skinny_rows(ctx, m, n, k):
    """9 to 32 rows (the batched-decode o_proj) take the skinny GEMM when its
    n / 16 workgroups fit the device's CUs, else the library GEMM; either way
    the result is within the f32-summation bound of the exact product, and a
    repeated call is bit-identical."""
    x = rand(300 + m, (m, k))
    w = rand(400 + n, (n, k), scale=k ** -0.5)
    names, got = matmul_kernels(ctx, x, w)
    assert names == (["skinny_gemm"] if n // 16 <= ctx.compute_units else ["gemm"]), names
    check_matmul(got, x, w, f"{m}x{n}x{k}")
    assert (run_matmul(ctx, x, w) == got).all()
    if n * k <= 1024 * 2048:
        ref = oracle.matmul(x, w)[1]
        assert np.abs(f16(got) - ref).max() <= 4 * half_spacing(ref).max() + 1e-3


def test_matmul_skinny_special_values(ctx):
    """Zeros, a row of ones against a row of ones (the sum k exactly), and
    products overflowing f16 to infinity, in rows spread over both 16-row
    blocks of the skinny GEMM."""
    m, n, k = 20, 32, 1024
    x = np.zeros((m, k), dtype=np.float32)
    w = np.zeros((n, k), dtype=np.float32)
    x[3], w[5] = 1.0, 1.0
    x[17, :4], w[30, :4] = 200.0, 200.0
    got = f16(run_matmul(ctx, bits(x), bits(w)))
    expected = np.zeros((m, n), dtype=np.float32)
    expected[3, 5] = k
    expected[3, 30] = expected[17, 5] = 800.0
    expected[17, 30] = np.inf
    assert np.array_equal(got, expected)


@pytest.mark.parametrize("pad,offset", [(64, 64), (8, 8), (64, 4)])
def test_matmul_skinny_views(ctx, pad, offset):
    """Row strides with padding keep the skinny path when rows stay 16-byte
    aligned; a view 8 bytes off alignment (offset 4) takes the library GEMM.
    Both match the exact product."""
    kernel = "gemm" if offset % 8 else "skinny_gemm"
    m, n, k = 24, 256, 1024
    x_store = rand(60 + pad + offset, (m, k + pad))
    w = rand(61, (n, k), scale=k ** -0.5)
    x_dev, w_dev = ctx.tensor(x_store), ctx.tensor(w)  # the view does not own its storage
    x_view = x_dev.view((m, k), (k + pad, 1), offset=offset)
    out = ctx.empty((m, n))
    ctx.take_kernel_profiles()
    ctx.set_kernel_profiling(True)
    try:
        batch = ctx.begin_batch()
        batch.matmul(x_view, w_dev, out=out)
        batch.finish()
        assert [name for name, _ in ctx.take_kernel_profiles()] == [kernel]
    finally:
        ctx.set_kernel_profiling(False)
    flat = x_store.reshape(-1)
    rows = np.stack([flat[offset + i * (k + pad):offset + i * (k + pad) + k] for i in range(m)])
    check_matmul(ctx.download(out), rows, w, f"view pad={pad} offset={offset}")


def test_captured_skinny_replays_match_eager(ctx):
    """The skinny GEMM recorded into a graph: every replay matches the eager
    call bit for bit."""
    m, n, k = 32, 4096, 4096
    x = ctx.tensor(rand(130, (m, k)))
    w = ctx.tensor(rand(131, (n, k), scale=k ** -0.5))
    out = ctx.empty((m, n))
    capture = ctx.begin_capture()
    capture.matmul(x, w, out=out)
    graph = capture.end_capture()
    for rep in range(3):
        ctx.upload(x, rand(140 + rep, (m, k)))
        graph.launch()
        ctx.synchronize()
        got = ctx.download(out)
        assert (got == ctx.download(ctx.matmul(x, w))).all(), f"replay {rep}"
    graph.destroy()


@pytest.mark.parametrize("m,n,k", [(1, 33, 1001), (3, 70, 7), (12, 5, 130), (1, 4096, 4096),
                                   (2, 5120, 8192)])
def test_matmul_odd_and_large_shapes(ctx, m, n, k):
    x = rand(m + n, (m, k))
    w = rand(n + k, (n, k), scale=k ** -0.5)
    check_matmul(run_matmul(ctx, x, w), x, w, f"{m}x{n}x{k}")


def test_matmul_prefill_o_proj_sampled_rows(ctx):
    """c3's o_proj, [2048, 2048] x [1024, 2048]^T, checked on 48 rows."""
    x = rand(7, (2048, 2048))
    w = rand(8, (1024, 2048), scale=2048 ** -0.5)
    got = run_matmul(ctx, x, w)
    rows = np.random.default_rng(9).choice(2048, 48, replace=False)
    check_matmul(got[rows], x[rows], w, "2048x1024x2048")


@pytest.mark.parametrize("m", [4, 40])
def test_matmul_strided_views(ctx, m):
    n, k, pad = 96, 256, 64
    x_store = rand(30 + m, (m, k + pad))
    w = rand(31, (n, k), scale=0.1)
    x_dev = ctx.tensor(x_store)
    x_view = x_dev.view((m, k), (k + pad, 1), offset=pad)
    out_store = ctx.tensor(np.zeros((m, n + 32), dtype=np.uint16))
    out_view = out_store.view((m, n), (n + 32, 1), offset=32)
    batch = ctx.begin_batch()
    batch.matmul(x_view, ctx.tensor(w), out=out_view)
    batch.finish()
    full = ctx.download(out_store)
    check_matmul(full[:, 32:], np.ascontiguousarray(x_store[:, pad:]), w, f"view m={m}")
    assert (full[:, :32] == 0).all()


def test_matmul_empty_products(ctx):
    """Skinny-range row counts (16) with an empty product: n == 0 launches
    nothing and succeeds, k == 0 writes zeros. Views of real storage, so no
    zero-byte allocation is involved."""
    x_dev = ctx.tensor(rand(90, (16, 64)))
    w_dev = ctx.tensor(rand(91, (32, 64)))
    out_dev = ctx.tensor(np.full((16, 32), 0x3C00, dtype=np.uint16))  # 1.0 everywhere
    batch = ctx.begin_batch()
    batch.matmul(x_dev, w_dev.view((0, 64), (64, 1)), out=out_dev.view((16, 0), (32, 1)))
    batch.matmul(x_dev.view((16, 0), (64, 1)), w_dev.view((32, 0), (64, 1)), out=out_dev)
    batch.finish()
    assert (ctx.download(out_dev) == 0).all()


def test_matmul_errors(ctx):
    x = ctx.tensor(rand(1, (2, 3)))
    w = ctx.tensor(rand(2, (5, 4)))
    batch = ctx.begin_batch()
    with pytest.raises(mi_attn.MiError, match="matmul inner dimensions differ: 3 and 4"):
        batch.matmul(x, w)
    with pytest.raises(mi_attn.MiError, match=r"expected matrix, got \[2, 3, 1\]"):
        batch.matmul(x.reshape((2, 3, 1)), w)
    with pytest.raises(mi_attn.MiError, match="unsupported dtype"):
        batch.matmul(ctx.empty((2, 4), dtype=mi_attn.F32), w)
    with pytest.raises(mi_attn.MiError, match=r"output must have shape \[2, 5\]"):
        batch.matmul(ctx.tensor(rand(3, (2, 4))), w, out=ctx.empty((5, 2)))
    batch.abandon()


# ---------------------------------------------------- RMSNorm / RoPE -------

def check_rms_norm(got_bits, x_bits, w_bits, eps, label=""):
    _, ref32 = oracle.rms_norm(x_bits, w_bits, epsilon=eps)
    width = x_bits.shape[-1]
    # RNE of the f32 value, plus both sides' f32 sum-of-squares error
    bound = half_spacing(ref32) + np.abs(ref32) * (width * EPS_F32 + 16 * EPS_F32) + 1e-30
    err = np.abs(f16(got_bits).astype(np.float64) - ref32)
    assert (err <= bound).all(), f"{label}: max excess {(err - bound).max():.3e}"


def test_rms_norm_reference_case(ctx):
    # gpu.rs:273-296 (simd_rms_norm_matches_cpu)
    x = ((np.arange(3 * 65) % 23).astype(np.float32) / 11.0 - 1.0).reshape(3, 65)
    w = 0.5 + np.arange(65, dtype=np.float32) / 130.0
    got = ctx.download(ctx.rms_norm(ctx.tensor(bits(x)), ctx.tensor(bits(w)), 1e-6))
    scale = 1.0 / np.sqrt((x * x).sum(axis=1, dtype=np.float32) / np.float32(65) + np.float32(1e-6))
    assert np.abs(f16(got) - x * scale[:, None] * w).max() <= REFERENCE_TOLERANCE
    check_rms_norm(got, bits(x), bits(w), 1e-6, "3x65")


@pytest.mark.parametrize("shape", [(5, 1024), (7, 16, 128), (3, 8, 64), (2, 4096), (9, 100),
                                   (1, 2, 3, 24)])
def test_rms_norm_parity(ctx, shape):
    x = rand(sum(shape), shape)
    w = (1.0 + 0.1 * np.random.default_rng(5).standard_normal(shape[-1])).astype(np.float16)
    w = w.view(np.uint16)
    got = ctx.download(ctx.rms_norm(ctx.tensor(x), ctx.tensor(w), 1e-6))
    check_rms_norm(got, x, w, 1e-6, str(shape))


def test_rms_norm_on_a_head_view_of_a_fused_projection(ctx):
    """Query heads as a [T, 16, 128] view of a [T, 32 * 128] buffer."""
    T = 6
    store = rand(40, (T, 32 * 128))
    w = rand(41, (128,), scale=0.2)
    dev = ctx.tensor(store)
    view = dev.view((T, 16, 128), (32 * 128, 128, 1))
    got = ctx.download(ctx.rms_norm(view, ctx.tensor(w), 1e-6))
    q = np.ascontiguousarray(store.reshape(T, 32, 128)[:, :16])
    check_rms_norm(got, q, w, 1e-6, "head view")


def rope_tolerance(oracle_bits, x_bits, offset):
    """The oracle and the kernel run the same uncontracted f32 steps; their
    powf / sinf / cosf may differ in the last f32 bit, which moves the result
    by at most the f32 error model of the rotation (relative to the pair's
    magnitude, growing with the position) plus one f16 spacing."""
    x = f16(x_bits).astype(np.float64)
    half = x.shape[-1] // 2
    pair = np.sqrt(x[..., :half] ** 2 + x[..., half:] ** 2)
    pair = np.concatenate((pair, pair), axis=-1)
    pos = offset + np.arange(x.shape[0], dtype=np.float64).reshape(-1, 1, 1)
    return 2 * half_spacing(f16(oracle_bits)) + pair * (2e-6 + 2.4e-7 * (pos + 1))


@pytest.mark.parametrize("T,H,D,offset,theta", [(4, 16, 128, 0, 1e6), (3, 8, 128, 2047, 1e6),
                                                (300, 8, 128, 5, 1e6), (2, 4, 64, 16384, 1e4),
                                                (5, 3, 8, 1, 1e4), (6, 70, 256, 7, 1e6)])
def test_rope_parity(ctx, T, H, D, offset, theta):
    x = rand(T * H + D, (T, H, D))
    got = ctx.download(ctx.rope(ctx.tensor(x), offset, theta))
    expected = oracle.rope(x, offset=offset, theta=theta)
    err = np.abs(f16(got).astype(np.float64) - f16(expected))
    assert (err <= rope_tolerance(expected, x, offset)).all()
    if offset == 0:
        assert (got[0] == x[0]).all()  # position 0 is the identity


def test_rope_aligned_and_unaligned_rows_agree_bit_for_bit(ctx):
    """16-byte aligned rows take the per-token kernel, others the per-thread
    kernel; both run the same f32 steps per element, so the same rows give the
    same bits through either."""
    T, H, D = 9, 12, 128
    x = rand(77, (T, H, D))
    aligned = ctx.download(ctx.rope(ctx.tensor(x), 40, 1e6))
    # The same rows 8 bytes past a 16-byte boundary: a view at offset 4 halves.
    store = np.zeros(T * H * D + 8, dtype=np.uint16)
    store[4:4 + T * H * D] = x.reshape(-1)
    shifted = ctx.tensor(store).view((T, H, D), (H * D, D, 1), offset=4)
    unaligned = ctx.download(ctx.rope(shifted, 40, 1e6))
    assert (aligned == unaligned).all()
    assert (np.abs(f16(aligned).astype(np.float64) - f16(oracle.rope(x, offset=40, theta=1e6)))
            <= rope_tolerance(oracle.rope(x, offset=40, theta=1e6), x, 40)).all()


def test_rope_on_a_key_view_and_errors(ctx):
    T = 3
    store = rand(50, (T, 24, 128))          # fused [T, Hq + 2 Hkv, D]
    dev = ctx.tensor(store)
    key_view = dev.view((T, 4, 128), (24 * 128, 128, 1), offset=16 * 128)
    got = ctx.download(ctx.rope(key_view, 9, 1e6))
    k = np.ascontiguousarray(store[:, 16:20])
    expected = oracle.rope(k, offset=9, theta=1e6)
    assert (np.abs(f16(got).astype(np.float64) - f16(expected)) <= rope_tolerance(expected, k, 9)).all()
    batch = ctx.begin_batch()
    with pytest.raises(mi_attn.MiError, match=r"RoPE expects \[tokens, heads, head_dim\]"):
        batch.rope(ctx.tensor(rand(1, (4, 8))), 0, 1e4)
    with pytest.raises(mi_attn.MiError, match="RoPE head_dim must be even"):
        batch.rope(ctx.tensor(rand(1, (2, 2, 7))), 0, 1e4)
    with pytest.raises(mi_attn.MiError, match=r"rms_norm weight must have shape \[65\]"):
        batch.rms_norm(ctx.tensor(rand(1, (2, 65))), ctx.tensor(rand(2, (64,))), 1e-6)
    batch.abandon()


# ------------------------------------------------ unfused Q/K path -------

def test_unfused_qk_path_matches_fused_kernel(ctx):
    """gpu.rs:540-576: rms_norm + rope + copy_into_cache against
    qk_norm_rope_cache on the reference's inputs."""
    q = bits((np.arange(32, dtype=np.float32) / 16.0 - 1.0).reshape(2, 2, 8))
    k = bits((np.arange(16, dtype=np.float32) / 12.0 - 0.5).reshape(2, 1, 8))
    w = bits(0.75 + np.arange(8, dtype=np.float32) / 16.0)
    qt, kt, wt = ctx.tensor(q), ctx.tensor(k), ctx.tensor(w)
    expected_cache = ctx.tensor(np.zeros((4, 1, 8), dtype=np.uint16))
    actual_cache = ctx.tensor(np.zeros((4, 1, 8), dtype=np.uint16))
    expected_q = ctx.rope(ctx.rms_norm(qt, wt, 1e-6), 1, 10_000.0)
    expected_k = ctx.rope(ctx.rms_norm(kt, wt, 1e-6), 1, 10_000.0)
    ctx.copy_into_cache(expected_k, expected_cache, 1)
    batch = ctx.begin_batch()
    actual_q = batch.qk_norm_rope_cache(qt, kt, wt, wt, actual_cache,
                                        mi_attn.QkNormRopeCacheConfig(1, 10_000.0, 1e-6))
    batch.finish()
    eq, aq = f16(ctx.download(expected_q)), f16(ctx.download(actual_q))
    ec, ac = f16(ctx.download(expected_cache)), f16(ctx.download(actual_cache))
    assert np.abs(eq - aq).max() <= REFERENCE_TOLERANCE
    assert np.abs(ec - ac).max() <= REFERENCE_TOLERANCE
    assert (ec[[0, 3]] == 0).all() and (ac[[0, 3]] == 0).all()
    oq, ok = oracle.qk_norm_rope(q, k, w, w, offset=1, theta=10_000.0, epsilon=1e-6)
    assert np.abs(aq - f16(oq)).max() <= 2e-3 and np.abs(ac[1:3] - f16(ok)).max() <= 2e-3


def _unfused_step(batch, q_in, k_in, v_in, qw, kw, wo, key, value, pos, hq, hkv, d, o_out=None):
    """forward_layer with qk_rope_cache off, one token (qwen3.rs:717-752)."""
    q = batch.rope(batch.rms_norm(q_in, qw, 1e-6), pos, 1_000_000.0)
    k = batch.rope(batch.rms_norm(k_in, kw, 1e-6), pos, 1_000_000.0)
    batch.copy_into_cache(k, key, pos)
    batch.copy_into_cache(v_in, value, pos)
    cfg = mi_attn.AttentionConfig(hq, hkv, d, True, pos)
    attn = batch.attention(q, key.prefix(pos + 1), value.prefix(pos + 1), cfg,
                           mi_attn.FLASH_DECODE)
    return attn, batch.matmul(attn.reshape((1, hq * d)), wo, out=o_out)


def test_unfused_decode_step_with_o_proj(ctx):
    hq, hkv, d, cap, pos = 16, 8, 128, 1024, 777
    cache = ctx.kv_cache(1, hkv, d, cap)
    key, value = cache.layer(0)
    k_hist, v_hist = rand(60, (pos, hkv, d)), rand(61, (pos, hkv, d))
    ctx.copy_into_cache(ctx.tensor(k_hist), key, 0)
    ctx.copy_into_cache(ctx.tensor(v_hist), value, 0)
    q_in, k_in, v_in = rand(62, (1, hq, d)), rand(63, (1, hkv, d)), rand(64, (1, hkv, d))
    qw, kw = rand(65, (d,), scale=0.3), rand(66, (d,), scale=0.3)
    wo = rand(67, (1024, hq * d), scale=(hq * d) ** -0.5)
    batch = ctx.begin_batch()
    attn, o = _unfused_step(batch, ctx.tensor(q_in), ctx.tensor(k_in), ctx.tensor(v_in),
                            ctx.tensor(qw), ctx.tensor(kw), ctx.tensor(wo), key, value, pos,
                            hq, hkv, d)
    batch.finish()
    # stage by stage against the oracle
    q_rot = oracle.rope(oracle.rms_norm(q_in, qw, epsilon=1e-6)[0], offset=pos, theta=1e6)
    k_rot = oracle.rope(oracle.rms_norm(k_in, kw, epsilon=1e-6)[0], offset=pos, theta=1e6)
    k_all = ctx.download(key.prefix(pos + 1))
    assert (k_all[:pos] == k_hist).all()
    assert np.abs(f16(k_all[pos]) - f16(k_rot[0])).max() <= 2e-3
    assert (ctx.download(value.prefix(pos + 1))[pos] == v_in[0]).all()
    ref = oracle.attention(q_rot, k_all, ctx.download(value.prefix(pos + 1)), q_heads=hq,
                           kv_heads=hkv, head_dim=d, causal=True, query_offset=pos,
                           want=("f32",))["f32"]
    attn_bits = ctx.download(attn)
    assert np.abs(f16(attn_bits) - ref).max() <= 2e-3
    check_matmul(ctx.download(o), attn_bits.reshape(1, hq * d), wo, "o_proj")
    cache.close()


def test_captured_unfused_decode_step_replays_match_eager(ctx):
    hq, hkv, d, cap, pos = 16, 8, 128, 1024, 500
    cache = ctx.kv_cache(1, hkv, d, cap)
    key, value = cache.layer(0)
    ctx.copy_into_cache(ctx.tensor(rand(70, (pos, hkv, d))), key, 0)
    ctx.copy_into_cache(ctx.tensor(rand(71, (pos, hkv, d))), value, 0)
    qw, kw = ctx.tensor(rand(72, (d,), scale=0.3)), ctx.tensor(rand(73, (d,), scale=0.3))
    wo = ctx.tensor(rand(74, (1024, hq * d), scale=(hq * d) ** -0.5))
    q_in, k_in, v_in = ctx.empty((1, hq, d)), ctx.empty((1, hkv, d)), ctx.empty((1, hkv, d))
    o_graph = ctx.empty((1, 1024))
    capture = ctx.begin_capture()
    _unfused_step(capture, q_in, k_in, v_in, qw, kw, wo, key, value, pos, hq, hkv, d,
                  o_out=o_graph)
    graph = capture.end_capture()
    for rep in range(3):
        ctx.upload(q_in, rand(80 + rep, (1, hq, d)))
        ctx.upload(k_in, rand(90 + rep, (1, hkv, d)))
        ctx.upload(v_in, rand(100 + rep, (1, hkv, d)))
        graph.launch()
        ctx.synchronize()
        got = ctx.download(o_graph)
        batch = ctx.begin_batch()
        _, o_eager = _unfused_step(batch, q_in, k_in, v_in, qw, kw, wo, key, value, pos,
                                   hq, hkv, d)
        batch.finish()
        assert (got == ctx.download(o_eager)).all(), f"replay {rep}"
    graph.destroy()
    cache.close()


def test_captured_gemm_replays_match_eager(ctx):
    """A prefill-sized o_proj (hipBLASLt) recorded into a graph."""
    m, n, k = 64, 1024, 2048
    x = ctx.tensor(rand(110, (m, k)))
    w = ctx.tensor(rand(111, (n, k), scale=k ** -0.5))
    out = ctx.empty((m, n))
    capture = ctx.begin_capture()
    capture.matmul(x, w, out=out)
    graph = capture.end_capture()
    for rep in range(3):
        ctx.upload(x, rand(120 + rep, (m, k)))
        graph.launch()
        ctx.synchronize()
        got = ctx.download(out)
        assert (got == ctx.download(ctx.matmul(x, w))).all(), f"replay {rep}"
    graph.destroy()
