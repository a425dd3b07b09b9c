"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against something other than its own
formula: a library routine (numpy float64 matmul, scipy's normal CDF /
logistic, torch's bf16 cast and layer_norm), brute force on tiny inputs,
closed forms and invariants chosen so that a dropped term, a swapped half or
a transposed operand fails.  Where the reference's own tests hold vectors for
this path, they are used (GeGLU: src/archs/modernbert.rs:746-757; SwiGLU
generator: src/archs/qwen35_text.rs:1097-1104).
"""
import itertools
import math

import numpy as np
import pytest
import scipy.special
import scipy.stats


def _rel_fro(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


# ------------------------------------------------------------------ GEMM ---

@pytest.mark.parametrize("M,N,K", [(1, 1, 8), (3, 5, 7), (17, 48, 64), (64, 300, 776),
                                   (333, 129, 1000), (130, 67, 257)])
def test_linear_f32_matches_numpy_f64(orc, M, N, K):
    x = orc.fill_normal((M, K), 11 + M)
    w = orc.fill_normal((N, K), 13 + N, 0.02)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    y = orc.linear_f32(x, w)
    assert y.shape == (M, N) and y.dtype == np.float32
    assert _rel_fro(y, ref) < 1e-6
    y64 = orc.linear_f64(x, w)
    assert np.abs(y64 - ref).max() <= 1e-12 * max(1.0, np.abs(ref).max()) * K


def test_linear_brute_force_tiny(orc):
    x = np.array([[1.0, 2.0, -3.0], [0.5, 0.0, 4.0]], np.float32)
    w = np.array([[1.0, 0.0, 0.0], [0.0, 1.0, 0.0], [0.0, 0.0, 1.0], [1.0, -1.0, 2.0]], np.float32)
    b = np.array([0.0, 1.0, -1.0, 0.5], np.float32)
    expect = [[sum(x[m][k] * w[n][k] for k in range(3)) + b[n] for n in range(4)] for m in range(2)]
    np.testing.assert_allclose(orc.linear_f32(x, w, b), expect, rtol=0, atol=1e-6)
    np.testing.assert_allclose(orc.linear_f64(x, w, b), expect, rtol=0, atol=1e-12)


def test_linear_weight_is_out_by_in(orc):
    """Weight [out, in]: a non-square identity-like weight must select input
    columns (a transposed operand would fail the shape or the values)."""
    x = orc.fill_normal((9, 16), 3)
    w = np.zeros((4, 16), np.float32)
    for n, k in enumerate((0, 5, 7, 15)):
        w[n, k] = 1.0
    np.testing.assert_array_equal(orc.linear_f32(x, w), x[:, [0, 5, 7, 15]])


def test_linear_closed_forms_and_invariants(orc):
    M, N, K = 40, 24, 96
    x = orc.fill_normal((M, K), 5)
    w = orc.fill_normal((N, K), 6, 0.05)
    # Rank one: x = u v^T -> y = u (W v)^T.
    u = orc.fill_normal((M, 1), 7)
    v = orc.fill_normal((1, K), 8)
    y = orc.linear_f32(u @ v, w)
    np.testing.assert_allclose(y, u @ (w @ v.T).T, rtol=1e-4, atol=1e-5)
    # Linearity in x.
    x2 = orc.fill_normal((M, K), 9)
    np.testing.assert_allclose(orc.linear_f32(2 * x - x2, w),
                               2 * orc.linear_f32(x, w) - orc.linear_f32(x2, w), rtol=1e-4, atol=1e-5)
    # Row independence: permuting tokens permutes outputs exactly.
    perm = np.random.default_rng(0).permutation(M)
    np.testing.assert_array_equal(orc.linear_f32(x[perm], w), orc.linear_f32(x, w)[perm])
    # K-split additivity.
    y_split = orc.linear_f32(x[:, :40], w[:, :40]) + orc.linear_f32(x[:, 40:], w[:, 40:])
    np.testing.assert_allclose(y_split, orc.linear_f32(x, w), rtol=1e-5, atol=1e-5)
    # Bias adds per output feature.
    b = orc.fill_normal((N,), 10)
    np.testing.assert_allclose(orc.linear_f32(x, w, b), orc.linear_f32(x, w) + b, rtol=0, atol=1e-6)


def test_linear_flattens_leading_dims(orc):
    x = orc.fill_normal((2, 3, 32), 1)
    w = orc.fill_normal((8, 32), 2)
    y = orc.linear_f32(x, w)
    assert y.shape == (2, 3, 8)
    np.testing.assert_array_equal(y.reshape(6, 8), orc.linear_f32(x.reshape(6, 32), w))


# ----------------------------------------------------------- activations ---

# The 16 values of the reference's fused GeGLU test (src/archs/modernbert.rs:746-757).
GEGLU_VALUES = [-4.0, -1.5, -0.25, 0.0, 0.5, 1.25, 3.0, 5.0, 2.0, -0.75, 0.125, -3.5, 1.0, 0.5,
                -2.0, 4.5]


def test_gelu_erf_against_normal_cdf(orc):
    v = np.linspace(-8, 8, 4001).astype(np.float32)
    expect = v.astype(np.float64) * scipy.stats.norm.cdf(v.astype(np.float64))
    np.testing.assert_allclose(orc.gelu_erf(v), expect, rtol=2e-7, atol=1e-7)
    # Special values and the odd-part identity gelu(v) - gelu(-v) = v.
    assert orc.lib().orc_gelu_erf(0.0) == 0.0
    assert abs(orc.lib().orc_gelu_erf(1.0) - 0.8413447460685429) < 1e-7
    g = orc.gelu_erf(v) - orc.gelu_erf(-v)
    np.testing.assert_allclose(g, v, rtol=1e-6, atol=1e-6)


def test_gelu_tanh_against_torch_and_closed_forms(orc):
    """The tanh-approximate GELU (candle's gelu; the vision tower's fc1)
    against torch's gelu(approximate="tanh") in float64, and what the formula
    fixes: 0 at 0, the odd-part identity gelu(v) - gelu(-v) = v (tanh is
    odd), v itself far right, and a gap of ~1e-3 to the exact GELU near 1
    (so the erf form in its place fails)."""
    torch = pytest.importorskip("torch")
    v = np.linspace(-8, 8, 4001).astype(np.float32)
    expect = torch.nn.functional.gelu(torch.from_numpy(v.astype(np.float64)), approximate="tanh").numpy()
    np.testing.assert_allclose(orc.gelu_tanh(v), expect, rtol=2e-7, atol=1e-7)
    # far left the oracle keeps full relative precision (torch's 1 + tanh
    # form loses it): against v sigmoid(2y) in float64 (no cancellation)
    vl = np.linspace(-9, -4, 501).astype(np.float32)
    vd = vl.astype(np.float64)
    yl = np.sqrt(2 / np.pi) * (vd + 0.044715 * vd ** 3)
    np.testing.assert_allclose(orc.gelu_tanh(vl), vd * scipy.special.expit(2 * yl), rtol=1e-6)
    assert orc.gelu_tanh(np.zeros(1))[0] == 0.0
    np.testing.assert_allclose(orc.gelu_tanh(v) - orc.gelu_tanh(-v), v, rtol=1e-6, atol=1e-6)
    assert orc.gelu_tanh(np.array([12.0]))[0] == np.float32(12.0)
    d = abs(float(orc.gelu_tanh(np.array([1.5]))[0]) - float(orc.gelu_erf(np.array([1.5]))[0]))
    assert 1e-4 < d < 1e-2


def test_geglu_reference_vector(orc):
    """Reference input [2, 8] -> [2, 4]; first half is the gated (gelu) half."""
    inp = np.array(GEGLU_VALUES, np.float32).reshape(2, 8)
    out = orc.geglu(inp)
    a, b = inp[:, :4].astype(np.float64), inp[:, 4:].astype(np.float64)
    expect = a * scipy.stats.norm.cdf(a) * b
    assert out.shape == (2, 4)
    # f32 tolerance of the reference test (src/archs/modernbert.rs:758).
    assert np.abs(out - expect).max() <= 1e-5
    swapped = b * scipy.stats.norm.cdf(b) * a
    assert np.abs(out - swapped).max() > 1e-2


def test_silu_and_swiglu_reference_generator(orc):
    """Generator of src/archs/qwen35_text.rs:1097-1104: g = ((i*97 % 1601) - 800)/73,
    up = -0.5 g + 0.25, over [7, 4096]."""
    i = np.arange(4096 * 7)
    g = (((i * 97) % 1601).astype(np.float32) - 800.0) / 73.0
    g = g.reshape(7, 4096)
    up = (-0.5 * g + 0.25).astype(np.float32)
    out = orc.swiglu(g, up)
    g64 = g.astype(np.float64)
    expect = g64 * scipy.special.expit(g64) * up.astype(np.float64)
    assert np.abs(out - expect).max() <= 1e-5
    s = orc.silu(g) - orc.silu(-g)  # silu(v) - silu(-v) = v
    np.testing.assert_allclose(s, g, rtol=1e-6, atol=1e-5)


def test_rms_norm_against_torch_and_closed_form(orc):
    """Qwen3.5 RMSNorm(1 + w) (src/archs/qwen35_text.rs:178-203) against
    torch's rms_norm in float64 with weight 1 + w, and a constant row c,
    whose output is c (1 + w) / sqrt(c^2 + eps)."""
    torch = pytest.importorskip("torch")
    x = orc.fill_normal((37, 512), 71) * 3.0 + 0.5
    w = orc.fill_normal((512,), 72, 0.2)
    expect = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (512,),
                                          weight=1.0 + torch.from_numpy(w).double(), eps=1e-6).numpy()
    np.testing.assert_allclose(orc.rms_norm(x, w, 1e-6), expect, rtol=2e-6, atol=2e-6)
    c = np.full((1, 64), -2.5, np.float32)
    w2 = np.linspace(-0.5, 0.5, 64).astype(np.float32)
    np.testing.assert_allclose(orc.rms_norm(c, w2, 1e-6)[0], -2.5 * (1 + w2) / np.sqrt(6.25 + 1e-6),
                               rtol=1e-6)


def test_layer_norm_bf16_rounding_sequence(orc):
    """ModernBERT's bf16 LayerNorm: normalised value cast to bf16, times the
    weight, rounded (candle-nn LayerNorm on a bf16 input).  Pinned by its
    invariants: every output is a bf16 value; with weight 1 it equals the
    rounded f32 norm; it is invariant to a per-row shift and a positive
    per-row scale of the input (up to the eps term); it is torch's float64
    layer_norm within bf16 rounding."""
    torch = pytest.importorskip("torch")
    x = orc.round_bf16(orc.fill_normal((20, 768), 73) * 2.0 + 1.0)
    g = orc.round_bf16(1.0 + orc.fill_normal((768,), 74, 0.1))
    y = orc.layer_norm_bf16(x, g, 1e-5)
    np.testing.assert_array_equal(y, orc.round_bf16(y))
    np.testing.assert_array_equal(orc.layer_norm_bf16(x, np.ones(768, np.float32), 1e-5),
                                  orc.round_bf16(orc.layer_norm(x, np.ones(768, np.float32), None, 1e-5)))
    y2 = orc.layer_norm_bf16(x * 4.0 + 3.0, g, 1e-5)
    assert np.abs(y2 - y).max() <= 4 * 2.0 ** -8 * np.abs(y).max()
    t = torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (768,),
                                       weight=torch.from_numpy(g).double(), eps=1e-5).numpy()
    assert np.abs(y - t).max() <= 2 * 2.0 ** -8 * np.abs(t).max()


def _conv_ref_gen():
    """The reference's own conv test inputs (src/archs/qwen35_text.rs:1266-1284):
    batch 2, length 7, channels 31, kernel 4."""
    b, L, C, k = 2, 7, 31, 4
    p = (((np.arange(b * L * C) * 17) % 41) - 20).astype(np.float32) * 0.04
    w = (((np.arange(C * k) * 11) % 23) - 11).astype(np.float32) * 0.02
    return p.reshape(b * L, C), w.reshape(C, k), np.tile(np.arange(L, dtype=np.int32), b), (b, L, C, k)


def test_conv_silu_f32_against_padded_loop_and_torch(orc):
    """DeltaNet causal conv + SiLU (src/archs/qwen35_text.rs:632-650), f32:
    a float64 restatement of the reference's padded-rectangle form
    (pad_with_zeros, then tap-by-tap accumulation), and torch's depthwise
    conv1d with left padding, on the reference's own test generator."""
    torch = pytest.importorskip("torch")
    p, w, pos, (b, L, C, k) = _conv_ref_gen()
    got = orc.conv_silu(p, w, pos, bf16=False)
    pr = p.reshape(b, L, C).astype(np.float64)
    padded = np.concatenate([np.zeros((b, k - 1, C)), pr], axis=1)
    mixed = np.zeros((b, L, C))
    for tap in range(k):
        mixed += padded[:, tap:tap + L, :] * w[:, tap].astype(np.float64)[None, None, :]
    ref = (mixed / (1 + np.exp(-mixed))).reshape(b * L, C)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-7)
    t = torch.nn.functional.conv1d(torch.from_numpy(pr).permute(0, 2, 1), torch.from_numpy(w).double()[:, None, :],
                                   padding=k - 1, groups=C)[:, :, :L]
    t = torch.nn.functional.silu(t).permute(0, 2, 1).reshape(b * L, C).numpy()
    np.testing.assert_allclose(got, t, rtol=1e-5, atol=1e-7)


def test_conv_silu_bf16_against_torch_bf16_ops(orc):
    """The bf16 path follows the reference's bf16 tensor arithmetic: each
    product and partial sum rounded (candle bf16 ops; the CUDA kernel's
    T(product) and T(fadd)).  Restated independently with torch bf16 tensor
    ops; SiLU in f32 then rounded.  At most 1 bf16 ulp apart (exp's last
    bit), nearly all bit-equal."""
    torch = pytest.importorskip("torch")
    p, w, pos, (b, L, C, k) = _conv_ref_gen()
    p, w = orc.round_bf16(p), orc.round_bf16(w)
    got = orc.conv_silu(p, w, pos, bf16=True)
    pt = torch.from_numpy(p.reshape(b, L, C)).to(torch.bfloat16)
    padded = torch.cat([torch.zeros(b, k - 1, C, dtype=torch.bfloat16), pt], 1)
    mixed = torch.zeros(b, L, C, dtype=torch.bfloat16)
    wt = torch.from_numpy(w).to(torch.bfloat16)
    for tap in range(k):
        mixed = mixed + padded[:, tap:tap + L, :] * wt[:, tap].reshape(1, 1, C)
    ref = torch.nn.functional.silu(mixed.float()).to(torch.bfloat16).float().reshape(b * L, C).numpy()
    diff = np.abs(got - ref)
    assert (diff <= 2.0 ** -8 * np.abs(ref) + 1e-30).all()
    assert (diff == 0).mean() > 0.99


def test_conv_tap_rounding_gap(orc):
    """The GPU conv accumulates its four taps in f32 and rounds once; the
    reference rounds every product and partial sum to bf16
    (src/kernels/qwen35.cu:18-24).  On the same bf16 inputs (unit-normal
    projection, conv weights N(0, 0.25), ragged sequences) the two differ by
    ~4.2e-3 relative Frobenius and ~1e-2 max-abs/max, which is the whole of
    the GPU in_proj+conv error against the reference chain; against the exact
    f64 conv, the single rounding is the closer of the two."""
    rng = np.random.default_rng(0)
    M, C = 4096, 512
    p = orc.round_bf16(rng.standard_normal((M, C)).astype(np.float32))
    w = orc.round_bf16((rng.standard_normal((C, 4)) * 0.5).astype(np.float32))
    pos = np.concatenate([np.arange(n) for n in (1000, 900, 1200, 996)]).astype(np.int32)
    ref = orc.conv_silu(p, w, pos, bf16=True)
    once = orc.round_bf16(orc.conv_silu(p, w, pos, bf16=False))
    d = once - ref
    rel = np.linalg.norm(d) / np.linalg.norm(ref)
    assert 2e-3 < rel < 6e-3, rel
    assert np.abs(d).max() <= 1.5e-2 * np.abs(ref).max()
    exact = np.zeros((M, C))
    for tap in range(4):
        back = 3 - tap
        shifted = np.zeros((M, C))
        shifted[back:] = p[:M - back]
        exact += np.where((pos >= back)[:, None], shifted, 0.0) * w[:, tap].astype(np.float64)[None, :]
    exact = exact / (1 + np.exp(-exact))
    err_ref = np.linalg.norm(ref - exact) / np.linalg.norm(exact)
    err_once = np.linalg.norm(once - exact) / np.linalg.norm(exact)
    assert err_once < 0.6 * err_ref, (err_once, err_ref)


def test_conv_silu_closed_forms(orc):
    """Identity tap: weight 1 on the newest tap gives silu(p); an impulse
    at one row spreads to the next three rows of its sequence only, with the
    taps reversed; a sequence start cuts the history."""
    C = 8
    p = orc.round_bf16(orc.fill_normal((10, C), 81))
    pos = np.arange(10, dtype=np.int32)
    w = np.zeros((C, 4), np.float32)
    w[:, 3] = 1.0
    np.testing.assert_array_equal(orc.conv_silu(p, w, pos), orc.round_bf16(p / (1 + np.exp(-p.astype(np.float64)))))
    imp = np.zeros((10, C), np.float32)
    imp[4] = 1.0
    w2 = np.tile(np.array([0.5, 0.25, -0.75, 2.0], np.float32), (C, 1))
    pre = orc.conv_silu(imp, w2, pos, bf16=False)
    silu = lambda v: v / (1 + np.exp(-v))
    for r, tap in ((4, 3), (5, 2), (6, 1), (7, 0)):
        np.testing.assert_allclose(pre[r], silu(w2[0, tap]) * np.ones(C), rtol=1e-6)
    assert np.all(pre[[0, 1, 2, 3, 8, 9]] == 0)
    pos2 = np.array([0, 1, 2, 3, 4, 0, 1, 2, 3, 4], np.int32)  # a new sequence at row 5
    pre2 = orc.conv_silu(imp, w2, pos2, bf16=False)
    np.testing.assert_allclose(pre2[4], pre[4])
    assert np.all(pre2[5:] == 0)


def test_layer_norm_against_torch(orc):
    torch = pytest.importorskip("torch")
    x = orc.fill_normal((13, 768), 4) * 3 + 1
    g = orc.fill_normal((768,), 5)
    b = orc.fill_normal((768,), 6)
    expect = torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (768,),
                                            torch.from_numpy(g).double(),
                                            torch.from_numpy(b).double(), 1e-5).numpy()
    np.testing.assert_allclose(orc.layer_norm(x, g, b, 1e-5), expect, rtol=1e-5, atol=1e-5)


def test_argmax_ties_take_lowest_index(orc):
    """src/models/laya.rs:909-916 keeps the lowest index among equal maxima."""
    assert orc.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert orc.argmax([5.0]) == 0
    assert orc.argmax([-1.0, -1.0]) == 0
    assert orc.argmax([0.0, 1.0, 2.0, 7.0]) == 3


# --------------------------------------------------------------- bf16 ----

def test_round_bf16_round_to_nearest_even(orc):
    cases = {1.0: 1.0, 1.0 + 2 ** -8: 1.0, 1.0 + 3 * 2 ** -8: 1.0 + 2 ** -6,
             1.0 + 2 ** -8 + 2 ** -20: 1.0 + 2 ** -7, -2.5: -2.5, 0.0: 0.0}
    for v, r in cases.items():
        assert orc.lib().orc_round_bf16(v) == np.float32(r), v
    torch = pytest.importorskip("torch")
    x = orc.fill_normal((1 << 16,), 77) * 1000
    expect = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(orc.round_bf16(x), expect)
    bits = orc.to_bf16_bits(x)
    np.testing.assert_array_equal(orc.from_bf16_bits(bits), expect)


# --------------------------------------------------------- seeded data ---

def test_fill_normal_distribution_and_reproducibility(orc):
    a = orc.fill_normal((200_000,), 1234)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    assert scipy.stats.kstest(a[:20000], "norm").pvalue > 1e-3
    b = orc.fill_normal((1000,), 1234)
    np.testing.assert_array_equal(a[:1000], b)  # element i depends only on (seed, i)
    w = orc.fill_normal((50_000,), 99, 0.02)
    assert abs(w.std() - 0.02) < 0.0005
    assert not np.array_equal(orc.fill_normal((10,), 1), orc.fill_normal((10,), 2))


@pytest.mark.parametrize("seed", [0, 1, 7, 12345])
def test_pack_ragged_contract(orc, seed):
    lengths = orc.pack_ragged(seed, 16, 512, 8192)
    assert lengths.sum() <= 8192 and ((lengths >= 16) & (lengths <= 512)).all()
    # The next draw would overflow the budget (SplitMix64 element len(lengths)).
    from sys1_amd.batching import splitmix64
    nxt = 16 + int(splitmix64(seed, np.array([len(lengths)]))[0] % np.uint64(497))
    assert lengths.sum() + nxt > 8192 or lengths.sum() == 8192
    exact = orc.pack_ragged(seed, 64, 2048, 8192, exact=True)
    assert exact.sum() == 8192 and (exact[:-1] >= 64).all()


# ------------------------------------------------------------- golden ----

def test_oracle_matches_golden_fixtures(orc):
    """Fixtures written by tests/golden/make_golden.py from numpy/scipy
    (independent of the oracle)."""
    import json
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "projection_golden.json")
    with open(path) as f:
        gold = json.load(f)
    for case in gold["linear"]:
        x = np.array(case["x"], np.float32)
        w = np.array(case["w"], np.float32)
        b = np.array(case["bias"], np.float32) if case["bias"] is not None else None
        np.testing.assert_allclose(orc.linear_f64(x, w, b), case["y"], rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(orc.linear_f32(x, w, b), case["y"], rtol=1e-5, atol=1e-5)
    g = gold["geglu"]
    np.testing.assert_allclose(orc.geglu(np.array(g["input"], np.float32)), g["output"], atol=1e-6)
    s = gold["swiglu"]
    np.testing.assert_allclose(orc.swiglu(np.array(s["gate"], np.float32), np.array(s["up"], np.float32)),
                               s["output"], atol=1e-5, rtol=1e-6)
    r = gold["bf16"]
    np.testing.assert_array_equal(orc.to_bf16_bits(np.array(r["input"], np.float32)), r["bits"])


def _transformers_rope(q, k, cos_half, sin_half):
    """transformers' ModernBERT apply_rotary_pos_emb (rotate-half RoPE, a
    library routine independent of the reference) on [B, heads, L, dim]."""
    torch = pytest.importorskip("torch")
    mb = pytest.importorskip("transformers.models.modernbert.modeling_modernbert")
    cos = torch.from_numpy(np.concatenate([cos_half, cos_half], -1))[None]
    sin = torch.from_numpy(np.concatenate([sin_half, sin_half], -1))[None]
    qo, ko = mb.apply_rotary_pos_emb(torch.from_numpy(q), torch.from_numpy(k), cos, sin)
    return qo.numpy(), ko.numpy()


def test_rope_qkv_reference_fixture_against_transformers(orc):
    """The reference's own fused-RoPE test (src/archs/modernbert.rs:768-816):
    qkv (2, 5, 3, 2, 8) from ((i*37 % 127) - 63)/21, cos/sin (5, 4) from
    i*0.13; the oracle on the packed tokens (position = token % 5) against
    transformers' rotate-half RoPE and the untouched v."""
    B, L, heads, dim = 2, 5, 2, 8
    vals = ((np.arange(480) * 37 % 127).astype(np.float32) - 63.0) / 21.0
    qkv = vals.reshape(B, L, 3, heads, dim)
    ang = np.arange(20, dtype=np.float32) * np.float32(0.13)
    cos_t, sin_t = np.cos(ang).reshape(L, dim // 2), np.sin(ang).reshape(L, dim // 2)
    packed = qkv.reshape(B * L, 3 * heads * dim)
    pos = np.arange(B * L) % L
    out = orc.rope_qkv(packed, cos_t, sin_t, pos, heads, dim)
    q = np.ascontiguousarray(qkv[:, :, 0].transpose(0, 2, 1, 3))   # [B, heads, L, dim]
    k = np.ascontiguousarray(qkv[:, :, 1].transpose(0, 2, 1, 3))
    eq, ek = _transformers_rope(q, k, cos_t, sin_t)
    got = out.reshape(3, B, L, heads, dim).transpose(0, 1, 3, 2, 4)  # -> [3, B, heads, L, dim]
    np.testing.assert_allclose(got[0], eq, rtol=0, atol=2e-6)
    np.testing.assert_allclose(got[1], ek, rtol=0, atol=2e-6)
    np.testing.assert_array_equal(got[2], qkv[:, :, 2].transpose(0, 2, 1, 3))


def test_rope_tables_and_invariants(orc):
    """Tables against their closed form in float64 (inv_freq[0] = 1, so
    column 0 is cos/sin of the position itself); RoPE at position 0 is the
    identity; every rotated (c, c + dim/2) pair keeps its norm; a wrong sign
    or a swapped half would break the transformers comparison above."""
    dim, P = 64, 300
    c, s = orc.rope_tables(160000.0, dim, P)
    p = np.arange(P, dtype=np.float64)[:, None]
    inv = 1.0 / 160000.0 ** (np.arange(0, dim, 2, dtype=np.float64) / dim)
    np.testing.assert_allclose(c, np.cos(p * inv.astype(np.float32)), atol=3e-5)
    np.testing.assert_allclose(s, np.sin(p * inv.astype(np.float32)), atol=3e-5)
    np.testing.assert_allclose(c[:, 0], np.cos(np.arange(P)), atol=3e-5)
    rng = np.random.default_rng(5)
    heads = 3
    qkv = rng.standard_normal((7, 3 * heads * dim)).astype(np.float32)
    out = orc.rope_qkv(qkv, c, s, np.zeros(7, np.int32), heads, dim)
    np.testing.assert_allclose(out.transpose(1, 0, 2).reshape(7, -1), qkv, atol=1e-6)
    pos = rng.integers(0, P, 7)
    out = orc.rope_qkv(qkv, c, s, pos, heads, dim)
    half = dim // 2
    for plane in range(2):
        a = qkv[:, plane * heads * dim:(plane + 1) * heads * dim].reshape(7, heads, 2, half)
        b = out[plane].reshape(7, heads, 2, half)
        np.testing.assert_allclose(np.hypot(a[:, :, 0], a[:, :, 1]), np.hypot(b[:, :, 0], b[:, :, 1]),
                                   rtol=2e-5, atol=1e-5)


# ------------------------------------------------------- composite chains ---

def _torch_scorer_f64(h, ln_w, ln_b, w_in, b_in, w_out, b_out):
    """Independent restatement through torch f64 library calls:
    layer_norm -> addmm -> gelu(erf) -> addmm (src/models/laya.rs:510-520)."""
    import torch
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    z = torch.nn.functional.layer_norm(t(h), (h.shape[1],), t(ln_w), t(ln_b), 1e-5)
    z = torch.nn.functional.gelu(torch.addmm(t(b_in), z, t(w_in).T), approximate="none")
    return torch.addmm(t(b_out), z, t(w_out).T)[:, 0].numpy()


def test_laya_scorer_against_torch_f64(orc):
    rng = np.random.default_rng(5)
    H = 96
    h = orc.fill_normal((37, H), 3)
    ln_w = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    ln_b = (0.1 * rng.standard_normal(H)).astype(np.float32)
    w_in = orc.fill_normal((H, H), 4, 0.1)
    b_in = (0.1 * rng.standard_normal(H)).astype(np.float32)
    w_out = orc.fill_normal((1, H), 6, 0.1)
    b_out = np.array([0.25], np.float32)
    got = orc.laya_scorer_f32(h, ln_w, ln_b, w_in, b_in, w_out, b_out)
    ref = _torch_scorer_f64(h, ln_w, ln_b, w_in, b_in, w_out, b_out)
    assert got.shape == (37,)
    assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    # A GELU applied before the bias (a plausible slip) moves the logits well
    # beyond that bound: the bias is large enough to matter.
    wrong = _torch_scorer_f64(h, ln_w, ln_b, w_in, 0 * b_in, w_out, b_out)
    assert np.abs(wrong - ref).max() > 1e-3


def test_laya_scorer_closed_forms(orc):
    H = 64
    rng = np.random.default_rng(9)
    h = orc.fill_normal((5, H), 8)
    ln_w = np.ones(H, np.float32)
    ln_b = np.zeros(H, np.float32)
    b_in = rng.standard_normal(H).astype(np.float32)
    w_out = rng.standard_normal((1, H)).astype(np.float32)
    b_out = np.array([-0.75], np.float32)
    # Zero w_in: every row gives gelu(b_in) . w_out + b_out, whatever h is.
    got = orc.laya_scorer_f32(h, ln_w, ln_b, np.zeros((H, H), np.float32), b_in, w_out, b_out)
    gel = 0.5 * b_in.astype(np.float64) * (1 + np.array([math.erf(v / math.sqrt(2)) for v in b_in]))
    want = float(gel @ w_out[0].astype(np.float64) + b_out[0])
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)
    # Identity w_in, zero biases and LN weight 1: logit = sum_k gelu(ln(h)_k) w_out[k];
    # with ln_b = 0 the normalised row has mean 0 and variance 1 (eps aside).
    got = orc.laya_scorer_f32(h, ln_w, ln_b, np.eye(H, dtype=np.float32), np.zeros(H, np.float32),
                              w_out, np.zeros(1, np.float32))
    hd = h.astype(np.float64)
    z = (hd - hd.mean(1, keepdims=True)) / np.sqrt(hd.var(1, keepdims=True) + 1e-5)
    gz = 0.5 * z * (1 + scipy.special.erf(z / math.sqrt(2)))
    assert np.allclose(got, gz @ w_out[0], rtol=1e-5, atol=1e-5)
    # The LayerNorm is applied: scaling a row (LN is scale-invariant up to eps)
    # leaves its logit, while a row shift leaves it too (mean removed).
    base = orc.laya_scorer_f32(h, ln_w, ln_b, np.eye(H, dtype=np.float32), b_in, w_out, b_out)
    moved = orc.laya_scorer_f32((3 * h + 2).astype(np.float32), ln_w, ln_b, np.eye(H, dtype=np.float32),
                                b_in, w_out, b_out)
    assert np.allclose(base, moved, rtol=1e-4, atol=1e-4)


def _mb_weights(orc, H, I, seed):
    return [orc.fill_normal((3 * H, H), seed, 0.05), orc.fill_normal((H, H), seed + 1, 0.05),
            orc.fill_normal((2 * I, H), seed + 2, 0.05), orc.fill_normal((H, I), seed + 3, 0.05)]


def test_modernbert_layer_against_numpy_f64(orc):
    """The layer chain of src/archs/modernbert.rs:857-887 (with the V-block
    attention stand-in) restated in numpy f64: Wqkv -> V block -> Wo + h ->
    Wi -> gelu(first half) * second half -> Wo + h1."""
    H, I = 32, 48
    h = orc.fill_normal((19, H), 2)
    wqkv, wo, wi, wo2 = _mb_weights(orc, H, I, 20)
    d = lambda a: np.asarray(a, np.float64)
    qkv = d(h) @ d(wqkv).T
    h1 = qkv[:, 2 * H:] @ d(wo).T + d(h)
    u = h1 @ d(wi).T
    g = 0.5 * u[:, :I] * (1 + scipy.special.erf(u[:, :I] / math.sqrt(2))) * u[:, I:]
    ref = g @ d(wo2).T + h1
    got = orc.modernbert_layer_f32(h, wqkv, wo, wi, wo2)
    assert got.shape == h.shape
    assert _rel_fro(got, ref) < 1e-5


def test_modernbert_layer_closed_forms(orc):
    H, I = 16, 24
    h = orc.fill_normal((7, H), 4)
    wqkv, wo, wi, wo2 = _mb_weights(orc, H, I, 30)
    z = lambda a: np.zeros_like(a)
    # All weights zero: both residuals carry h through unchanged, exactly.
    assert np.array_equal(orc.modernbert_layer_f32(h, z(wqkv), z(wo), z(wi), z(wo2)), h)
    # A one-hot V block (rows 2H.. of Wqkv = I) with Wo = I and the MLP off:
    # out = h + V = 2h.  The same one-hot placed in the q or k block gives h.
    eye = np.eye(H, dtype=np.float32)
    for blk, want in ((2, 2 * h), (0, h), (1, h)):
        w = np.zeros((3 * H, H), np.float32)
        w[blk * H:(blk + 1) * H] = eye
        got = orc.modernbert_layer_f32(h, w, eye, z(wi), z(wo2))
        assert np.allclose(got, want, rtol=0, atol=1e-6), blk
    # Each residual alone: attention branch off (Wo = 0) leaves h + MLP(h);
    # MLP off leaves h + attention(h).
    d = lambda a: np.asarray(a, np.float64)
    u = d(h) @ d(wi).T
    mlp = (0.5 * u[:, :I] * (1 + scipy.special.erf(u[:, :I] / math.sqrt(2))) * u[:, I:]) @ d(wo2).T
    got = orc.modernbert_layer_f32(h, wqkv, z(wo), wi, wo2)
    assert _rel_fro(got, d(h) + mlp) < 1e-5
    attn = (d(h) @ d(wqkv).T)[:, 2 * H:] @ d(wo).T
    got = orc.modernbert_layer_f32(h, wqkv, wo, z(wi), wo2)
    assert _rel_fro(got, d(h) + attn) < 1e-5
    # The gate is the first half of Wi's output: swapping the halves changes it.
    swapped = np.concatenate([wi[I:], wi[:I]])
    mlp_of = lambda w: orc.modernbert_layer_f32(h, wqkv, z(wo), w, wo2).astype(np.float64) - h
    assert _rel_fro(mlp_of(swapped), mlp_of(wi)) > 0.5
