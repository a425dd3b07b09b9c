"""GPU parity of the pre-norm projections (sys1hip_fold_norm_weight,
sys1hip_norm_linear_bf16) against the oracle's unfused reference chain:
norm -> bf16 -> projection -> epilogue, as the reference runs it
(ModernBERT: bias-free LayerNorm, src/archs/modernbert.rs:865-868,884,1005-1034;
Qwen3.5: RMSNorm(1+w), src/archs/qwen35_text.rs:178-203,933,939).

Bar: the projection path's parity metrics, relative Frobenius error <= 1e-2
and max-abs error <= 2e-2 * max|ref|, per output.  The fused path folds the
norm weight into the bf16 weight and normalises the f32 accumulators, so it
rounds in different places from the reference (which rounds the normalised
activations); the bar is the tolerance, not bit equality.  The inputs carry
per-row offsets and a few large columns, as residual streams do, so that
the LayerNorm mean term (r_m mu_m colsum_n) is exercised.
"""
import numpy as np
import pytest

from gpu_helpers import assert_parity, to_gpu_bf16, to_np

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from sys1_amd.device import HipDevice
    d = HipDevice(0)
    yield d
    d.set_kernel(-1)
    d.set_grid(0)


def _stream(orc, M, K, seed):
    """Residual-stream-like rows: N(0,1) + a per-row offset, 4 columns x6."""
    x = orc.fill_normal((M, K), seed)
    x += orc.fill_normal((M, 1), seed + 7, 0.7)
    x[:, [1, K // 3, K // 2, K - 2]] *= 6.0
    return orc.round_bf16(x)


def _weights(orc, N, K, seed, kind):
    w = orc.round_bf16(orc.fill_normal((N, K), seed, 0.02))
    g = orc.fill_normal((K,), seed + 3, 0.1)
    g = orc.round_bf16(1.0 + g) if kind == "layer" else orc.round_bf16(g)  # LN weight ~1; RMS w ~0
    return w, g


def _ref(orc, x, w, g, kind, eps, gated):
    if kind == "layer":
        xn = orc.layer_norm_bf16(x, g, eps)
    else:
        xn = orc.round_bf16(orc.rms_norm(x, g, eps))
    proj = orc.linear_f32(xn, w)
    if gated == "gelu":
        return orc.geglu(proj)
    if gated == "silu":
        return orc.swiglu(*np.split(proj, 2, axis=1))
    return orc.round_bf16(proj)


CASES = [
    # (kind, gated, M, N, K): ModernBERT-base Wqkv / Wi, Qwen-small qkv and gate/up shapes
    ("layer", None, 1000, 2304, 768),
    ("layer", "gelu", 1000, 2304, 768),
    ("layer", None, 64, 768, 768),
    ("layer", "gelu", 200, 5248, 1024),
    ("rms", None, 1000, 4608, 2048),
    ("rms", "silu", 700, 2048, 2048),
    ("rms", None, 128, 1024, 2048),
    ("rms", "silu", 33, 1024, 512),
    ("layer", None, 40, 256, 8200),   # rows longer than the register-resident statistics path
    ("rms", None, 40, 256, 8200),
]


@pytest.mark.parametrize("kind,gated,M,N,K", CASES)
def test_norm_linear_matches_unfused_chain(dev, orc, kind, gated, M, N, K):
    from sys1_amd.norm import NormLinear
    eps = 1e-5 if kind == "layer" else 1e-6
    print(f"[gpu] norm={kind} gated={gated} M={M} N={N} K={K}", flush=True)
    x = _stream(orc, M, K, 11 + M)
    w, g = _weights(orc, N, K, 5 + N, kind)
    lin = NormLinear(to_gpu_bf16(w, torch), torch.from_numpy(g), kind, eps, gated, device=dev)
    y = to_np(lin(to_gpu_bf16(x, torch)))
    ref = _ref(orc, x, w, g, kind, eps, gated)
    assert y.shape == ref.shape
    rel, mx = assert_parity(y, ref, f"{kind}/{gated} M={M} N={N} K={K}")
    print(f"[gpu]   rel_fro={rel:.2e} max_abs/max={mx:.2e}", flush=True)


@pytest.mark.parametrize("offset", [4.0, 16.0])
def test_layernorm_rows_with_large_means(dev, orc, offset):
    """Rows whose mean is large against their spread: the epilogue's r (acc -
    mu c) cancels heavily, and the -mu c term (a bf16 hi/lo-split MFMA in
    the kernel) must keep the result within the projection tolerance, on the
    producer-wave 128x128 shape and on the plain one."""
    from sys1_amd import kernel_names
    from sys1_amd.norm import NormLinear
    M, N, K = 600, 2304, 768
    x = orc.fill_normal((M, K), 61)
    x += offset * (1.0 + orc.fill_normal((M, 1), 62, 0.25))
    x = orc.round_bf16(x)
    w, g = _weights(orc, N, K, 63, "layer")
    ref = _ref(orc, x, w, g, "layer", 1e-5, None)
    lin = NormLinear(to_gpu_bf16(w, torch), torch.from_numpy(g), "layer", 1e-5, None, device=dev)
    try:
        for name in ("tile_128x128_s2_w2x2_p4", "tile_128x128_s2_w2x2", None):
            dev.set_kernel(kernel_names().index(name) if name else -1)
            print(f"[gpu] layernorm offset={offset} kernel={name or 'auto'}", flush=True)
            rel, mx = assert_parity(to_np(lin(to_gpu_bf16(x, torch))), ref, f"offset {offset} {name}")
            print(f"[gpu]   rel_fro={rel:.2e} max_abs/max={mx:.2e}", flush=True)
    finally:
        dev.set_kernel(-1)


def test_fold_is_exact_and_colsum_sums_the_folded_rows(dev, orc):
    from sys1_amd.norm import fold_norm_weight
    N, K = 300, 1032
    for kind in ("layer", "rms"):
        w, g = _weights(orc, N, K, 17, kind)
        print(f"[gpu] fold {kind} N={N} K={K}", flush=True)
        wf, cs = fold_norm_weight(to_gpu_bf16(w, torch), torch.from_numpy(g), kind, device=dev)
        a = g if kind == "layer" else 1.0 + g.astype(np.float32)
        expect = orc.round_bf16(w * a[None, :].astype(np.float32))
        np.testing.assert_array_equal(to_np(wf), expect)
        if kind == "layer":
            s64 = expect.astype(np.float64).sum(axis=1)
            got = cs.cpu().numpy().astype(np.float64)
            assert np.abs(got - s64).max() <= 1e-5 * np.abs(expect).sum(axis=1).max()
        else:
            assert cs is None


def test_every_kernel_with_every_norm_epilogue(dev, orc):
    """Force each kernel id (tile and stream-K schedules) through the four
    pre-norm epilogues on a ragged shape."""
    from sys1_amd import kernel_names
    from sys1_amd.norm import NormLinear
    M, N, K = 300, 384, 328
    x = _stream(orc, M, K, 23)
    xg = to_gpu_bf16(x, torch)
    try:
        for kind, gated in (("layer", None), ("layer", "gelu"), ("rms", None), ("rms", "silu")):
            eps = 1e-5 if kind == "layer" else 1e-6
            w, g = _weights(orc, N, K, 29, kind)
            lin = NormLinear(to_gpu_bf16(w, torch), torch.from_numpy(g), kind, eps, gated, device=dev)
            ref = _ref(orc, x, w, g, kind, eps, gated)
            for kid, name in enumerate(kernel_names()):
                # (the gated epilogues need whole 32-row gate/up groups)
                if gated and name.startswith("skinny_") and int(name.split("_")[1].split("x")[1]) % 32:
                    continue
                dev.set_kernel(kid)
                print(f"[gpu] {name} norm={kind} gated={gated}", flush=True)
                assert_parity(to_np(lin(xg)), ref, f"{name} {kind}/{gated}")
    finally:
        dev.set_kernel(-1)


def test_rows_are_independent_and_repeat_bitwise(dev, orc):
    """Row statistics are per row: a permutation of the rows permutes the
    output exactly, and a second call gives the same bits."""
    from sys1_amd.norm import NormLinear
    M, N, K = 513, 768, 768
    x = _stream(orc, M, K, 31)
    w, g = _weights(orc, N, K, 37, "layer")
    lin = NormLinear(to_gpu_bf16(w, torch), torch.from_numpy(g), "layer", 1e-5, device=dev)
    xg = to_gpu_bf16(x, torch)
    y1 = lin(xg)
    y2 = lin(xg)
    assert torch.equal(y1, y2)
    perm = torch.from_numpy(np.random.default_rng(0).permutation(M)).to(xg.device)
    yp = lin(xg[perm].contiguous())
    assert torch.equal(yp, y1[perm])


def test_norm_linear_errors(dev, orc):
    from sys1_amd import _lib
    from sys1_amd.norm import NormLinear
    w = torch.zeros(64, 64, dtype=torch.bfloat16, device="cuda:0")
    g = torch.ones(64)
    with pytest.raises(ValueError):
        NormLinear(w, g, "batch", 1e-5, device=dev)
    with pytest.raises(ValueError):
        NormLinear(w, torch.ones(32), "layer", 1e-5, device=dev)
    lin = NormLinear(w, g, "layer", 1e-5, device=dev)
    with pytest.raises(ValueError):
        lin(torch.zeros(4, 32, dtype=torch.bfloat16, device="cuda:0"))
    # RMSNorm with GeGLU is not a combination the reference has.
    with pytest.raises(_lib.Sys1HipError):
        NormLinear(torch.zeros(64, 64, dtype=torch.bfloat16, device="cuda:0"), g, "rms", 1e-6,
                   "gelu", device=dev)(torch.zeros(4, 64, dtype=torch.bfloat16, device="cuda:0"))


def test_blocked_weight_with_every_norm_epilogue_is_bitwise_row_major(dev, orc):
    """The folded weight in the blocked layout (what ProjectionStack(norms=True,
    blocked=True) and the bench run) gives the row-major folded weight's
    results bit for bit, on a forced kernel of every family (tile, stream-K,
    skinny) and every pre-norm epilogue, with N and K not multiples of the
    32 x 64 block."""
    from sys1_amd import kernel_names
    from sys1_amd.norm import NormLinear
    names = kernel_names()
    picks = [next(i for i, n in enumerate(names) if n.startswith(f)) for f in ("tile_", "stream_", "skinny_")]
    picks += [i for i, n in enumerate(names) if n.startswith("skinny_") and int(n.split("_")[1].split("x")[1]) % 32 == 0][:1]
    M, N, K = 150, 352, 328
    x = _stream(orc, M, K, 41)
    xg = to_gpu_bf16(x, torch)
    try:
        for kind, gated in (("layer", None), ("layer", "gelu"), ("rms", None), ("rms", "silu")):
            eps = 1e-5 if kind == "layer" else 1e-6
            w, g = _weights(orc, N, K, 43, kind)
            wg, gg = to_gpu_bf16(w, torch), torch.from_numpy(g)
            rm = NormLinear(wg, gg, kind, eps, gated, device=dev)
            bl = NormLinear(wg, gg, kind, eps, gated, device=dev, blocked=True)
            ref = _ref(orc, x, w, g, kind, eps, gated)
            for kid in picks:
                name = names[kid]
                if gated and name.startswith("skinny_") and int(name.split("_")[1].split("x")[1]) % 32:
                    continue
                dev.set_kernel(kid)
                print(f"[gpu] blocked norm {name} {kind}/{gated}", flush=True)
                a, b = rm(xg), bl(xg)
                assert torch.equal(a, b), f"{name} {kind}/{gated}"
                assert_parity(to_np(b), ref, f"blocked {name} {kind}/{gated}")
    finally:
        dev.set_kernel(-1)
