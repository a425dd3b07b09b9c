"""GPU parity of the DeltaNet in_proj with its causal conv + SiLU fused
(sys1hip_linear_conv_silu_bf16) against the oracle: the projection, then the
reference's bf16 conv arithmetic (src/archs/qwen35_text.rs:515-526,632-650;
src/kernels/qwen35.cu:3-29) over packed ragged sequences.

Two checks per case:
  - against the unfused reference chain (the oracle's f32 projection, then
    the reference's bf16 conv arithmetic): the projection tolerance
    (rel. Frobenius <= 1e-2, max-abs <= 2e-2 max|ref|);
  - the conv arithmetic itself: the oracle's conv with f32 accumulation
    (the kernel's arithmetic) applied to the GPU's own unfused projection
    must match the fused output to 1 bf16 ulp, nearly all bit for bit
    (the last bits of exp and the reciprocal may differ); forced stream-K
    schedules, whose split tiles recompute halo rows with another K split,
    are allowed a few ulp on under 0.1% of the outputs.
Sequences start inside tiles, on tile-row boundaries and in the overlapped
halo rows, so the taps that cross tile rows and sequence starts are covered.
"""
import numpy as np
import pytest

from gpu_helpers import assert_parity, bf16_ulp, to_gpu_bf16, to_np

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


def _lengths(M, seed):
    """Ragged lengths summing to M, with sequence starts at 125 and 128 (the
    first tile-row boundaries of a 128-row tile with a 3-row halo) and
    runs of 1- and 2-token sequences."""
    rng = np.random.default_rng(seed)
    cuts = {0, 125, 128, 129, 131, M}
    cuts |= set(int(v) for v in rng.integers(1, M, size=max(1, M // 40)))
    c = sorted(v for v in cuts if 0 <= v <= M)
    return np.diff(c).astype(np.int64)


def _case(orc, M, N, C, K, seed, norm):
    from sys1_amd import batching
    x = orc.round_bf16(orc.fill_normal((M, K), seed))
    w = orc.round_bf16(orc.fill_normal((N, K), seed + 1, 0.04))
    cw = orc.round_bf16(orc.fill_normal((C, 4), seed + 2, 0.5))
    g = orc.round_bf16(orc.fill_normal((K,), seed + 3, 0.1)) if norm else None
    pos = batching.positions(_lengths(M, seed))
    assert pos.size == M
    return x, w, cw, g, pos


def _run(dev, x, w, cw, g, pos, C):
    from sys1_amd.deltanet import InProjConv
    m = InProjConv(to_gpu_bf16(w, torch), torch.from_numpy(cw), C,
                   torch.from_numpy(g) if g is not None else None, 1e-6, device=dev)
    return to_np(m(to_gpu_bf16(x, torch), torch.from_numpy(pos).cuda()))


def _gpu_projection(dev, x, w, g):
    """The unfused GPU projection (plain GEMM, or the fused RMSNorm GEMM)."""
    from sys1_amd.linear import Linear
    from sys1_amd.norm import NormLinear
    if g is None:
        return to_np(Linear(to_gpu_bf16(w, torch), device=dev)(to_gpu_bf16(x, torch)))
    return to_np(NormLinear(to_gpu_bf16(w, torch), torch.from_numpy(g), "rms", 1e-6, device=dev)(
        to_gpu_bf16(x, torch)))


def _check(orc, dev, y, x, w, cw, g, pos, C, what, split_k=False):
    # 1. against the oracle chain from its f32 projection
    xin = orc.round_bf16(orc.rms_norm(x, g, 1e-6)) if g is not None else x
    proj = orc.round_bf16(orc.linear_f32(xin, w))
    ref = np.concatenate([orc.conv_silu(proj[:, :C], cw, pos), proj[:, C:]], axis=1)
    rel, mx = assert_parity(y, ref, what)
    # 2. the conv arithmetic on the GPU's own projection
    pg = _gpu_projection(dev, x, w, g)
    conv32 = orc.round_bf16(orc.conv_silu(pg[:, :C], cw, pos, bf16=False))
    ref2 = np.concatenate([conv32, pg[:, C:]], axis=1)
    d = np.abs(y.astype(np.float64) - ref2)
    ulp = bf16_ulp(ref2) + 1e-30
    bad = d > ulp
    if split_k:
        # A stream-K schedule splits K differently in the two tiles that
        # compute a halo row, so the conv may read that row's projection one
        # bf16 ulp away from the stored one (f32 partial sums added in another
        # order): a few conv outputs then move by a few ulp.
        # (Near-zero outputs of a cancelling sum can move by more ulps of
        # their own; the bound is 4 ulp or 1e-3 of the largest output.)
        tol = 4 * ulp + 1e-3 * np.abs(ref2).max()
        assert bad.mean() < 1e-3 and (d <= tol).all(), \
            f"{what}: {bad.sum()} elements > 1 ulp, worst {(d / tol).max():.2f} of the bound"
    else:
        assert not bad.any(), f"{what}: {bad.sum()} elements > 1 ulp from the conv of the GPU projection"
    exact = float((d == 0).mean())
    assert exact > 0.98, f"{what}: only {exact:.4f} bit-equal"
    print(f"[gpu]   rel_fro={rel:.2e} max_abs/max={mx:.2e} bit-equal to conv(GPU proj) {exact:.5f}",
          flush=True)


CASES = [
    # (M, N, conv_ch, K, norm): Qwen-small-like in_proj (qkv | z | b | a), small and large M
    (1000, 1056, 512, 256, False),
    (1000, 1056, 512, 256, True),
    (128, 2080, 1024, 512, True),     # one tile row (stream-K)
    (40, 768, 768, 320, False),       # all channels convolved
    (333, 544, 256, 200, False),      # ragged K and N
]


@pytest.mark.parametrize("M,N,C,K,norm", CASES)
def test_inproj_conv_matches_oracle(dev, orc, M, N, C, K, norm):
    print(f"[gpu] inproj conv M={M} N={N} C={C} K={K} norm={norm}", flush=True)
    x, w, cw, g, pos = _case(orc, M, N, C, K, 100 + M, norm)
    y = _run(dev, x, w, cw, g, pos, C)
    _check(orc, dev, y, x, w, cw, g, pos, C, f"M={M} N={N} C={C} K={K} norm={norm}")


def test_every_conv_kernel_and_grid(dev, orc):
    """The fused form: each kernel with a conv epilogue, forced, over
    several grids (tile rows split across workgroups, stream-K partial
    tiles)."""
    from sys1_amd import kernel_names
    M, N, C, K = 700, 544, 384, 328
    x, w, cw, g, pos = _case(orc, M, N, C, K, 7, False)
    # (waves spanning every row; producer-wave shapes have no conv epilogue)
    names = [n for n in kernel_names() if "_w1x" in n and "_p" not in n.split("_w1x")[1]]
    assert len(names) >= 3
    try:
        for name in names:
            for grid in (0, 1, 7, 64):
                dev.set_kernel(kernel_names().index(name))
                dev.set_grid(grid)
                print(f"[gpu] conv kernel {name} grid={grid}", flush=True)
                y = _run(dev, x, w, cw, g, pos, C)
                _check(orc, dev, y, x, w, cw, g, pos, C, f"{name} grid={grid}", name.startswith("stream_"))
    finally:
        dev.set_kernel(-1)
        dev.set_grid(0)


def test_two_pass_on_a_forced_tile_kernel(dev, orc):
    """A forced kernel without the conv epilogue runs the two-pass form (its
    projection, then the in-place conv): the same checks."""
    from sys1_amd import kernel_names
    M, N, C, K = 520, 544, 256, 264
    x, w, cw, g, pos = _case(orc, M, N, C, K, 3, True)
    try:
        dev.set_kernel(kernel_names().index("tile_128x128_s2_w2x2"))
        y = _run(dev, x, w, cw, g, pos, C)
        _check(orc, dev, y, x, w, cw, g, pos, C, "two-pass on tile_128x128_s2_w2x2")
    finally:
        dev.set_kernel(-1)


def test_two_pass_long_segments(dev, orc):
    """From 8192 rows with enough channels the conv pass walks 64-row
    segments (four chunks per thread, halos only every 64 rows): sequence
    starts on, just before and just after those boundaries."""
    from sys1_amd import batching
    M, C, K = 8192, 8192, 64
    N = C + 32
    x = orc.round_bf16(orc.fill_normal((M, K), 61))
    w = orc.round_bf16(orc.fill_normal((N, K), 62, 0.1))
    cw = orc.round_bf16(orc.fill_normal((C, 4), 63, 0.5))
    cuts = sorted({0, 63, 64, 65, 127, 128, 130, 2048, 4095, 4096, 4097, 6001, 8190, M})
    pos = batching.positions(np.diff(cuts))
    print(f"[gpu] conv two-pass long segments M={M} N={N} C={C} K={K}", flush=True)
    y = _run(dev, x, w, cw, None, pos, C)
    _check(orc, dev, y, x, w, cw, None, pos, C, "long segments")


def test_two_pass_segments_and_halos(dev, orc):
    """Rows cut into many conv segments (M well above the 64-row segment),
    sequence starts on and next to segment boundaries."""
    from sys1_amd import batching
    M, N, C, K = 1000, 288, 256, 64
    x = orc.round_bf16(orc.fill_normal((M, K), 51))
    w = orc.round_bf16(orc.fill_normal((N, K), 52, 0.1))
    cw = orc.round_bf16(orc.fill_normal((C, 4), 53, 0.5))
    cuts = sorted({0, 64, 127, 128, 129, 190, 192, 256, 511, 512, 700, 703, M})
    pos = batching.positions(np.diff(cuts))
    y = _run(dev, x, w, cw, None, pos, C)
    _check(orc, dev, y, x, w, cw, None, pos, C, "segments")
