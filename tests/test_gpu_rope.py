"""GPU parity of Wqkv with the fused RoPE epilogue (sys1hip_linear_rope_qkv_bf16)
against the CPU oracle's restatement of the reference's fused RoPE + q/k/v
split (src/kernels/modernbert.cu:31-74, tables src/archs/modernbert.rs:67-83).

Expected: the oracle's float64 projection of the same bf16 inputs, rounded
to bf16 (the projection's own rounding), rotated in f32 and rounded once.
Elementwise bound: one bf16 ulp of the result plus the propagated input
rounding -- the GPU's f32-accumulated projection may round each of x0, x1 to
the neighbouring bf16 (one ulp, as for a plain projection), and the rotation
carries that through with weights |cos|, |sin| <= 1, so up to two bf16 ulps
of the pair's norm, which the rotation preserves (near cancellation the
result's own ulp is far smaller than its inputs').  Plus the projection
parity bar.  v equals the plain projection bit for bit.
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


def _expected(orc, x, w, cos, sin, pos, heads):
    proj = orc.round_bf16(orc.linear_f64(orc.round_bf16(x), orc.round_bf16(w)).astype(np.float32))
    return orc.round_bf16(orc.rope_qkv(proj, cos, sin, pos, heads, 64)), proj


def _pair_norm(proj, plane, heads):
    """|(x0, x1)| of every element's rotation pair (columns c, c + 32)."""
    H = heads * 64
    blk = proj[:, plane * H:(plane + 1) * H].reshape(-1, heads, 2, 32).astype(np.float64)
    n = np.hypot(blk[:, :, 0], blk[:, :, 1])
    return np.concatenate([n, n], axis=-1).reshape(-1, H)


def _check(orc, got, exp, what, norm=None):
    tol = bf16_ulp(exp) + 1e-6
    if norm is not None:
        tol = tol + 2 * bf16_ulp(norm)
    bad = np.abs(got.astype(np.float64) - exp) > tol
    assert not bad.any(), f"{what}: {bad.sum()} elements off by >1 ulp"
    assert_parity(got, exp, what)


def test_rope_tables_match_oracle(orc):
    from sys1_amd.rope import rope_tables
    c, s = rope_tables(160000.0, 64, 8192, "cuda")
    oc, os_ = orc.rope_tables(160000.0, 64, 8192)
    # Both round (nearly) exact cos/sin of the same f32 frequencies.
    np.testing.assert_allclose(c.cpu().numpy(), oc, atol=2.5e-7)
    np.testing.assert_allclose(s.cpu().numpy(), os_, atol=2.5e-7)


@pytest.mark.parametrize("hidden,heads,seed", [(768, 12, 3), (1024, 16, 4)])
def test_rope_qkv_ragged_batch(dev, orc, hidden, heads, seed):
    """ModernBERT base / large Wqkv on a ragged packed batch (positions restart
    per sequence), global-layer theta."""
    from sys1_amd.batching import draw_lengths, positions
    from sys1_amd.linear import Linear
    from sys1_amd.rope import RopeQkvLinear, rope_tables
    lengths = draw_lengths(seed, 16, 512, 3000)
    M = int(lengths.sum())
    pos = positions(lengths)
    cos, sin = orc.rope_tables(160000.0, 64, 512)
    x = orc.fill_normal((M, hidden), seed)
    w = orc.fill_normal((3 * hidden, hidden), seed + 1, 0.02)
    exp, proj = _expected(orc, x, w, cos, sin, pos, heads)
    gc, gs = rope_tables(160000.0, 64, 512, "cuda")
    rq = RopeQkvLinear(to_gpu_bf16(w, torch), heads, gc, gs, device=dev)
    print(f"[gpu] rope-qkv M={M} hidden={hidden} kernel={dev.query_kernel(M, 3 * hidden, hidden)[1]}",
          flush=True)
    # The device tables (torch) and the oracle's (C) may differ in the last
    # float bit; the bar is against the oracle's tables either way.
    rq.cos, rq.sin = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    got = to_np(rq(to_gpu_bf16(x, torch), torch.from_numpy(pos).cuda()))
    for p, name in enumerate("qkv"):
        _check(orc, got[p], exp[p], f"{name} plane", _pair_norm(proj, p, heads) if p < 2 else None)
    plain = to_np(Linear(to_gpu_bf16(w, torch), device=dev)(to_gpu_bf16(x, torch)))
    np.testing.assert_array_equal(got[2], plain[:, 2 * hidden:])


def test_rope_qkv_every_head_aligned_kernel(dev, orc):
    """Force each kernel whose wave columns are one 64-wide head (tile and
    stream-K), small ragged shapes with row tails."""
    from sys1_amd import kernel_names, Sys1HipError
    from sys1_amd.batching import positions
    from sys1_amd.rope import RopeQkvLinear
    heads, hidden = 4, 256
    cos, sin = orc.rope_tables(10000.0, 64, 128)   # rows cover every position below
    gc, gs = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    w = orc.fill_normal((3 * hidden, hidden), 8, 0.02)
    rq = RopeQkvLinear(to_gpu_bf16(w, torch), heads, gc, gs, device=dev)
    tested = 0
    try:
        for kid, name in enumerate(kernel_names()):
            dev.set_kernel(kid)
            for M in (37, 300):
                lengths = [M // 3, M - 2 * (M // 3), M // 3]
                pos = positions(lengths)
                x = orc.fill_normal((M, hidden), M)
                try:
                    got = to_np(rq(to_gpu_bf16(x, torch), torch.from_numpy(pos).cuda()))
                except Sys1HipError as e:
                    assert "head-aligned" in str(e)
                    break
                exp, proj = _expected(orc, x, w, cos, sin, pos, heads)
                print(f"[gpu] rope-qkv forced {name} M={M}", flush=True)
                for p in range(3):
                    _check(orc, got[p], exp[p], f"{name} M={M} plane {p}",
                           _pair_norm(proj, p, heads) if p < 2 else None)
                tested += 1
    finally:
        dev.set_kernel(-1)
    assert tested >= 12


def test_rope_qkv_clamps_positions_into_the_tables(dev, orc):
    """Out-of-range positions read the nearest table row, never past it."""
    from sys1_amd.rope import RopeQkvLinear
    heads, hidden, M = 2, 128, 8
    cos, sin = orc.rope_tables(10000.0, 64, 16)
    w = orc.fill_normal((3 * hidden, hidden), 9, 0.02)
    x = orc.fill_normal((M, hidden), 10)
    rq = RopeQkvLinear(to_gpu_bf16(w, torch), heads, torch.from_numpy(cos).cuda(),
                       torch.from_numpy(sin).cuda(), device=dev)
    bad = np.array([0, 15, 16, 1000, -1, -50, 7, 99999], np.int32)
    got = to_np(rq(to_gpu_bf16(x, torch), torch.from_numpy(bad).cuda()))
    ref = to_np(rq(to_gpu_bf16(x, torch), torch.from_numpy(np.clip(bad, 0, 15)).cuda()))
    np.testing.assert_array_equal(got, ref)


def test_rope_qkv_errors(dev):
    from sys1_amd import Sys1HipError
    from sys1_amd.rope import RopeQkvLinear, rope_tables
    c, s = rope_tables(10000.0, 64, 16, "cuda")
    w = torch.zeros(3 * 128, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        RopeQkvLinear(w, 3, c, s, device=dev)          # 3 heads != 384 / 192
    rq = RopeQkvLinear(w, 2, c, s, device=dev)
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        rq(x, torch.zeros(4, dtype=torch.int64, device="cuda"))
    assert rq(x, torch.zeros(4, dtype=torch.int32, device="cuda")).shape == (3, 4, 128)
