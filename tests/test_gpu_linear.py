"""GPU parity of the projection kernels against the CPU oracle, through the
C ABI (libsys1hip.so via sys1_amd.linear).

Bar (per projection output): relative Frobenius error <= 1e-2 and max-abs
error <= 2e-2 * max|ref| against the oracle's f32 projection of the reference
f32 inputs, and -- stronger, on the same bf16 inputs -- every element within
one bf16 ulp of the correctly rounded float64 result.
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


def _inputs(orc, M, N, K, seed):
    x = orc.fill_normal((M, K), seed)
    w = orc.fill_normal((N, K), seed + 1, 0.02)
    return x, w


def _check_close_to_rounded(orc, out, ref64, what):
    """Every element within 1 bf16 ulp (+tiny abs) of bf16(ref64)."""
    r = orc.round_bf16(ref64.astype(np.float32))
    err = np.abs(out.astype(np.float64) - r)
    tol = bf16_ulp(r) + 1e-6
    bad = err > tol
    assert not bad.any(), f"{what}: {bad.sum()} elements off by >1 ulp, worst {err.max():.3e}"
    return float((err == 0).mean())


SHAPES = [
    (1, 64, 64), (15, 48, 136), (64, 768, 768), (100, 1000, 200), (256, 2304, 768),
    (257, 768, 1152), (300, 130, 64), (1024, 768, 768), (1024, 2304, 768), (777, 520, 328),
]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_linear_auto_kernel_matches_oracle(dev, orc, M, N, K):
    from sys1_amd.linear import Linear
    print(f"[gpu] linear auto M={M} N={N} K={K} kernel={dev.query_kernel(M, N, K)[1]}", flush=True)
    x, w = _inputs(orc, M, N, K, 100 + M)
    lin = Linear(to_gpu_bf16(w, torch), device=dev)
    y = to_np(lin(to_gpu_bf16(x, torch)))
    # The reference f32 path on the f32 inputs (the stated tolerance).
    assert_parity(y, orc.linear_f32(x, w), f"M={M} N={N} K={K} vs f32 oracle")
    # The same bf16 inputs: within one bf16 ulp of the exact product.
    xb, wb = orc.round_bf16(x), orc.round_bf16(w)
    exact = _check_close_to_rounded(orc, y, orc.linear_f64(xb, wb), f"M={M} N={N} K={K}")
    assert exact > 0.9


def _kernel_ids():
    from sys1_amd import kernel_names
    return list(enumerate(kernel_names()))


@pytest.mark.parametrize("kid,name", _kernel_ids())
def test_every_kernel_every_epilogue(dev, orc, kid, name):
    """Force each kernel id and check every epilogue on ragged shapes."""
    from sys1_amd import _lib
    from sys1_amd.linear import GatedLinear, Linear
    skinny = name.startswith("skinny_")
    if name.startswith("stream_"):
        cap = int(name.split("_")[1].split("x")[0])
        Ms = sorted({max(1, cap // 2 + 3), cap, 300})
    elif skinny:  # one tile row, and several with a ragged last one
        cap = int(name.split("_")[1].split("x")[0])
        Ms = sorted({1, max(1, cap // 2 + 3), cap, 300})
    else:
        Ms = [300, 513]
    # (skinny kernels with whole 32-row gate/up groups run the gated epilogues)
    gated_ok = not skinny or int(name.split("_")[1].split("x")[1]) % 32 == 0
    dev.set_kernel(kid)
    try:
        for M in Ms:
            N, K = 384, 328
            print(f"[gpu] kernel={name} M={M} N={N} K={K}", flush=True)
            x, w = _inputs(orc, M, N, K, 7 + M)
            xb, wb = orc.round_bf16(x), orc.round_bf16(w)
            xg, wg = to_gpu_bf16(x, torch), to_gpu_bf16(w, torch)
            proj = orc.linear_f64(xb, wb).astype(np.float32)
            p16 = orc.round_bf16(proj)
            bias = orc.fill_normal((N,), 3)
            bb = orc.round_bf16(bias)
            res = orc.fill_normal((M, N), 4)
            rb = orc.round_bf16(res)
            # none
            y = to_np(Linear(wg, device=dev)(xg))
            _check_close_to_rounded(orc, y, proj, f"{name} none")
            # bias: bf16(bf16(p) + b)
            y = to_np(Linear(wg, to_gpu_bf16(bias, torch), device=dev)(xg))
            assert_parity(y, orc.round_bf16(p16 + bb), f"{name} bias")
            assert np.abs(y - orc.round_bf16(p16 + bb)).max() <= 2 * bf16_ulp(np.abs(p16 + bb).max())
            # residual
            y = to_np(Linear(wg, device=dev)(xg, residual=to_gpu_bf16(res, torch)))
            ref = orc.round_bf16(p16 + rb)
            assert_parity(y, ref, f"{name} residual")
            assert np.abs(y - ref).max() <= 2 * bf16_ulp(np.abs(ref).max())
            # bias + residual
            y = to_np(Linear(wg, to_gpu_bf16(bias, torch), device=dev)(xg, residual=to_gpu_bf16(res, torch)))
            assert_parity(y, orc.round_bf16(orc.round_bf16(p16 + bb) + rb), f"{name} bias+residual")
            # bias + gelu (Laya scorer_in)
            y = to_np(Linear(wg, to_gpu_bf16(bias, torch), device=dev)(xg, gelu=True))
            assert_parity(y, orc.round_bf16(orc.gelu_erf(orc.round_bf16(p16 + bb))), f"{name} bias+gelu")
            # bias + tanh-approximate gelu (the vision tower's fc1)
            y = to_np(Linear(wg, to_gpu_bf16(bias, torch), device=dev)(xg, gelu="tanh"))
            assert_parity(y, orc.round_bf16(orc.gelu_tanh(orc.round_bf16(p16 + bb))), f"{name} bias+gelu_tanh")
            if not gated_ok:
                continue
            # gated: GeGLU and SwiGLU over [2I, K] = [gate; up], I = N/2
            I = N // 2
            g16, u16 = p16[:, :I], p16[:, I:]
            ref_geglu = orc.round_bf16(orc.round_bf16(orc.gelu_erf(g16)) * u16)
            ref_swiglu = orc.round_bf16(orc.round_bf16(orc.silu(g16)) * u16)
            y = to_np(GatedLinear(wg, "gelu", device=dev)(xg))
            assert y.shape == (M, I)
            assert_parity(y, ref_geglu, f"{name} geglu")
            # unfused f32 reference (src/archs/modernbert.rs:531-532 on f32 tensors)
            assert_parity(y, orc.geglu(orc.linear_f32(x, w)), f"{name} geglu vs f32")
            y = to_np(GatedLinear(wg, "silu", device=dev)(xg))
            assert_parity(y, ref_swiglu, f"{name} swiglu")
            assert_parity(y, orc.swiglu(*np.split(orc.linear_f32(x, w), 2, axis=1)), f"{name} swiglu vs f32")
    finally:
        dev.set_kernel(-1)


def test_strided_input_and_output(dev, orc):
    """x as a column slice of a wider buffer (the V block of a qkv output) and
    y written into a slice of a wider buffer."""
    from sys1_amd.linear import Linear
    M, H = 200, 256
    qkv = orc.fill_normal((M, 3 * H), 21)
    w = orc.fill_normal((H, H), 22, 0.02)
    qkv_g = to_gpu_bf16(qkv, torch)
    out = torch.zeros(M, 2 * H, dtype=torch.bfloat16, device="cuda:0")
    Linear(to_gpu_bf16(w, torch), device=dev).forward_into(qkv_g[:, 2 * H:], out[:, H:])
    y = to_np(out)
    assert (y[:, :H] == 0).all()
    assert_parity(y[:, H:], orc.linear_f32(qkv[:, 2 * H:], w), "strided")


def test_leading_dims_flatten_and_empty(dev, orc):
    from sys1_amd.linear import Linear
    w = to_gpu_bf16(orc.fill_normal((64, 32), 1, 0.02), torch)
    lin = Linear(w, device=dev)
    x = orc.fill_normal((2, 5, 32), 2)
    y = lin(to_gpu_bf16(x, torch))
    assert y.shape == (2, 5, 64)
    assert_parity(to_np(y).reshape(10, 64), orc.linear_f32(x.reshape(10, 32), orc.round_bf16(orc.fill_normal((64, 32), 1, 0.02))), "3d")
    e = lin(torch.empty(0, 32, dtype=torch.bfloat16, device="cuda:0"))
    assert e.shape == (0, 64)


def test_tiny_output_width(dev, orc):
    """N = 1 (the Laya scorer's last projection, src/models/laya.rs:516) with bias."""
    from sys1_amd.linear import Linear
    M, K = 37, 768
    x = orc.fill_normal((M, K), 5)
    w = orc.fill_normal((1, K), 6, 0.02)
    b = orc.fill_normal((1,), 7)
    y = to_np(Linear(to_gpu_bf16(w, torch), to_gpu_bf16(b, torch), device=dev)(to_gpu_bf16(x, torch)))
    assert y.shape == (M, 1)
    assert_parity(y, orc.linear_f32(x, w, b), "N=1")


def test_stream_k_is_deterministic_and_rearms(dev, orc):
    """Stream-K partial tiles are reduced in workgroup order: repeated calls
    are bit-identical, every forced grid agrees with the oracle, and the
    tile counters re-arm between calls of different shapes."""
    from sys1_amd.linear import Linear
    outs = []
    for (M, N, K) in [(64, 1024, 4096), (32, 768, 2048), (64, 1024, 4096), (200, 4096, 2048),
                      (128, 520, 1000)]:
        _, name = dev.query_kernel(M, N, K)
        print(f"[gpu] stream-k M={M} N={N} K={K} {name}", flush=True)
        x, w = _inputs(orc, M, N, K, 50 + M + N)
        y = to_np(Linear(to_gpu_bf16(w, torch), device=dev)(to_gpu_bf16(x, torch)))
        assert_parity(y, orc.linear_f32(x, w), f"stream-k {M}x{N}x{K}")
        outs.append(y)
    np.testing.assert_array_equal(outs[0], outs[2])
    # forced grid sizes on a stream-K kernel: every head/tail/fix-up pattern
    from sys1_amd import kernel_names
    kid = kernel_names().index("stream_64x256_s3_w2x4")
    M, N, K = 50, 700, 1024
    x, w = _inputs(orc, M, N, K, 77)
    ref = orc.linear_f32(x, w)
    dev.set_kernel(kid)
    try:
        prev = None
        for g in (1, 2, 3, 5, 7, 16, 48, 1000):
            dev.set_grid(g)
            print(f"[gpu] forced grid={g} {dev.query_kernel(M, N, K)[1]}", flush=True)
            y = to_np(Linear(to_gpu_bf16(w, torch), device=dev)(to_gpu_bf16(x, torch)))
            assert_parity(y, ref, f"grid={g}")
            if prev is not None:
                assert np.abs(y - prev).max() <= 2 * np.abs(ref).max() * 2 ** -8
            prev = y
            z = to_np(Linear(to_gpu_bf16(w, torch), device=dev)(to_gpu_bf16(x, torch)))
            np.testing.assert_array_equal(y, z)  # deterministic, counters re-armed
    finally:
        dev.set_grid(0)
        dev.set_kernel(-1)


@pytest.mark.parametrize("kname", ["stream_128x128_s4_w2x2_p4", "stream_128x256_s3_w2x4"])
def test_hybrid_tile_then_stream_phase(dev, orc, kname):
    """Stream-K kernels on large M: the first dp tiles run whole, the rest
    are split over every workgroup.  Every split (pure stream-K, one tile
    whole, half, all but one, all) and small grids (several tiles per
    workgroup in both phases) agree with the oracle, bit-identically across
    repeats."""
    from sys1_amd import kernel_names
    from sys1_amd.linear import GatedLinear, Linear
    M, N, K = 1000, 768, 328
    bm, bn = (int(v) for v in kname.split("_")[1].split("x"))
    tiles = -(-M // bm) * -(-N // bn)
    x, w = _inputs(orc, M, N, K, 31)
    xb, wb = orc.round_bf16(x), orc.round_bf16(w)
    proj = orc.linear_f64(xb, wb).astype(np.float32)
    p16 = orc.round_bf16(proj)
    res = orc.fill_normal((M, N), 5)
    ref_res = orc.round_bf16(p16 + orc.round_bf16(res))
    I = N // 2
    ref_geglu = orc.round_bf16(orc.round_bf16(orc.gelu_erf(p16[:, :I])) * p16[:, I:])
    xg, wg, rg = to_gpu_bf16(x, torch), to_gpu_bf16(w, torch), to_gpu_bf16(res, torch)
    lin, glu = Linear(wg, device=dev), GatedLinear(wg, "gelu", device=dev)
    dev.set_kernel(kernel_names().index(kname))
    try:
        for g in (3, 7, 40):
            dev.set_grid(g)
            for dp in sorted({0, 1, tiles // 2, tiles - 1, tiles}):
                dev.set_dp_tiles(dp)
                print(f"[gpu] hybrid {kname} grid={g} dp={dp} tiles={tiles} "
                      f"{dev.query_kernel(M, N, K)[1]}", flush=True)
                y = to_np(lin(xg))
                _check_close_to_rounded(orc, y, proj, f"{kname} g={g} dp={dp} none")
                np.testing.assert_array_equal(y, to_np(lin(xg)))
                y = to_np(lin(xg, residual=rg))
                assert np.abs(y - ref_res).max() <= 2 * bf16_ulp(np.abs(ref_res).max())
                y = to_np(glu(xg))
                assert_parity(y, ref_geglu, f"{kname} g={g} dp={dp} geglu")
    finally:
        dev.set_dp_tiles(-1)
        dev.set_grid(0)
        dev.set_kernel(-1)


def test_tile_kernel_small_forced_grid(dev, orc):
    """A persistent tile grid smaller than the 8 XCDs still covers every tile."""
    from sys1_amd import kernel_names
    from sys1_amd.linear import Linear
    M, N, K = 700, 640, 200
    x, w = _inputs(orc, M, N, K, 41)
    proj = orc.linear_f64(orc.round_bf16(x), orc.round_bf16(w)).astype(np.float32)
    lin = Linear(to_gpu_bf16(w, torch), device=dev)
    xg = to_gpu_bf16(x, torch)
    dev.set_kernel(kernel_names().index("tile_128x128_s2_w2x2"))
    try:
        for g in (1, 3, 8, 9, 13):
            dev.set_grid(g)
            print(f"[gpu] tile grid={g} {dev.query_kernel(M, N, K)[1]}", flush=True)
            _check_close_to_rounded(orc, to_np(lin(xg)), proj, f"tile grid={g}")
    finally:
        dev.set_grid(0)
        dev.set_kernel(-1)


@pytest.mark.parametrize("kname", [n for n in __import__("sys1_amd").kernel_names()
                                   if n.startswith("tile_")])
def test_tile_kernels_short_k_and_small_grids(dev, orc, kname):
    """Streams of 1..6 k-tiles per tile and 1..n tiles per workgroup: the
    pipeline prologue and refill cursors at every stream length."""
    from sys1_amd import kernel_names
    from sys1_amd.linear import Linear
    dev.set_kernel(kernel_names().index(kname))
    try:
        for K in (40, 72, 136, 328):
            M, N = 520, 520
            x, w = _inputs(orc, M, N, K, 43 + K)
            proj = orc.linear_f64(orc.round_bf16(x), orc.round_bf16(w)).astype(np.float32)
            lin = Linear(to_gpu_bf16(w, torch), device=dev)
            xg = to_gpu_bf16(x, torch)
            for g in (0, 1, 3, 9):
                dev.set_grid(g)
                print(f"[gpu] {kname} K={K} grid={g} {dev.query_kernel(M, N, K)[1]}", flush=True)
                _check_close_to_rounded(orc, to_np(lin(xg)), proj, f"{kname} K={K} grid={g}")
    finally:
        dev.set_grid(0)
        dev.set_kernel(-1)


@pytest.mark.parametrize("kname", ["tile_128x96_s2_w4x1_p4", "tile_128x192_s3_w4x2_p4"])
def test_residual_staged_in_lds_ragged_and_multi_tile(dev, orc, kname):
    """The 128x96 producer-wave kernel copies each tile's residual block into
    LDS during the tile's k-loop; the 128x192 one, the other residual shape,
    reads it from HBM in the epilogue.  Ragged N (the last tile's columns
    clamped), N not a multiple of 8 and K within one k-tile (both read the
    residual from HBM on the 128x96 kernel too), K of two k-tiles, and small
    grids (several tiles per workgroup, each re-staging its block) must all
    match bf16(bf16(x.W) + r)."""
    from sys1_amd import kernel_names
    from sys1_amd.linear import Linear
    dev.set_kernel(kernel_names().index(kname))
    try:
        for M, N, K in ((333, 776, 200), (333, 770, 200), (300, 384, 64), (300, 384, 128), (700, 384, 328)):
            x, w = _inputs(orc, M, N, K, 71 + N + K)
            proj = orc.round_bf16(orc.linear_f64(orc.round_bf16(x), orc.round_bf16(w)).astype(np.float32))
            res = orc.round_bf16(orc.fill_normal((M, N), 73))
            ref = orc.round_bf16(proj + res)
            lin = Linear(to_gpu_bf16(w, torch), device=dev)
            xg, rg = to_gpu_bf16(x, torch), to_gpu_bf16(res, torch)
            for g in (0, 1, 3, 7):
                dev.set_grid(g)
                print(f"[gpu] {kname} residual M={M} N={N} K={K} grid={g}", flush=True)
                assert_parity(to_np(lin(xg, residual=rg)), ref, f"M={M} N={N} K={K} grid={g}")
    finally:
        dev.set_grid(0)
        dev.set_kernel(-1)


def test_plan_cache_and_forcing(dev, orc):
    """The chosen plan is cached per (M, N, K, epilogue).  A forced kernel or
    grid bypasses the cache (the forced choice is reported and run), and
    clearing the force returns the cached automatic choice.  Every call's
    result matches the oracle, and repeated queries of several M return the
    same choice as the first."""
    from sys1_amd import kernel_names
    from sys1_amd.linear import Linear
    M, N, K = 300, 1024, 512
    x, w = _inputs(orc, M, N, K, 91)
    ref = orc.round_bf16(orc.linear_f64(orc.round_bf16(x), orc.round_bf16(w)).astype(np.float32))
    lin = Linear(to_gpu_bf16(w, torch), device=dev)
    xg = to_gpu_bf16(x, torch)
    auto = dev.query_kernel(M, N, K)
    assert_parity(to_np(lin(xg)), ref, "auto")
    assert dev.query_kernel(M, N, K) == auto
    other = next(i for i, n in enumerate(kernel_names()) if i != auto[0] and n.startswith("tile_"))
    try:
        dev.set_kernel(other)
        assert dev.query_kernel(M, N, K)[0] == other
        assert_parity(to_np(lin(xg)), ref, f"forced {kernel_names()[other]}")
        dev.set_kernel(-1)
        dev.set_grid(3)
        assert "_g3" in dev.query_kernel(M, N, K)[1]
        assert_parity(to_np(lin(xg)), ref, "forced grid 3")
    finally:
        dev.set_kernel(-1)
        dev.set_grid(0)
    assert dev.query_kernel(M, N, K) == auto
    assert_parity(to_np(lin(xg)), ref, "auto again")
    picks = {m: dev.query_kernel(m, N, K) for m in (1, 64, 128, 256, 1024, 8192)}
    for m, p in picks.items():
        assert dev.query_kernel(m, N, K) == p


def test_gelu_every_bf16_input(dev, orc):
    """The GeGLU epilogue's GELU over every finite bf16 gate value (the gate is
    the bf16-rounded projection, so these are all the inputs it can see),
    against the reference's f32 sequence 0.5 v (1 + erf(v / sqrt 2)) with a
    correctly rounded f32 erf, each result rounded to bf16: a projection with
    an identity gate block and an up block that reads a column of ones makes
    the output exactly bf16(gelu(v)).  At most 0.1% may differ, by one bf16
    ulp (the hardware exponential and reciprocal inside erfc)."""
    import math
    from sys1_amd.linear import GatedLinear
    bits = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    v = bits[np.isfinite(bits)]
    v = np.concatenate([v, np.zeros((-v.size) % 64, np.float32)])
    M = v.size // 64
    x = np.zeros((M, 128), np.float32)
    x[:, :64] = v.reshape(M, 64)
    x[:, 64] = 1.0
    gate = np.zeros((64, 128), np.float32)
    gate[:, :64] = np.eye(64, dtype=np.float32)
    up = np.zeros((64, 128), np.float32)
    up[:, 64] = 1.0
    lin = GatedLinear(gate=to_gpu_bf16(gate, torch), up=to_gpu_bf16(up, torch), activation="gelu", device=dev)
    print(f"[gpu] gelu over {v.size} bf16 values", flush=True)
    y = to_np(lin(to_gpu_bf16(x, torch))).reshape(-1)
    erf32 = np.array([math.erf(float(a) / math.sqrt(2.0)) for a in v], np.float64).astype(np.float32)
    ref = orc.round_bf16((np.float32(0.5) * v * (np.float32(1.0) + erf32)).astype(np.float32))
    diff = (y != ref) & ~((y == 0) & (ref == 0))
    print(f"[gpu]   {int(diff.sum())} of {v.size} differ", flush=True)
    assert diff.mean() <= 1e-3, f"{int(diff.sum())} of {v.size} differ"
    if diff.any():
        assert (np.abs(y[diff] - ref[diff]) <= bf16_ulp(ref[diff]) + 1e-30).all()



def test_gelu_tanh_every_bf16_input(dev, orc):
    """The bias + tanh-GELU epilogue over every finite bf16 value (the value
    the activation sees is the bf16-rounded biased projection): a projection
    with an identity weight block and a zero bias makes the output exactly
    bf16(gelu_tanh(v)).  Against the oracle (float64, correctly rounded to
    f32, then bf16): at most 0.1% may differ, by one bf16 ulp (the hardware
    exponential and reciprocal)."""
    from sys1_amd.linear import Linear
    bits = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    v = bits[np.isfinite(bits)]
    v = np.concatenate([v, np.zeros((-v.size) % 64, np.float32)])
    M = v.size // 64
    x = np.zeros((M, 64), np.float32)
    x[:, :64] = v.reshape(M, 64)
    w = np.eye(64, dtype=np.float32)
    lin = Linear(to_gpu_bf16(w, torch), torch.zeros(64, dtype=torch.bfloat16, device="cuda"), device=dev)
    print(f"[gpu] gelu_tanh over {v.size} bf16 values", flush=True)
    y = to_np(lin(to_gpu_bf16(x, torch), gelu="tanh")).reshape(-1)
    ref = orc.round_bf16(orc.gelu_tanh(v))
    diff = (y != ref) & ~((y == 0) & (ref == 0)) & ~(np.isnan(y) & np.isnan(ref))
    print(f"[gpu]   {int(diff.sum())} of {v.size} differ", flush=True)
    assert diff.mean() <= 1e-3, f"{int(diff.sum())} of {v.size} differ"
    if diff.any():
        assert (np.abs(y[diff] - ref[diff]) <= bf16_ulp(ref[diff]) + 1e-30).all()

def test_silu_every_bf16_input(dev, orc):
    """The SwiGLU epilogue's SiLU over every finite bf16 gate value, against
    the f32 sequence v / (1 + exp(-v)) with a correctly rounded exp and
    division, rounded to bf16 (the same identity-gate construction as the
    GELU test).  At most 0.1% may differ, by one bf16 ulp (the hardware
    exponential and reciprocal)."""
    import math
    from sys1_amd.linear import GatedLinear
    bits = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    v = bits[np.isfinite(bits)]
    v = np.concatenate([v, np.zeros((-v.size) % 64, np.float32)])
    M = v.size // 64
    x = np.zeros((M, 128), np.float32)
    x[:, :64] = v.reshape(M, 64)
    x[:, 64] = 1.0
    gate = np.zeros((64, 128), np.float32)
    gate[:, :64] = np.eye(64, dtype=np.float32)
    up = np.zeros((64, 128), np.float32)
    up[:, 64] = 1.0
    lin = GatedLinear(gate=to_gpu_bf16(gate, torch), up=to_gpu_bf16(up, torch), activation="silu", device=dev)
    print(f"[gpu] silu over {v.size} bf16 values", flush=True)
    y = to_np(lin(to_gpu_bf16(x, torch))).reshape(-1)
    with np.errstate(over="ignore"):
        e32 = np.array([math.exp(min(-float(a), 700.0)) for a in v], np.float64).astype(np.float32)
        den = (np.float32(1.0) + e32).astype(np.float32)
        ref = orc.round_bf16((v.astype(np.float64) / den.astype(np.float64)).astype(np.float32))
    diff = (y != ref) & ~((y == 0) & (ref == 0))
    print(f"[gpu]   {int(diff.sum())} of {v.size} differ", flush=True)
    assert diff.mean() <= 1e-3, f"{int(diff.sum())} of {v.size} differ"
    if diff.any():
        assert (np.abs(y[diff] - ref[diff]) <= bf16_ulp(ref[diff]) + 1e-30).all()


def test_python_errors(dev, orc):
    from sys1_amd import Sys1HipError
    from sys1_amd.linear import GatedLinear, Linear
    w = torch.zeros(64, 64, dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(ValueError):
        Linear(w.float(), device=dev)
    lin = Linear(w, device=dev)
    with pytest.raises(ValueError):
        lin(torch.zeros(4, 32, dtype=torch.bfloat16, device="cuda:0"))
    with pytest.raises(ValueError):
        lin(torch.zeros(4, 64, dtype=torch.float32, device="cuda:0"))
    big = torch.zeros(4, 72, dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(Sys1HipError) as e:
        lin(big[:, 1:65])  # 2-byte offset: misaligned rows
    assert e.value.code == -14
    with pytest.raises(ValueError):
        GatedLinear(torch.zeros(80, 64, dtype=torch.bfloat16, device="cuda:0"), device=dev)


@pytest.mark.parametrize("kname", [n for n in __import__("sys1_amd").kernel_names()
                                   if n.startswith("skinny_")])
def test_skinny_kernels_ragged_shapes(dev, orc, kname):
    """The skinny-M kernels: K split over the waves with empty, one-step and
    tail (K % 32 != 0) ranges, N not a multiple of the tile width (the last
    tile's weight rows clamped, its columns stored element by element), M
    within one tile row and over several with a ragged last one, and
    repeated calls bit-identical (the waves' partials are summed in a fixed
    order)."""
    from sys1_amd import kernel_names
    from sys1_amd.linear import GatedLinear, Linear
    cap = int(kname.split("_")[1].split("x")[0])
    gated = int(kname.split("_")[1].split("x")[1]) % 32 == 0
    dev.set_kernel(kernel_names().index(kname))
    try:
        for (M, N, K) in [(1, 1, 40), (cap, 17, 72), (max(1, cap - 5), 520, 136), (cap, 1000, 1000),
                          (min(cap, 7), 48, 4104), (cap, 64, 8), (2 * cap + 5, 200, 328)]:
            print(f"[gpu] {kname} M={M} N={N} K={K}", flush=True)
            x, w = _inputs(orc, M, N, K, 91 + M + K)
            proj = orc.linear_f64(orc.round_bf16(x), orc.round_bf16(w)).astype(np.float32)
            lin = Linear(to_gpu_bf16(w, torch), device=dev)
            xg = to_gpu_bf16(x, torch)
            y = to_np(lin(xg))
            _check_close_to_rounded(orc, y, proj, f"{kname} M={M} N={N} K={K}")
            np.testing.assert_array_equal(y, to_np(lin(xg)))
            if gated and N % 32 == 0:
                p16 = orc.round_bf16(proj)
                I = N // 2
                ref = orc.round_bf16(orc.round_bf16(orc.silu(p16[:, :I])) * p16[:, I:])
                assert_parity(to_np(GatedLinear(to_gpu_bf16(w, torch), "silu", device=dev)(xg)), ref,
                              f"{kname} swiglu M={M} N={N} K={K}")
    finally:
        dev.set_kernel(-1)


def test_stream_switch_waits_for_the_old_stream(dev, orc):
    """sys1hip_set_stream (via HipDevice.follow_torch_stream) makes the new
    stream wait for the work queued on the old one: the context's workspace
    and counters are shared by all its calls.  A long spin queued on stream
    A holds back work queued on stream B after the switch."""
    from sys1_amd.linear import Linear
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    x, w = _inputs(orc, 64, 256, 256, 3)
    lin = Linear(to_gpu_bf16(w, torch), device=dev)
    xg = to_gpu_bf16(x, torch)
    torch.cuda.synchronize()
    try:
        with torch.cuda.stream(a):
            dev.follow_torch_stream()
            torch.cuda._sleep(200_000_000)  # ~0.1 s of spinning on A
            ya = lin(xg)
        with torch.cuda.stream(b):
            dev.follow_torch_stream()  # the switch: B waits for A's queue
            yb = lin(xg)
            done = torch.cuda.Event()
            done.record(b)
        print(f"[gpu] stream switch: B done before A's spin ended: {done.query()}", flush=True)
        assert not done.query(), "work on the new stream ran before the old stream's queue"
        torch.cuda.synchronize()
        assert done.query()
        assert torch.equal(ya, yb)
    finally:
        torch.cuda.synchronize()
        dev.follow_torch_stream()


def test_blocked_weight_layout_is_bitwise_row_major(dev, orc):
    """A weight in the blocked layout (pack_blocked_weight: 32-row x 64-k
    blocks, rows and K zero-padded) gives the row-major weight's results bit
    for bit on every kernel (the same values reach the same LDS and register
    positions): plain, residual and gated epilogues, N and K not multiples
    of the block, tile, stream-K and skinny plans."""
    from sys1_amd import kernel_names
    from sys1_amd.linear import GatedLinear, Linear
    names = kernel_names()
    try:
        for kid, name in enumerate(names):
            Ms = [70] if name.startswith(("stream_", "skinny_")) else [300]
            for M in Ms:
                for (N, K) in [(200, 328), (96, 1000)]:
                    print(f"[gpu] blocked {name} M={M} N={N} K={K}", flush=True)
                    x, w = _inputs(orc, M, N, K, 61 + N)
                    xg, wg = to_gpu_bf16(x, torch), to_gpu_bf16(w, torch)
                    res = to_gpu_bf16(orc.fill_normal((M, N), 62), torch)
                    dev.set_kernel(kid)
                    rm, bl = Linear(wg, device=dev), Linear(wg, device=dev, blocked=True)
                    assert torch.equal(rm(xg), bl(xg)), f"{name} none"
                    assert torch.equal(rm(xg, residual=res), bl(xg, residual=res)), f"{name} residual"
                    gated = not name.startswith("skinny_") or int(name.split("_")[1].split("x")[1]) % 32 == 0
                    if gated and N % 32 == 0:
                        g_rm = GatedLinear(wg, "silu", device=dev)
                        g_bl = GatedLinear(wg, "silu", device=dev, blocked=True)
                        assert torch.equal(g_rm(xg), g_bl(xg)), f"{name} swiglu"
    finally:
        dev.set_kernel(-1)
