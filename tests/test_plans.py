"""Host-side checks of the kernel chooser, without a device
(sys1hip_plan_kernel prices the plans with the shapes' fitted occupancies).

The first test pins the plans that the committed GPU measurements ran:
- the ModernBERT-base chain (profiles/gemm_tile_256x160_p4_modernbert-base_kernel-trace.md);
- the bench line's small-M object at M = 64 and 256
  (profiles/skinny_modernbert-large_m64-m256_kernel-trace.md);
- the Qwen3.5-27B weight stream at M = 128
  (profiles/gemm_weight-stream_qwen35-27b-m128_kernel-trace.md);
- the skinny kernels' per-CU byte limit, both sides of it
  (profiles/gemm_modernbert-large_m1024-m4096_kernel-sweep.md);
- the plans that the forced-kernel sweeps moved
  (profiles/gemm_all-workloads_forced-kernel-sweep.md).

A change of the cost model that moves them shows here first.  The rest are
invariants over every projection shape of the four configurations and a
sweep of packed M."""
import re

import pytest

from sys1_amd import _lib
from sys1_amd.stacks import CONFIGS

E = _lib


@pytest.mark.parametrize("M,N,K,epi,plan", [
    # ModernBERT-base at the bench's mean ragged M
    (8019, 2304, 768, E.EPI_NONE, "tile_256x160_s3_w8x1_p4_g256"),
    (8019, 768, 768, E.EPI_RESIDUAL, "tile_128x192_s3_w4x2_p4_g252"),
    (8019, 2304, 768, E.EPI_GEGLU, "tile_256x160_s3_w8x1_p4_g256"),
    (8019, 768, 1152, E.EPI_RESIDUAL, "tile_128x192_s3_w4x2_p4_g252"),
    # ModernBERT-large, small M: the skinny kernels
    (64, 3072, 1024, E.EPI_NONE, "skinny_32x32_w16_g192"),
    (64, 1024, 1024, E.EPI_RESIDUAL, "skinny_16x16_w16_g256"),
    (64, 5248, 1024, E.EPI_GEGLU, "skinny_64x32_w16_g164"),
    (64, 1024, 2624, E.EPI_RESIDUAL, "skinny_16x16_w16_g256"),
    (256, 3072, 1024, E.EPI_NONE, "skinny_64x48_w8_g256"),
    (256, 1024, 1024, E.EPI_RESIDUAL, "skinny_32x32_w16_g256"),
    (256, 5248, 1024, E.EPI_GEGLU, "skinny_128x64_w4_g164"),
    (256, 1024, 2624, E.EPI_RESIDUAL, "skinny_32x32_w16_g256"),
    # one round of skinny tiles up to 704 KB per CU (same-box A/B against the
    # stream-K plans they replaced)
    (1024, 1024, 2624, E.EPI_RESIDUAL, "skinny_64x64_w8_g256"),
    (64, 2048, 6144, E.EPI_RESIDUAL, "skinny_32x16_w16_g256"),
    (128, 1152, 4304, E.EPI_BIAS | E.EPI_RESIDUAL, "skinny_32x32_w16_g144"),
    # ... and not beyond it
    (128, 2048, 6144, E.EPI_RESIDUAL, "stream_128x128_s4_w2x2_p4_g80"),
    # the 256x192 two-stage shape past the L2: its long-K rate from K > 1536
    # once x exceeds 4 MB (same-box A/B), not at M = 1024 (x L2-resident)
    (8192, 4608, 2048, E.EPI_NONE, "tile_256x160_s3_w8x1_p4_g256"),
    (2048, 12288, 2048, E.EPI_SWIGLU, "tile_256x128_s3_w2x2_p4_g256"),
    (1024, 12288, 2048, E.EPI_SWIGLU, "tile_256x192_s2_w4x2_p4_g256"),
    # the 256x192 two-stage shape priced at 0.60 (0.75 with SwiGLU) after the
    # forced-kernel sweeps (profiles/gemm_all-workloads_forced-kernel-sweep.md)
    (16384, 5248, 1024, E.EPI_GEGLU, "tile_256x160_s3_w8x1_p4_g256"),
    (4096, 3072, 1024, E.EPI_NONE, "tile_128x192_s3_w4x2_p4_g256"),
    (2048, 5248, 1024, E.EPI_GEGLU, "tile_128x192_s3_w4x2_p4_g256"),
    # one round of whole 128x192 tiles over the large stream-K shapes at long K
    (1024, 5120, 17408, E.EPI_RESIDUAL, "tile_128x192_s3_w4x2_p4_g216"),
    # Qwen3.5-27B at M = 128: weights streamed from HBM on the full stream-K grid
    (128, 34816, 5120, E.EPI_SWIGLU, "tile_128x160_s3_w4x1_p4_g218"),
    (128, 5120, 17408, E.EPI_RESIDUAL, "stream_128x128_s4_w2x2_p4_g256"),
    (128, 16480, 5120, E.EPI_NONE, "stream_128x128_s4_w2x2_p4_g256"),
    # a 63 MB weight over several row panels: 128-row stream-K panels, not
    # nine 32-row ones that walk the weight nine times (out_proj / o_proj)
    (272, 5120, 6144, E.EPI_RESIDUAL, "stream_128x128_s4_w2x2_p4_g256"),
    (288, 5120, 6144, E.EPI_RESIDUAL, "stream_128x128_s4_w2x2_p4_g256"),
    # a 178 MB weight (beyond half the MALL): 256-row panels walk it half as
    # often as 128-row ones (down); the 63 MB out_proj keeps 128-row panels
    (512, 5120, 17408, E.EPI_RESIDUAL, "stream_256x128_s3_w4x2_g256"),
    (768, 5120, 17408, E.EPI_RESIDUAL, "stream_256x128_s3_w4x2_g256"),
    (512, 5120, 6144, E.EPI_RESIDUAL, "stream_128x128_s4_w2x2_p4_g256"),
    # SwiGLU at 272-896 tokens: not 128x128 tiles at two per CU
    (384, 34816, 5120, E.EPI_SWIGLU, "tile_256x160_s3_w8x1_p4_g256"),
    (640, 34816, 5120, E.EPI_SWIGLU, "tile_256x160_s3_w8x1_p4_g256"),
    (896, 34816, 5120, E.EPI_SWIGLU, "tile_128x192_s3_w4x2_p4_g256"),
    # small weights stay in the caches: 32-row panels remain the pick at a
    # few panels, 128-row ones take over as the walks add up
    (256, 2048, 6144, E.EPI_RESIDUAL, "stream_32x256_s4_w1x4_p4_g256"),
    (576, 2048, 6144, E.EPI_RESIDUAL, "stream_128x128_s4_w2x2_p4_g256"),
    (960, 2048, 4096, E.EPI_RESIDUAL, "stream_128x128_s4_w2x2_p4_g256"),
])
def test_plans_of_the_measured_workloads(M, N, K, epi, plan):
    kid, grid, name = _lib.plan_kernel(M, N, K, epi)
    assert name == plan
    assert _lib.kernel_names()[kid] == re.sub(r"_g\d+(_dp\d+)?$", "", name)
    assert grid == int(re.search(r"_g(\d+)", name).group(1))


def _tile(name):
    m = re.match(r"(tile|stream|skinny)_(\d+)x(\d+)_", name)
    return m.group(1), int(m.group(2)), int(m.group(3))


def _cdiv(a, b):
    return -(-a // b)


def _shapes():
    out = set()
    for make in CONFIGS.values():
        for layer in make().layers:
            for p in layer:
                out.add((p.N, p.K, p.epi))
    return sorted(out)


MS = [1, 7, 16, 64, 100, 128, 129, 256, 300, 1000, 1024, 4096, 4097, 8192, 16384]


@pytest.mark.parametrize("N,K,epi", _shapes())
def test_plan_invariants_over_m(N, K, epi):
    """For every projection shape of the four configurations and a sweep of
    M: the plan exists, its grid fits its schedule, and each family is used
    in its regime (the chooser's documented rules)."""
    names = _lib.kernel_names()
    weight_bytes = 2 * N * K
    for M in MS:
        kid, grid, name = _lib.plan_kernel(M, N, K, epi)
        kind, bm, bn = _tile(names[kid])
        tiles = _cdiv(M, bm) * _cdiv(N, bn)
        assert grid >= 1, (M, name)
        if kind == "skinny":
            # one workgroup per tile, one round over the CUs, small weights only
            assert grid == tiles <= 256, (M, name)
            assert M <= 4096 and weight_bytes <= 32 << 20, (M, name)
        elif kind == "tile":
            # a persistent tile grid: no more workgroups than tiles or slots;
            # up to 128 tokens only as one round of whole tiles covering M in
            # one tile row, over at least two thirds of the CUs (no split
            # tile to fix up after the weight stream)
            assert M > 128 or (64 < M <= bm and 2 * 256 <= 3 * tiles <= 3 * 256), (M, name)
            assert grid <= tiles and grid <= 512, (M, name)
        else:
            # stream-K: at most one workgroup per (tile, k-tile) iteration
            assert grid <= min(512, tiles * _cdiv(K, 64)), (M, name)
        if epi in (E.EPI_GEGLU, E.EPI_SWIGLU) and kind == "skinny":
            assert bn % 32 == 0, (M, name)  # whole gate/up row groups per workgroup


def test_plans_follow_the_cu_count():
    """Fewer CUs, no wider grid; the plan is deterministic."""
    for M, N, K, epi in [(8019, 2304, 768, E.EPI_NONE), (128, 34816, 5120, E.EPI_SWIGLU),
                         (64, 3072, 1024, E.EPI_NONE)]:
        full = _lib.plan_kernel(M, N, K, epi, cus=256)
        assert _lib.plan_kernel(M, N, K, epi, cus=256) == full
        kid, grid, name = _lib.plan_kernel(M, N, K, epi, cus=64)
        kind, bm, bn = _tile(_lib.kernel_names()[kid])
        if kind != "skinny":
            assert grid <= 64 * 2, name
        else:
            assert grid <= 64, name


@pytest.mark.parametrize("args", [
    (0, 64, 64, 64, 0),          # no CUs
    (256, 0, 64, 64, 0),         # empty M (the linear call itself is a no-op; a plan is refused)
    (256, 64, 64, -1, 0),        # bad K
    (256, 64, 64, 64, 3),        # GeGLU | bias is not an epilogue
    (256, 64, 48, 64, E.EPI_GEGLU),  # gated N not a multiple of 32
])
def test_plan_kernel_rejects_bad_arguments(args):
    L = _lib.load()
    assert L.sys1hip_plan_kernel(*args, None, None, 0) == _lib.EINVAL
    assert L.sys1hip_last_error(None)


def test_strided_x_beyond_2gib_rules_out_the_skinny_kernels():
    """The skinny kernels address x from row 0 with 32-bit byte offsets: an x
    view whose rows span 2 GiB or more (a large leading dimension) must get
    a tile or stream-K plan, and so must a weight that wide; the same shape
    with contiguous rows stays skinny."""
    M, N, K = 64, 1024, 1024
    _, _, plain = E.plan_kernel(M, N, K, E.EPI_NONE)
    assert plain.startswith("skinny_")
    ldx = (1 << 31) // (2 * (M - 1)) + 8  # 2 (M-1) ldx >= 2 GiB
    _, _, wide = E.plan_kernel(M, N, K, E.EPI_NONE, ldx=ldx)
    assert not wide.startswith("skinny_"), wide
    _, _, just = E.plan_kernel(M, N, K, E.EPI_NONE, ldx=(0x7ffffff0 - 2 * K) // (2 * (M - 1)) - 8)
    assert just.startswith("skinny_"), just
    _, _, wide_w = E.plan_kernel(M, N, K, E.EPI_NONE, ldw=(1 << 31) // (2 * N) + 8)
    assert not wide_w.startswith("skinny_"), wide_w
