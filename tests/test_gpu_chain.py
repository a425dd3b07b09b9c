"""GPU parity of the projection chain (sys1hip_linear_chain_bf16): several
row-local projections of a layer in one persistent launch, with per-row-panel
dependencies between them (src/archs/modernbert.rs:857-887: attn.Wo ->
Wi+GeGLU -> mlp.Wo -> next Wqkv; src/archs/qwen35_text.rs:932-940).

  - bit for bit the per-projection calls on the same tile kernel (the chain's
    128 x 192 tile: same operands, same k order, same epilogue rounding), at
    token counts from 65 to a config-2 ragged batch (64 and fewer run the
    weight-streaming chain, checked against the oracle at the end), on the ModernBERT-base and
    Qwen3.5-small shapes (partial row panels, a partial column tile);
  - every output of one chain launch against the oracle's f32 projections
    (relative Frobenius <= 1e-2, max-abs <= 2e-2 max|ref|);
  - the whole 22-layer stack with chains (the bench's object) against the
    per-projection stack, and its final state against the oracle chain;
  - the bounded dependency wait: forced to expire from the host, the launch
    still finishes and reports it, and the next launch is correct;
  - replays of a captured graph of chain launches equal the eager result.
Every launch's error word (sys1hip_chain_status) must read 0 unless the test
forces a wait to expire.
"""
import ctypes

import numpy as np
import pytest

from gpu_helpers import assert_parity, parity, to_gpu_bf16, to_np

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

CHAIN_TILE = "tile_128x192_s3_w4x2_p4"


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from sys1_amd.device import HipDevice
    d = HipDevice(0)
    yield d
    d.set_kernel(-1)
    d.set_chain_wait()


def _tile_id():
    from sys1_amd import kernel_names
    return kernel_names().index(CHAIN_TILE)


def _stacks(dev, cfg, M, ws, blocked=True):
    from sys1_amd.stacks import ProjectionStack
    a = ProjectionStack(cfg, dev, M, weights=ws, blocked=blocked, chain=True)
    b = ProjectionStack(cfg, dev, M, weights=ws, blocked=blocked)
    return a, b


def _run_both(dev, a, b, x, M):
    """Chain stack, then the per-projection stack, with every single call
    (the chain stack's first Wqkv too) forced onto the chain's tile; returns
    every buffer of both (first M rows) as int16 bit patterns (a deep
    norm-free chain may overflow to inf/nan, which compare bit for bit)."""
    dev.set_kernel(_tile_id())
    try:
        out_a = a.forward(x, M)
        torch.cuda.synchronize()
        assert dev.chain_status() == 0
        ra = {k: v[:M].clone().view(torch.int16) for k, v in a.buffers.items()}
        b.forward(x, M)
        torch.cuda.synchronize()
    finally:
        dev.set_kernel(-1)
    rb = {k: v[:M].clone().view(torch.int16) for k, v in b.buffers.items()}
    return out_a, ra, rb


@pytest.mark.parametrize("M", [65, 100, 127, 128, 129, 1000, 3001])
def test_modernbert_chain_bitwise_per_projection(dev, orc, M):
    from sys1_amd.stacks import modernbert
    cfg = modernbert(768, 1152, 3, "modernbert-base-3")
    print(f"[gpu] chain modernbert-base 3 layers M={M}", flush=True)
    ws = [[(torch.randn(p.N, p.K, device="cuda") * 0.02).to(torch.bfloat16) for p in layer]
          for layer in cfg.layers]
    a, b = _stacks(dev, cfg, M, ws)
    launches = a.prepare(to_gpu_bf16(orc.fill_normal((M, 768), 1), torch), M)
    assert len(launches) == 1 + 3, [type(p) for p, _, _ in launches]  # Wqkv, then one chain per layer
    x = to_gpu_bf16(orc.fill_normal((M, 768), 2 + M), torch)
    _, ra, rb = _run_both(dev, a, b, x, M)
    for k in ra:
        assert torch.equal(ra[k], rb[k]), k


def test_modernbert_chain_cfg2_ragged_bitwise(dev, orc):
    """All 22 layers on a config-2 ragged batch (lengths U[16,512] packed to
    8192): the chain stack equals the per-projection stack on the chain's
    tile bit for bit, row-major and blocked weights."""
    from sys1_amd.batching import draw_lengths
    from sys1_amd.stacks import CONFIGS
    cfg = CONFIGS["modernbert-base"]()
    M = int(draw_lengths(21, 16, 512, 8192).sum())
    ws = [[(torch.randn(p.N, p.K, device="cuda") * 0.02).to(torch.bfloat16) for p in layer]
          for layer in cfg.layers]
    x = to_gpu_bf16(orc.fill_normal((M, 768), 5), torch)
    for blocked in (True, False):
        print(f"[gpu] chain modernbert-base 22 layers M={M} blocked={blocked}", flush=True)
        a, b = _stacks(dev, cfg, M, ws, blocked)
        _, ra, rb = _run_both(dev, a, b, x, M)
        for k in ra:
            assert torch.equal(ra[k], rb[k]), (k, blocked)


@pytest.mark.parametrize("M", [77, 1000])
def test_qwen_small_chain_bitwise_per_projection(dev, orc, M):
    """Qwen3.5-small shapes: out_proj (K 4096) -> gate_up+SwiGLU (N 12288) ->
    down (K 6144) -> next in_proj (N 12320: a partial last column tile), and
    the attention layer's o_proj -> ... -> next q_k_v."""
    from sys1_amd.stacks import CONFIGS, StackConfig
    full = CONFIGS["qwen35-small"]()
    cfg = StackConfig("qwen35-small-2", full.hidden, [full.layers[0], full.layers[3], full.layers[0]])
    print(f"[gpu] chain qwen35-small 3 layers M={M}", flush=True)
    ws = [[(torch.randn(p.N, p.K, device="cuda") * 0.02).to(torch.bfloat16) for p in layer]
          for layer in cfg.layers]
    a, b = _stacks(dev, cfg, M, ws)
    x = to_gpu_bf16(orc.fill_normal((M, full.hidden), 9), torch)
    _, ra, rb = _run_both(dev, a, b, x, M)
    for k in ra:
        assert torch.equal(ra[k], rb[k]), k


def _chain_launch(dev, projs, M):
    from sys1_amd import _lib
    arr = (_lib.ChainProj * len(projs))(*projs)
    dev.follow_torch_stream()
    _lib.check(dev._L.sys1hip_linear_chain_bf16(dev.ctx, arr, len(projs), M), dev.ctx)


def _cp(x, w, y, epi, res=None, K=None, N=None):
    from sys1_amd import _lib
    return _lib.ChainProj(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                          res.data_ptr() if res is not None else None, res.stride(0) if res is not None else 0,
                          y.data_ptr(), y.stride(0), N or w.shape[0], K or w.shape[1], epi)


@pytest.mark.parametrize("M", [1024, 4097])
def test_one_chain_launch_against_the_oracle(dev, orc, M):
    """attn.Wo(+residual) -> Wi+GeGLU -> mlp.Wo(+residual) -> Wqkv of
    ModernBERT-base in one launch (cfg 1: M = 1024): each output against the
    oracle's f32 projection of the inputs the GPU chain fed it."""
    from sys1_amd import _lib
    from sys1_amd.linear import pack_gated_weight
    H, I = 768, 1152
    qkv_np = orc.round_bf16(orc.fill_normal((M, 3 * H), 3))
    h0_np = orc.round_bf16(orc.fill_normal((M, H), 4))
    w = [orc.round_bf16(orc.fill_normal(s, 10 + i, 0.02))
         for i, s in enumerate([(H, H), (2 * I, H), (H, I), (3 * H, H)])]
    qkv = to_gpu_bf16(qkv_np, torch)
    h = to_gpu_bf16(h0_np, torch)
    act = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    wg = [to_gpu_bf16(v, torch) for v in w]
    wi_packed = pack_gated_weight(wg[1], dev)
    qkv_out = torch.empty(M, 3 * H, dtype=torch.bfloat16, device="cuda")
    v_block = qkv[:, 2 * H:]
    projs = [_cp(v_block, wg[0], h, _lib.EPI_RESIDUAL, res=h),
             _cp(h, wi_packed, act, _lib.EPI_GEGLU),
             _cp(act, wg[2], h, _lib.EPI_RESIDUAL, res=h),
             _cp(h, wg[3], qkv_out, _lib.EPI_NONE)]
    _chain_launch(dev, projs, M)
    torch.cuda.synchronize()
    assert dev.chain_status() == 0
    # oracle, each step from the GPU chain's own (bf16) intermediate values
    h1_ref = orc.linear_f32(np.ascontiguousarray(qkv_np[:, 2 * H:]), w[0]) + h0_np
    act_np = to_np(act)
    assert_parity(act_np, orc.geglu(orc.linear_f32(orc.round_bf16(h1_ref), w[1])), f"Wi+GeGLU M={M}")
    h2_np = to_np(h)
    h2_ref = orc.linear_f32(act_np, w[2]) + orc.round_bf16(h1_ref)
    assert_parity(h2_np, h2_ref, f"mlp.Wo M={M}")
    assert_parity(to_np(qkv_out), orc.linear_f32(h2_np, w[3]), f"Wqkv M={M}")


def test_bounded_wait_expires_cleanly_and_the_next_launch_is_correct(dev, orc):
    """With every dependency target raised out of reach (a host-side knob),
    the first wait gives up after its time limit and the others at once: the
    launch finishes, reports bit 1, and the bank is left clear, so the next
    normal launch matches the per-projection result bit for bit."""
    from sys1_amd.stacks import modernbert
    cfg = modernbert(768, 1152, 2, "modernbert-base-2")
    M = 700
    ws = [[(torch.randn(p.N, p.K, device="cuda") * 0.02).to(torch.bfloat16) for p in layer]
          for layer in cfg.layers]
    a, b = _stacks(dev, cfg, M, ws)
    x = to_gpu_bf16(orc.fill_normal((M, 768), 6), torch)
    dev.set_chain_wait(wait_us=200, extra=1 << 20)
    try:
        print("[gpu] chain with unreachable dependencies (bounded waits expire)", flush=True)
        a.forward(x, M, check=False)
        flags = dev.chain_status()
        # forward's own check raises on the same condition
        with pytest.raises(RuntimeError, match="dependency wait expired"):
            a.forward(x, M)
    finally:
        dev.set_chain_wait()
    print(f"[gpu]   status flags {flags}", flush=True)
    assert flags & 1
    assert dev.chain_status() == 0  # cleared by the read
    _, ra, rb = _run_both(dev, a, b, x, M)
    for k in ra:
        assert torch.equal(ra[k], rb[k]), k


def test_chain_launches_replay_in_a_graph(dev, orc):
    """A stack of chain launches captured in a HIP graph: four replays, with
    eager chain launches (sharing the dependency bank) between them, each
    equal to the eager result; the bank is cleared inside every launch, so
    no memset node is recorded."""
    from sys1_amd.stacks import modernbert
    cfg = modernbert(768, 1152, 2, "modernbert-base-2")
    M = 1500
    ws = [[(torch.randn(p.N, p.K, device="cuda") * 0.02).to(torch.bfloat16) for p in layer]
          for layer in cfg.layers]
    a, _ = _stacks(dev, cfg, M, ws)
    x = to_gpu_bf16(orc.fill_normal((M, 768), 8), torch)
    x2 = to_gpu_bf16(orc.fill_normal((M, 768), 9), torch)
    eager = a.forward(x, M).clone().view(torch.int16)
    torch.cuda.synchronize()
    prepared = a.prepare(x, M)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dev.follow_torch_stream()
        a.run_prepared(prepared)
    dev.follow_torch_stream()
    torch.cuda.synchronize()
    for r in range(4):
        a.buffers["h"].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(a.buffers["h"][:M, :768].view(torch.int16), eager), f"replay {r}"
        a.forward(x2, M)  # eager work on the same bank between replays
        torch.cuda.synchronize()
    assert dev.chain_status() == 0
    del g


def test_chain_stack_against_the_oracle_chain(dev, orc):
    """The bench's default object with chains (ProjectionStack(blocked=True,
    chain=True), 22 ModernBERT-base layers) on a config-2 ragged batch from
    the oracle's seeded weights: the final hidden state against the oracle
    chain that rounds where the GPU path rounds, relative to the spread
    between the oracle's f32 and bf16-rounding chains (the norm-free stack
    amplifies rounding differences layer over layer)."""
    from sys1_amd.batching import draw_lengths
    from sys1_amd.stacks import CONFIGS, ProjectionStack
    import test_gpu_stack as T
    cfg = CONFIGS["modernbert-base"]()
    M = int(draw_lengths(33, 16, 512, 8192).sum())
    print(f"[gpu] chain stack vs oracle chain M={M}", flush=True)
    x = orc.fill_normal((M, 768), 41)
    ws = T._weights(orc, cfg, 900)
    stack = ProjectionStack(cfg, dev, M, weights=[[to_gpu_bf16(w, torch) for w in l] for l in ws],
                            blocked=True, chain=True)
    out = to_np(stack.forward(to_gpu_bf16(x, torch), M))
    torch.cuda.synchronize()
    assert dev.chain_status() == 0
    emul = T._oracle_chain_bf16(orc, cfg, x, ws, None)
    f32 = T._oracle_chain(orc, cfg, x, ws, None)
    rel, _ = parity(out, emul)
    spread, _ = parity(emul, f32)
    print(f"[gpu]   final hidden vs bf16-rounding oracle chain {rel:.3e}; oracle chains differ by {spread:.3e}",
          flush=True)
    assert rel < 4 * spread


# ---- up to 64 tokens: the weight-streaming chain (32-column items over the
# whole K, K split over the waves, every CU) -- not the tile kernels' summation
# order, so checked against the oracle, not bit for bit.

@pytest.mark.parametrize("M", [1, 17, 64])
def test_weight_streaming_chain_launch_against_the_oracle(dev, orc, M):
    """ModernBERT-large (config 3) attn.Wo(+residual) -> Wi+GeGLU ->
    mlp.Wo(+residual) -> Wqkv in one launch at small M, blocked weights:
    each output against the oracle's f32 projection of the GPU chain's own
    inputs."""
    from sys1_amd import _lib
    from sys1_amd.linear import pack_blocked_weight, pack_gated_weight
    H, I = 1024, 2624
    print(f"[gpu] weight-streaming chain modernbert-large M={M}", flush=True)
    qkv_np = orc.round_bf16(orc.fill_normal((M, 3 * H), 3))
    h0_np = orc.round_bf16(orc.fill_normal((M, H), 4))
    w = [orc.round_bf16(orc.fill_normal(s, 20 + i, 0.02))
         for i, s in enumerate([(H, H), (2 * I, H), (H, I), (3 * H, H)])]
    qkv = to_gpu_bf16(qkv_np, torch)
    h = to_gpu_bf16(h0_np, torch)
    act = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    wg = [to_gpu_bf16(v, torch) for v in w]
    wg[1] = pack_gated_weight(wg[1], dev)
    wb = [pack_blocked_weight(v, dev) for v in wg]
    qkv_out = torch.empty(M, 3 * H, dtype=torch.bfloat16, device="cuda")
    B = _lib.EPI_BLOCKED_W

    def cp(x, wi, y, epi, N, K, res=None):
        return _lib.ChainProj(x.data_ptr(), x.stride(0), wb[wi].data_ptr(), K,
                              res.data_ptr() if res is not None else None, res.stride(0) if res is not None else 0,
                              y.data_ptr(), y.stride(0), N, K, epi | B)
    projs = [cp(qkv[:, 2 * H:], 0, h, _lib.EPI_RESIDUAL, H, H, res=h),
             cp(h, 1, act, _lib.EPI_GEGLU, 2 * I, H),
             cp(act, 2, h, _lib.EPI_RESIDUAL, H, I, res=h),
             cp(h, 3, qkv_out, _lib.EPI_NONE, 3 * H, H)]
    _chain_launch(dev, projs, M)
    torch.cuda.synchronize()
    assert dev.chain_status() == 0
    h1_ref = orc.linear_f32(np.ascontiguousarray(qkv_np[:, 2 * H:]), w[0]) + h0_np
    act_np = to_np(act)
    assert_parity(act_np, orc.geglu(orc.linear_f32(orc.round_bf16(h1_ref), w[1])), f"Wi+GeGLU M={M}")
    h2_np = to_np(h)
    assert_parity(h2_np, orc.linear_f32(act_np, w[2]) + orc.round_bf16(h1_ref), f"mlp.Wo M={M}")
    assert_parity(to_np(qkv_out), orc.linear_f32(h2_np, w[3]), f"Wqkv M={M}")


@pytest.mark.parametrize("M", [16, 64])
def test_weight_streaming_chain_stack_against_per_projection_and_oracle(dev, orc, M):
    """The ModernBERT-large stack (4 layers) with chains at small M against
    the per-projection stack (skinny kernels, another summation order) and
    the oracle chain that rounds where the GPU path rounds; run twice, the
    same bits both times."""
    from sys1_amd.stacks import ProjectionStack, modernbert
    import test_gpu_stack as T
    cfg = modernbert(1024, 2624, 4, "modernbert-large-4")
    print(f"[gpu] weight-streaming chain stack modernbert-large 4 layers M={M}", flush=True)
    x = orc.fill_normal((M, 1024), 51)
    ws = T._weights(orc, cfg, 400)
    wg = [[to_gpu_bf16(w, torch) for w in l] for l in ws]
    a = ProjectionStack(cfg, dev, M, weights=wg, blocked=True, chain=True)
    b = ProjectionStack(cfg, dev, M, weights=wg, blocked=True)
    xg = to_gpu_bf16(x, torch)
    ya = a.forward(xg, M).clone()
    ya2 = a.forward(xg, M).clone()
    yb = b.forward(xg, M).clone()
    torch.cuda.synchronize()
    assert dev.chain_status() == 0
    assert torch.equal(ya.view(torch.int16), ya2.view(torch.int16))
    emul = T._oracle_chain_bf16(orc, cfg, x, ws, None)
    f32 = T._oracle_chain(orc, cfg, x, ws, None)
    spread, _ = parity(emul, f32)
    ra, _ = parity(to_np(ya), emul)
    rb, _ = parity(to_np(yb), emul)
    print(f"[gpu]   vs bf16-rounding oracle chain: chain {ra:.3e}, per-projection {rb:.3e}; oracle chains "
          f"differ by {spread:.3e}", flush=True)
    assert ra < max(4 * spread, 1e-2) and rb < max(4 * spread, 1e-2)


def test_weight_streaming_chain_bounded_wait(dev, orc):
    """The weight-streaming chain's waits, forced to expire from the host:
    the launch finishes and reports it; the next launch is clean."""
    from sys1_amd.stacks import ProjectionStack, modernbert
    cfg = modernbert(1024, 2624, 2, "modernbert-large-2")
    M = 32
    ws = [[(torch.randn(p.N, p.K, device="cuda") * 0.02).to(torch.bfloat16) for p in layer]
          for layer in cfg.layers]
    a = ProjectionStack(cfg, dev, M, weights=ws, blocked=True, chain=True)
    x = to_gpu_bf16(orc.fill_normal((M, 1024), 7), torch)
    ref = a.forward(x, M).clone()
    torch.cuda.synchronize()
    assert dev.chain_status() == 0
    dev.set_chain_wait(wait_us=200, extra=1 << 20)
    try:
        print("[gpu] weight-streaming chain with unreachable dependencies", flush=True)
        a.forward(x, M, check=False)
        flags = dev.chain_status()
        with pytest.raises(RuntimeError, match="dependency wait expired"):
            a.forward(x, M)
    finally:
        dev.set_chain_wait()
    assert flags & 1
    again = a.forward(x, M).clone()
    torch.cuda.synchronize()
    assert dev.chain_status() == 0
    assert torch.equal(again.view(torch.int16), ref.view(torch.int16))
