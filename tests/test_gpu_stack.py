"""GPU parity of whole projection stacks (the callers of the hot path)
against the CPU oracle, through the C ABI.

  - every projection of the chain, on the inputs the GPU chain actually fed
    it, against the oracle's f32 projection (rel. Frobenius <= 1e-2, max-abs
    <= 2e-2 * max|ref|);
  - the final hidden state of the bf16 GPU chain against the oracle's f32
    chain from the same seeded f32 inputs (reported, and bounded);
  - the decision logits of the Laya scorer (src/models/laya.rs:510-520) at
    option-marker rows: within 3e-2 of the oracle's f32 logits (the bound of
    the final hidden state: bf16 storage through 22 layers), and the
    argmax (src/models/laya.rs:909-916: lowest index on ties) identical on
    every request to the oracle chain that rounds where the GPU path rounds
    (bf16 storage of every activation, each projection and each epilogue op
    rounded to bf16), over at least 64 requests per configuration; the
    agreement with the f32 chain's argmax is printed alongside.

Chains apply the reference's pre-block norms (ModernBERT's bias-free
LayerNorm, Qwen's RMSNorm) as glue on both sides -- without them the
norm-free chain grows without bound and no precision comparison is
meaningful.  The attention stand-in (V block of Wqkv feeds Wo; z block feeds
out_proj; q block feeds o_proj) is the one the stacks use.
"""
import numpy as np
import pytest

from gpu_helpers import assert_parity, parity, to_gpu_bf16, to_np

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from sys1_amd.device import HipDevice
    return HipDevice(0)


def _weights(orc, cfg, seed):
    return [[orc.fill_normal((p.N, p.K), seed + 1000 * li + pi, 0.02) for pi, p in enumerate(layer)]
            for li, layer in enumerate(cfg.layers)]


def _norm_gpu(h, kind):
    """Pre-block norm as glue (not a projection): ModernBERT's bias-free
    LayerNorm (src/archs/modernbert.rs:1005-1034, weight 1) or Qwen's RMSNorm
    with alpha = 1 + w, w = 0 (src/archs/qwen35_text.rs:178-203), in f32."""
    hf = h.float()
    if kind == "ln":
        out = torch.nn.functional.layer_norm(hf, (hf.shape[-1],), eps=1e-5)
    else:
        out = hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-6)
    return out.to(torch.bfloat16)


def _norm_ref(orc, h, kind):
    h = np.asarray(h, np.float32)
    if kind == "ln":
        return orc.layer_norm(h, np.ones(h.shape[-1], np.float32), None, 1e-5)
    hd = h.astype(np.float64)
    return (hd / np.sqrt((hd ** 2).mean(-1, keepdims=True) + 1e-6)).astype(np.float32)


def _project_ref(orc, p, src, w, resid):
    """The oracle's f32 projection of one stack entry (with its epilogue)."""
    from sys1_amd import _lib
    proj = orc.linear_f32(src, w)
    if p.epi == _lib.EPI_GEGLU:
        return orc.geglu(proj)
    if p.epi == _lib.EPI_SWIGLU:
        I = p.N // 2
        return orc.swiglu(proj[:, :I], proj[:, I:])
    return proj + resid if p.resid else proj


def _chain_per_projection(orc, dev, cfg, x, ws, norm, check=True):
    """Run the stack projection by projection on the GPU (sys1_amd.linear
    modules) and (with `check`) each output against the oracle on the same
    input."""
    from sys1_amd import _lib
    from sys1_amd.linear import GatedLinear, Linear
    M = x.shape[0]
    h = to_gpu_bf16(x, torch)
    mix = None
    worst = 0.0
    for li, layer in enumerate(cfg.layers):
        for pi, p in enumerate(layer):
            w = ws[li][pi]
            if p.src == "h":
                src = _norm_gpu(h, norm) if norm else h
            else:
                src = mix[:, p.src_off:p.src_off + p.K]
            wg = to_gpu_bf16(w, torch)
            if p.epi in (_lib.EPI_GEGLU, _lib.EPI_SWIGLU):
                out = GatedLinear(wg, "gelu" if p.epi == _lib.EPI_GEGLU else "silu", device=dev)(src)
            elif p.resid:
                out = Linear(wg, device=dev)(src, residual=h)
            else:
                out = Linear(wg, device=dev)(src)
            if check:
                ref = _project_ref(orc, p, to_np(src), w, to_np(h) if p.resid else None)
                rel, _ = assert_parity(to_np(out), ref, f"layer {li} {p.name} M={M}")
                worst = max(worst, rel)
            if p.dst == "h":
                h = out
            else:
                mix = out
    return h, worst


def _oracle_chain(orc, cfg, x, ws, norm):
    """The same chain in f32 end to end (the reference's f32 CPU path)."""
    h = x.astype(np.float32)
    mix = None
    for li, layer in enumerate(cfg.layers):
        for pi, p in enumerate(layer):
            if p.src == "h":
                src = _norm_ref(orc, h, norm) if norm else h
            else:
                src = np.ascontiguousarray(mix[:, p.src_off:p.src_off + p.K])
            out = _project_ref(orc, p, src, ws[li][pi], h if p.resid else None)
            if p.dst == "h":
                h = out
            else:
                mix = out
    return h


def _oracle_chain_bf16(orc, cfg, x, ws, norm):
    """The same chain rounded where the GPU path rounds: the input, the
    weights and every stored activation are bf16; a projection accumulates
    in f32 and is rounded to bf16, then each epilogue op runs in f32 on the
    bf16 values and is rounded (residual: bf16(p + r); GeGLU / SwiGLU:
    bf16(bf16(act(g)) * u) on the bf16 gate and up); the norm glue runs in
    f32 and is rounded.  The GPU chain and this one differ only by the f32
    summation order inside each projection."""
    from sys1_amd import _lib
    rb = orc.round_bf16
    h = rb(x)
    mix = None
    for li, layer in enumerate(cfg.layers):
        for pi, p in enumerate(layer):
            if p.src == "h":
                src = rb(_norm_ref(orc, h, norm)) if norm else h
            else:
                src = np.ascontiguousarray(mix[:, p.src_off:p.src_off + p.K])
            proj = orc.linear_f32(src, rb(ws[li][pi]))
            if p.epi in (_lib.EPI_GEGLU, _lib.EPI_SWIGLU):
                I = p.N // 2
                g, u = rb(proj[:, :I]), rb(proj[:, I:])
                act = orc.gelu_erf(g) if p.epi == _lib.EPI_GEGLU else orc.silu(g)
                out = rb(rb(act) * u)
            else:
                out = rb(proj)
                if p.resid:
                    out = rb(out + h)
            if p.dst == "h":
                h = out
            else:
                mix = out
    return h


def _scorer_bf16_ref(orc, hidden_rows, params):
    """The scorer at the GPU path's rounding points (_gpu_scorer): LN in
    f32 -> bf16; projection -> bf16, + bias -> bf16, gelu -> bf16;
    projection -> bf16, + bias -> bf16 (the decision logits are bf16)."""
    rb = orc.round_bf16
    g, b, w_in, b_in, w_out, b_out = params
    z = rb(orc.layer_norm(hidden_rows, g, b, 1e-5))
    z = rb(orc.gelu_erf(rb(rb(orc.linear_f32(z, rb(w_in))) + rb(b_in))))
    return rb(rb(orc.linear_f32(z, rb(w_out))) + rb(b_out))[:, 0]


def _scorer(orc, H, seed):
    g = orc.fill_normal((H,), seed, 0.1) + 1.0
    b = orc.fill_normal((H,), seed + 1, 0.1)
    w_in = orc.fill_normal((H, H), seed + 2, 1.0 / np.sqrt(H))
    b_in = orc.fill_normal((H,), seed + 3, 0.1)
    w_out = orc.fill_normal((1, H), seed + 4, 1.0 / np.sqrt(H))
    b_out = orc.fill_normal((1,), seed + 5, 0.1)
    return g, b, w_in, b_in, w_out, b_out


def _gpu_scorer(dev, hidden_rows_gpu, params):
    """LN (torch, f32: not a projection) -> Linear+bias+gelu (fused) ->
    Linear+bias, the last two on the HIP kernels."""
    from sys1_amd.linear import Linear
    g, b, w_in, b_in, w_out, b_out = params
    z = torch.nn.functional.layer_norm(hidden_rows_gpu.float(), (g.size,),
                                       torch.from_numpy(g).cuda(), torch.from_numpy(b).cuda(), 1e-5)
    z = z.to(torch.bfloat16)
    z = Linear(to_gpu_bf16(w_in, torch), to_gpu_bf16(b_in, torch), device=dev)(z, gelu=True)
    return to_np(Linear(to_gpu_bf16(w_out, torch), to_gpu_bf16(b_out, torch), device=dev)(z))[:, 0]


def _markers(lengths, options, seed):
    """Option-marker rows: `options` distinct positions inside each sequence."""
    rng = np.random.default_rng(seed)
    rows, off = [], 0
    for L in lengths:
        rows.append(off + np.sort(rng.choice(L, size=min(options, L), replace=False)))
        off += L
    return rows


def _check_argmax(orc, dev, h_gpu, h_ref, h_emul, lengths, H, seed):
    """Scorer at the option markers after the encoder's final norm
    (src/models/modernbert.rs:988).  Returns (requests, agreeing with the
    bf16-emulating chain, agreeing with the f32 chain); asserts the logits
    within CHAIN_TOL of the f32 chain's."""
    params = _scorer(orc, H, seed)
    marks = _markers(lengths, 4, seed)
    flat = np.concatenate(marks)
    logits_ref = orc.laya_scorer_f32(_norm_ref(orc, h_ref[flat], "ln"), *params)
    logits_emul = _scorer_bf16_ref(orc, orc.round_bf16(_norm_ref(orc, h_emul[flat], "ln")), params)
    logits_gpu = _gpu_scorer(dev, _norm_gpu(h_gpu[torch.from_numpy(flat).cuda()], "ln"), params)
    rel = parity(logits_gpu, logits_ref)[0]
    assert rel <= CHAIN_TOL, f"logit rel err {rel:.3e}"  # (22 layers of bf16 storage, as the hidden state)
    off = same_emul = same_f32 = 0
    for r in marks:
        lg, le, lr = (v[off:off + len(r)] for v in (logits_gpu, logits_emul, logits_ref))
        off += len(r)
        same_emul += orc.argmax(lg) == orc.argmax(le)
        same_f32 += orc.argmax(lg) == orc.argmax(lr)
    print(f"[gpu]   batch: {same_emul}/{len(marks)} argmax = bf16-emulating chain, {same_f32}/{len(marks)} "
          f"= f32 chain; logit rel err vs f32 {rel:.3e}", flush=True)
    return len(marks), int(same_emul), int(same_f32)


def _decisions(orc, dev, cfg, batches, H, seed):
    """Chains over several packed batches (lists of sequence lengths): the
    first with every projection checked against the oracle, all with the
    decision argmax checked.  Every request's argmax must equal the
    bf16-emulating oracle chain's; at least 64 requests in all."""
    total = emul = f32 = 0
    worst = rel_final = 0.0
    for bi, lengths in enumerate(batches):
        M = int(sum(lengths))
        print(f"[gpu] {cfg.name} batch {bi}: M={M}, {len(lengths)} requests", flush=True)
        x = orc.fill_normal((M, H), seed + 17 * bi)
        ws = _weights(orc, cfg, 100 * (seed + bi))
        h_gpu, w = _chain_per_projection(orc, dev, cfg, x, ws, "ln", check=bi == 0)
        worst = max(worst, w)
        h_ref = _oracle_chain(orc, cfg, x, ws, "ln")
        h_emul = _oracle_chain_bf16(orc, cfg, x, ws, "ln")
        rel, _ = parity(to_np(h_gpu), h_ref)
        rel_final = max(rel_final, rel)
        print(f"[gpu]   final hidden vs f32 chain rel_fro={rel:.3e}, vs bf16-emulating chain "
              f"{parity(to_np(h_gpu), h_emul)[0]:.3e}", flush=True)
        assert rel < CHAIN_TOL
        n, e, f = _check_argmax(orc, dev, h_gpu, h_ref, h_emul, lengths, H, seed + bi)
        total, emul, f32 = total + n, emul + e, f32 + f
    print(f"[gpu] {cfg.name}: argmax identical to the bf16-emulating chain on {emul}/{total} requests, "
          f"to the f32 chain on {f32}/{total}; worst per-projection rel_fro {worst:.3e}, "
          f"worst final hidden rel_fro {rel_final:.3e}", flush=True)
    assert total >= 64
    assert emul == total


# The bf16 chain vs the f32 chain over 22 normed layers: about 1.3e-2 from
# bf16 rounding alone (emulating the bf16 chain with the oracle gives the same).
CHAIN_TOL = 3e-2


def test_modernbert_base_cfg1_chain(dev, orc):
    """BASELINE config 1 shapes: 22 layers, hidden 768, M = 8 x 128 = 1024,
    over 8 seeded batches (64 requests)."""
    from sys1_amd.stacks import CONFIGS
    cfg = CONFIGS["modernbert-base"]()
    _decisions(orc, dev, cfg, [[128] * 8] * 8, 768, 7)


def test_modernbert_base_ragged_chain(dev, orc):
    """lengths U[16,512] packed to an 8192-token budget,
    batches drawn until they hold at least 64 requests."""
    from sys1_amd.batching import draw_lengths
    from sys1_amd.stacks import CONFIGS
    cfg = CONFIGS["modernbert-base"]()
    batches, n = [], 0
    while n < 64:
        batches.append([int(v) for v in draw_lengths(3 + len(batches), 16, 512, 8192)])
        n += len(batches[-1])
    _decisions(orc, dev, cfg, batches, 768, 9)


def test_projection_stack_matches_module_chain(dev, orc):
    """The fused ProjectionStack (the bench's path: one C call per
    projection, in-place residual, V-slice stand-in) equals the
    module-by-module chain bit for bit on a ragged 8192-budget batch."""
    from sys1_amd.batching import draw_lengths
    from sys1_amd.linear import GatedLinear, Linear
    from sys1_amd.stacks import CONFIGS, ProjectionStack, modernbert
    cfg = modernbert(768, 1152, 3, "modernbert-base-3")
    M = int(draw_lengths(5, 16, 512, 8192).sum())
    x = to_gpu_bf16(orc.fill_normal((M, 768), 3), torch)
    ws = [[(torch.randn(p.N, p.K, device="cuda") * 0.02).to(torch.bfloat16) for p in layer]
          for layer in cfg.layers]
    stack = ProjectionStack(cfg, dev, M, weights=ws)
    out = stack.forward(x, M).clone()
    h = x
    for (wqkv, wo, wi, wo2) in ws:
        qkv = Linear(wqkv, device=dev)(h)
        h = Linear(wo, device=dev)(qkv[:, 1536:], residual=h)
        g = GatedLinear(wi, "gelu", device=dev)(h)
        h = Linear(wo2, device=dev)(g, residual=h)
    assert torch.equal(out, h)


def _oracle_chain_prenorm(orc, cfg, x, ws):
    """The f32 chain with each projection's own pre-norm (Proj.norm): the
    reference layer order, norm weights of a fresh model (LayerNorm weight
    1, eps 1e-5; RMSNorm weight 0, eps 1e-6)."""
    h = x.astype(np.float32)
    mix = None
    for li, layer in enumerate(cfg.layers):
        for pi, p in enumerate(layer):
            if p.src == "h":
                src = h
                if p.norm == "layer":
                    src = orc.layer_norm(h, np.ones(h.shape[-1], np.float32), None, 1e-5)
                elif p.norm == "rms":
                    src = orc.rms_norm(h, np.zeros(h.shape[-1], np.float32), 1e-6)
            else:
                src = np.ascontiguousarray(mix[:, p.src_off:p.src_off + p.K])
            out = _project_ref(orc, p, src, ws[li][pi], h if p.resid else None)
            if p.dst == "h":
                h = out
            else:
                mix = out
    return h


def _oracle_chain_prenorm_bf16(orc, cfg, x, ws):
    """_oracle_chain_prenorm rounded where the fused pre-norm GPU path rounds
    (ModernBERT, LayerNorm weight 1): activations stored in bf16; a normed
    projection is the raw bf16 input times the bf16 weight in f32, corrected
    per row as r_m (acc - mu_m c_n) with mu_m, r_m the row's f32 mean and
    1/sqrt(var + eps) and c_n the f32 sum of weight row n, then rounded (the
    gated ones: gate and up rounded, act rounded, product rounded); plain
    projections and residual adds as in _oracle_chain_bf16."""
    from sys1_amd import _lib
    rb = orc.round_bf16
    h = rb(x)
    mix = None
    for li, layer in enumerate(cfg.layers):
        for pi, p in enumerate(layer):
            w = rb(ws[li][pi])
            src = h if p.src == "h" else np.ascontiguousarray(mix[:, p.src_off:p.src_off + p.K])
            proj = orc.linear_f32(src, w)
            if p.norm == "layer" and p.src == "h":
                hd = src.astype(np.float64)
                mu = hd.mean(1, keepdims=True)
                r = 1.0 / np.sqrt(((hd - mu) ** 2).mean(1, keepdims=True) + 1e-5)
                c = w.astype(np.float64).sum(1)[None, :]
                proj = (r * (proj.astype(np.float64) - mu * c)).astype(np.float32)
            elif p.norm is not None and p.src == "h":
                raise ValueError("the emulation covers LayerNorm only")
            if p.epi in (_lib.EPI_GEGLU, _lib.EPI_SWIGLU):
                I = p.N // 2
                g, u = rb(proj[:, :I]), rb(proj[:, I:])
                act = orc.gelu_erf(g) if p.epi == _lib.EPI_GEGLU else orc.silu(g)
                out = rb(rb(act) * u)
            else:
                out = rb(proj)
                if p.resid:
                    out = rb(out + h)
            if p.dst == "h":
                h = out
            else:
                mix = out
    return h


@pytest.mark.parametrize("family,M", [("modernbert", 1024), ("qwen", 512)])
def test_stack_with_fused_norms_matches_f32_chain(dev, orc, family, M):
    """The bench stack with its pre-norms fused (ProjectionStack(norms=True):
    ModernBERT's LayerNorms before Wqkv (not in layer 0) and Wi, Qwen's
    RMSNorms before in_proj / q,k,v and gate/up) against the f32 chain with
    the same norms unfused."""
    from sys1_amd.stacks import ProjectionStack, modernbert, qwen35
    if family == "modernbert":
        cfg = modernbert(768, 1152, 4, "modernbert-base-4")
    else:
        cfg = qwen35(2048, 4, 16, 2, 128, 6144, 2048, 4096, 16, 2048, "qwen35-small-4")
    print(f"[gpu] {cfg.name} fused pre-norm stack M={M}", flush=True)
    x = orc.fill_normal((M, cfg.hidden), 17)
    ws = _weights(orc, cfg, 500)
    stack = ProjectionStack(cfg, dev, M, weights=[[to_gpu_bf16(w, torch) for w in l] for l in ws],
                            norms=True)
    h_gpu = to_np(stack.forward(to_gpu_bf16(x, torch), M))
    torch.cuda.synchronize()
    h_ref = _oracle_chain_prenorm(orc, cfg, x, ws)
    rel, mx = parity(h_gpu, h_ref)
    print(f"[gpu] {cfg.name} final hidden vs f32 chain: rel_fro={rel:.3e} max={mx:.3e}", flush=True)
    assert rel < CHAIN_TOL and mx < 5 * CHAIN_TOL


def test_fused_norm_stack_matches_module_chain(dev, orc):
    """The stack's pre-norm calls are the NormLinear module's calls: the
    two chains agree bit for bit."""
    from sys1_amd.linear import Linear
    from sys1_amd.norm import NormLinear
    from sys1_amd.stacks import ProjectionStack, modernbert
    cfg = modernbert(768, 1152, 3, "modernbert-base-3")
    M = 777
    x = to_gpu_bf16(orc.fill_normal((M, 768), 5), torch)
    ws = [[(torch.randn(p.N, p.K, device="cuda") * 0.02).to(torch.bfloat16) for p in layer]
          for layer in cfg.layers]
    out = ProjectionStack(cfg, dev, M, weights=ws, norms=True).forward(x, M).clone()
    h = x
    for li, (wqkv, wo, wi, wo2) in enumerate(ws):
        qkv = (NormLinear(wqkv, torch.ones(768), "layer", 1e-5, device=dev) if li else
               Linear(wqkv, device=dev))(h)
        h = Linear(wo, device=dev)(qkv[:, 1536:], residual=h)
        g = NormLinear(wi, torch.ones(768), "layer", 1e-5, "gelu", device=dev)(h)
        h = Linear(wo2, device=dev)(g, residual=h)
    assert torch.equal(out, h)


@pytest.mark.parametrize("M,layers", [(64, 4), (256, 4), (1024, 4), (4096, 2), (16384, 1)])
def test_modernbert_large_chain(dev, orc, M, layers):
    """BASELINE config 3 shapes (hidden 1024, GeGLU 2x2624) over its whole M
    sweep {64, 256, 1024, 4096, 16384}: weight-streaming stream-K (64, 256),
    128x128 tiles with deep-K stream-K (1024), 128x128 and 256x256 tiles
    (4096, 16384).  Fewer layers at large M keep the CPU oracle to seconds."""
    from sys1_amd.stacks import modernbert
    cfg = modernbert(1024, 2624, layers, f"modernbert-large-{layers}")
    print(f"[gpu] modernbert-large 4 layers M={M}", flush=True)
    x = orc.fill_normal((M, 1024), 21)
    ws = _weights(orc, cfg, 500)
    h_gpu, worst = _chain_per_projection(orc, dev, cfg, x, ws, "ln")
    rel, _ = parity(to_np(h_gpu), _oracle_chain(orc, cfg, x, ws, "ln"))
    print(f"[gpu] large M={M}: final rel_fro={rel:.3e}, worst per-projection {worst:.3e}", flush=True)
    assert rel < CHAIN_TOL


@pytest.mark.parametrize("name,M,both", [("qwen35-small", 256, True), ("qwen35-small", 1000, True),
                                         ("qwen35-small", 8192, True), ("qwen35-27b", 128, True),
                                         ("qwen35-27b", 1024, True), ("qwen35-27b", 4096, True)])
def test_qwen_layers(dev, orc, name, M, both):
    """One DeltaNet layer and (where `both`) one gated-attention layer of the
    Qwen3.5-style configs (4 and 5), at their real projection shapes and the
    BASELINE token counts (config 4: exactly 8192; config 5: 128, 1024 and
    4096), per projection."""
    from sys1_amd.stacks import CONFIGS, StackConfig
    full = CONFIGS[name]()
    cfg = StackConfig(name, full.hidden, [full.layers[0], full.layers[3]] if both else [full.layers[0]])
    print(f"[gpu] {name} DeltaNet + attention layer M={M}", flush=True)
    x = orc.fill_normal((M, full.hidden), 31)
    ws = _weights(orc, cfg, 700)
    h_gpu, worst = _chain_per_projection(orc, dev, cfg, x, ws, "rms")
    rel, _ = parity(to_np(h_gpu), _oracle_chain(orc, cfg, x, ws, "rms"))
    print(f"[gpu] {name} M={M}: final rel_fro={rel:.3e}, worst per-projection rel_fro={worst:.3e}",
          flush=True)
    assert rel < CHAIN_TOL


def test_row_permutation_is_exact(dev, orc):
    """Row independence: permuting the packed tokens permutes the outputs
    bit for bit (same kernel, same split), which is what makes packing the
    reference's padded rectangle exact."""
    from sys1_amd.linear import GatedLinear, Linear
    for (M, N, K) in [(8000, 2304, 768), (200, 3072, 1024)]:
        x = torch.randn(M, K, device="cuda").to(torch.bfloat16)
        w = (torch.randn(N, K, device="cuda") * 0.02).to(torch.bfloat16)
        perm = torch.randperm(M, device="cuda")
        lin = Linear(w, device=dev)
        assert torch.equal(lin(x)[perm], lin(x[perm]))
        g = GatedLinear(w, "gelu", device=dev)
        assert torch.equal(g(x)[perm], g(x[perm]))


def test_stack_from_safetensors_checkpoint(dev, orc, tmp_path):
    """A ProjectionStack loaded from a checkpoint in the reference's tensor
    names equals the stack built from the same tensors, and follows the f32
    oracle layer (src/archs/modernbert.rs:857-887 with the stand-in)."""
    st = pytest.importorskip("safetensors.torch")
    from sys1_amd import weights as W
    from sys1_amd.stacks import ProjectionStack
    cfg_json = {"hidden_size": 128, "intermediate_size": 192, "num_hidden_layers": 2,
                "num_attention_heads": 2}
    g = torch.Generator().manual_seed(7)
    t = {}
    for i in range(2):
        p = f"model.layers.{i}."
        t[p + "attn.Wqkv.weight"] = torch.randn(384, 128, generator=g) * 0.05
        t[p + "attn.Wo.weight"] = torch.randn(128, 128, generator=g) * 0.05
        t[p + "mlp.Wi.weight"] = torch.randn(384, 128, generator=g) * 0.05
        t[p + "mlp.Wo.weight"] = torch.randn(128, 192, generator=g) * 0.05
    path = str(tmp_path / "m.safetensors")
    st.save_file(t, path)
    M = 200
    x = to_gpu_bf16(orc.fill_normal((M, 128), 17), torch)
    stack = W.load_stack(path, "modernbert", cfg_json, dev, M)
    out = stack.forward(x, M).clone()
    ws = [[t[f"model.layers.{i}.{n}.weight"].to(torch.bfloat16).cuda() for n in
           ("attn.Wqkv", "attn.Wo", "mlp.Wi", "mlp.Wo")] for i in range(2)]
    direct = ProjectionStack(W.modernbert_config(cfg_json), dev, M, weights=ws).forward(x, M)
    assert torch.equal(out, direct)
    h = to_np(x)
    for i in range(2):
        f = [to_np(w) for w in ws[i]]
        h = orc.modernbert_layer_f32(h, *f)
    rel, _ = parity(to_np(out), h)
    print(f"[gpu] checkpoint stack vs f32 oracle: rel_fro={rel:.3e}", flush=True)
    assert rel < CHAIN_TOL


def test_stack_with_norms_from_safetensors_checkpoint(dev, orc, tmp_path):
    """load_stack(norms=True): projection and pre-norm weights by the
    reference's names (attn_norm from layer 1, mlp_norm), eps from the
    config; equals the stack built from the same tensors and follows the f32
    chain with those norms."""
    st = pytest.importorskip("safetensors.torch")
    from sys1_amd import weights as W
    from sys1_amd.stacks import ProjectionStack
    cfg_json = {"hidden_size": 128, "intermediate_size": 192, "num_hidden_layers": 2,
                "num_attention_heads": 2, "layer_norm_eps": 1e-5}
    g = torch.Generator().manual_seed(9)
    t = {}
    for i in range(2):
        p = f"model.layers.{i}."
        t[p + "attn.Wqkv.weight"] = torch.randn(384, 128, generator=g) * 0.05
        t[p + "attn.Wo.weight"] = torch.randn(128, 128, generator=g) * 0.05
        t[p + "mlp.Wi.weight"] = torch.randn(384, 128, generator=g) * 0.05
        t[p + "mlp.Wo.weight"] = torch.randn(128, 192, generator=g) * 0.05
        t[p + "mlp_norm.weight"] = 1.0 + 0.1 * torch.randn(128, generator=g)
        if i:
            t[p + "attn_norm.weight"] = 1.0 + 0.1 * torch.randn(128, generator=g)
    path = str(tmp_path / "mn.safetensors")
    st.save_file(t, path)
    M = 300
    xf = orc.fill_normal((M, 128), 19)
    x = to_gpu_bf16(xf, torch)
    print(f"[gpu] checkpoint stack with norms M={M}", flush=True)
    out = W.load_stack(path, "modernbert", cfg_json, dev, M, norms=True).forward(x, M).clone()
    cfg = W.modernbert_config(cfg_json)
    ws = W.read_projection_weights(path, "modernbert", cfg)
    nw = W.read_norm_weights(path, "modernbert", cfg)
    direct = ProjectionStack(cfg, dev, M, weights=[[w.cuda() for w in l] for l in ws], norms=True,
                             norm_weights=nw).forward(x, M)
    assert torch.equal(out, direct)
    h = to_np(x)
    for li, layer in enumerate(cfg.layers):
        f = [to_np(w) for w in ws[li]]
        g0 = nw[li][0].numpy() if nw[li][0] is not None else None
        src = orc.layer_norm(h, g0, None, 1e-5) if g0 is not None else h
        qkv = orc.linear_f32(src, f[0])
        h = orc.linear_f32(np.ascontiguousarray(qkv[:, 256:]), f[1]) + h
        act = orc.geglu(orc.linear_f32(orc.layer_norm(h, nw[li][2].numpy(), None, 1e-5), f[2]))
        h = orc.linear_f32(act, f[3]) + h
    rel, _ = parity(to_np(out), h)
    print(f"[gpu] checkpoint stack with norms vs f32 oracle: rel_fro={rel:.3e}", flush=True)
    assert rel < CHAIN_TOL


def test_qwen_stack_with_norms_and_conv_matches_f32_chain(dev, orc):
    """The Qwen3.5 stack with its input RMSNorms and the DeltaNet causal
    conv + SiLU fused into in_proj (ProjectionStack(norms=True, conv=True))
    on ragged packed sequences, against the f32 chain with both unfused
    (src/archs/qwen35_text.rs:515-526,632-650,932-940)."""
    from sys1_amd import batching
    from sys1_amd.stacks import ProjectionStack, qwen35
    cfg = qwen35(2048, 4, 16, 2, 128, 6144, 2048, 4096, 16, 2048, "qwen35-small-4")
    lengths = batching.draw_lengths(21, 16, 300, 700)
    M = int(lengths.sum())
    pos = batching.positions(lengths)
    print(f"[gpu] qwen stack norms+conv M={M} ({len(lengths)} sequences)", flush=True)
    x = orc.fill_normal((M, cfg.hidden), 23)
    ws = _weights(orc, cfg, 700)
    cws = [orc.round_bf16(orc.fill_normal((layer[0].conv_ch, 4), 900 + li, 0.5)) if layer[0].conv_ch else None
           for li, layer in enumerate(cfg.layers)]
    stack = ProjectionStack(cfg, dev, M, weights=[[to_gpu_bf16(w, torch) for w in l] for l in ws],
                            norms=True, conv=True,
                            conv_weights=[torch.from_numpy(c) if c is not None else None for c in cws])
    h_gpu = to_np(stack.forward(to_gpu_bf16(x, torch), M, torch.from_numpy(pos).cuda()))
    torch.cuda.synchronize()
    h = x.astype(np.float32)
    mix = None
    for li, layer in enumerate(cfg.layers):
        for pi, p in enumerate(layer):
            if p.src == "h":
                src = orc.rms_norm(h, np.zeros(h.shape[-1], np.float32), 1e-6) if p.norm else h
            else:
                src = np.ascontiguousarray(mix[:, p.src_off:p.src_off + p.K])
            out = _project_ref(orc, p, src, ws[li][pi], h if p.resid else None)
            if p.conv_ch:
                out = np.concatenate([orc.conv_silu(out[:, :p.conv_ch], cws[li], pos, bf16=False),
                                      out[:, p.conv_ch:]], axis=1)
            if p.dst == "h":
                h = out
            else:
                mix = out
    rel, mx = parity(h_gpu, h)
    print(f"[gpu] qwen norms+conv final hidden vs f32 chain: rel_fro={rel:.3e} max={mx:.3e}", flush=True)
    assert rel < CHAIN_TOL and mx < 5 * CHAIN_TOL


def test_bench_stack_object_at_cfg2_size(dev, orc):
    """The object bench.py times, at its size: ProjectionStack(blocked=True)
    over all 22 ModernBERT-base layers on a config-2 ragged batch (lengths
    U[16,512] packed to 8192).  Its prepared calls run one at a time; every
    projection's output is checked against the oracle's f32 projection of
    the input (and residual) the GPU chain actually fed it, and the whole
    stack enqueued at once (as the bench does) must give the same bits.
    The stack has no norms (they are not projections), so the hidden state
    grows layer over layer; the final state is compared with the oracle
    chain that rounds where the GPU path rounds, and reported."""
    from sys1_amd.batching import draw_lengths
    from sys1_amd.stacks import CONFIGS, ProjectionStack
    cfg = CONFIGS["modernbert-base"]()
    M = int(draw_lengths(11, 16, 512, 8192).sum())
    print(f"[gpu] bench stack object: modernbert-base 22 layers blocked M={M}", flush=True)
    x = orc.fill_normal((M, 768), 29)
    ws = _weights(orc, cfg, 300)
    xg = to_gpu_bf16(x, torch)
    stack = ProjectionStack(cfg, dev, M, weights=[[to_gpu_bf16(w, torch) for w in l] for l in ws],
                            blocked=True)
    prepared = stack.prepare(xg, M)
    assert len(prepared) == 4 * 22
    bufs = stack.buffers
    h_prev = xg  # the residual source of the first output projection is x itself
    worst = 0.0
    dev.follow_torch_stream()
    for i, (p, fn, args) in enumerate(prepared):
        li = i // 4
        src = xg if (p.src == "h" and i == 0) else (bufs[p.src][:M, p.src_off:p.src_off + p.K]
                                                    if p.src != "h" else bufs["h"][:M, :768])
        src_np = to_np(src)
        resid_np = to_np(h_prev) if p.resid else None
        stack.run_prepared([(p, fn, args)])
        torch.cuda.synchronize()
        out = bufs[p.dst][:M, :p.nout]
        ref = _project_ref(orc, p, src_np, ws[li][i % 4], resid_np)
        rel, _ = assert_parity(to_np(out), ref, f"layer {li} {p.name} M={M}")
        worst = max(worst, rel)
        if p.dst == "h":
            h_prev = bufs["h"][:M, :768].clone()
    step_by_step = bufs["h"][:M, :768].clone()
    once = stack.forward(xg, M).clone()
    torch.cuda.synchronize()
    assert torch.equal(step_by_step, once)
    # Without norms the chain amplifies any rounding difference layer over
    # layer: the oracle's own f32 and bf16-rounding chains already differ by
    # a large fraction.  The GPU chain must stay within a small multiple of
    # that spread (a wrong projection anywhere would be far outside it).
    emul = _oracle_chain_bf16(orc, cfg, x, ws, None)
    f32 = _oracle_chain(orc, cfg, x, ws, None)
    rel, _ = parity(to_np(once), emul)
    spread, _ = parity(emul, f32)
    rel32, _ = parity(to_np(once), f32)
    print(f"[gpu] bench stack object: worst per-projection rel_fro {worst:.3e}; final hidden rel_fro vs the "
          f"bf16-rounding oracle chain {rel:.3e}, vs the f32 chain {rel32:.3e} (the two oracle chains "
          f"differ by {spread:.3e})", flush=True)
    assert rel < 4 * spread and rel32 < 4 * spread


def test_bench_norm_stack_object_decisions_at_cfg2_size(dev, orc):
    """The object `bench.py --norms` times: ProjectionStack(norms=True,
    blocked=True) over 22 ModernBERT-base layers (LayerNorms fused before
    Wqkv from layer 1 and before Wi) on config-2 ragged batches.  With the
    norms the chain is well conditioned: the final hidden state is checked
    against the oracle's f32 chain with the same norms, and the decision
    argmax (src/models/laya.rs:510-520, :909-916) at the option markers of
    at least 64 requests must equal, on every request, the argmax of the
    oracle chain that rounds where the fused path rounds (agreement with the
    f32 chain's argmax is reported: near-ties flip under bf16 storage)."""
    from sys1_amd.batching import draw_lengths
    from sys1_amd.stacks import CONFIGS, ProjectionStack
    cfg = CONFIGS["modernbert-base"]()
    ws = _weights(orc, cfg, 800)
    stack = ProjectionStack(cfg, dev, 8192, weights=[[to_gpu_bf16(w, torch) for w in l] for l in ws],
                            norms=True, blocked=True)
    total = same = 0
    bi = 0
    while total < 64:
        lengths = [int(v) for v in draw_lengths(40 + bi, 16, 512, 8192)]
        M = sum(lengths)
        print(f"[gpu] bench norm stack object batch {bi}: M={M}, {len(lengths)} requests", flush=True)
        x = orc.fill_normal((M, 768), 50 + bi)
        h_gpu = stack.forward(to_gpu_bf16(x, torch), M).clone()
        torch.cuda.synchronize()
        h_ref = _oracle_chain_prenorm(orc, cfg, x, ws)
        rel, mx = parity(to_np(h_gpu), h_ref)
        assert rel < CHAIN_TOL and mx < 5 * CHAIN_TOL, (rel, mx)
        h_emul = _oracle_chain_prenorm_bf16(orc, cfg, x, ws)
        print(f"[gpu]   final hidden rel_fro vs f32 chain {rel:.3e}, vs the fused-norm bf16-rounding chain "
              f"{parity(to_np(h_gpu), h_emul)[0]:.3e}", flush=True)
        params = _scorer(orc, 768, 60 + bi)
        marks = _markers(lengths, 4, 60 + bi)
        flat = np.concatenate(marks)
        logits_ref = orc.laya_scorer_f32(_norm_ref(orc, h_ref[flat], "ln"), *params)
        logits_emul = _scorer_bf16_ref(orc, orc.round_bf16(_norm_ref(orc, h_emul[flat], "ln")), params)
        logits_gpu = _gpu_scorer(dev, _norm_gpu(h_gpu[torch.from_numpy(flat).cuda()], "ln"), params)
        off = agree = agree32 = 0
        for r in marks:
            sl = slice(off, off + len(r))
            agree += orc.argmax(logits_gpu[sl]) == orc.argmax(logits_emul[sl])
            agree32 += orc.argmax(logits_gpu[sl]) == orc.argmax(logits_ref[sl])
            off += len(r)
        print(f"[gpu]   argmax = bf16-rounding chain on {agree}/{len(marks)}, = f32 chain on "
              f"{agree32}/{len(marks)}", flush=True)
        total, same, bi = total + len(marks), same + int(agree), bi + 1
    assert same == total, f"{same}/{total}"
