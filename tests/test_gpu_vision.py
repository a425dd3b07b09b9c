"""GPU parity of the Qwen3.5 vision tower's projections
(src/archs/qwen35_vision.rs:15-57,163-171): every Linear with its bias,
attn.proj and mlp.fc2 with the residual add, mlp.fc1 with candle's
tanh-approximate GELU fused (bias, then GELU, each rounded as the unfused
bf16 sequence rounds).  Each projection of the first block against the
oracle's f32 projection of the same inputs (relative Frobenius <= 1e-2,
max-abs <= 2e-2 max|ref|); the whole stack (the ProjectionStack object the
bench times, blocked weights) against the oracle chain that rounds where the
GPU path rounds, relative to the spread between the oracle's f32 and
bf16-rounding chains."""
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


def _params(orc, cfg, seed):
    ws = [[orc.fill_normal((p.N, p.K), seed + 100 * li + pi, 0.02) for pi, p in enumerate(layer)]
          for li, layer in enumerate(cfg.layers)]
    bs = [[orc.fill_normal((p.nout,), seed + 7 + 100 * li + pi, 0.02) for pi, p in enumerate(layer)]
          for li, layer in enumerate(cfg.layers)]
    return ws, bs


def _act(orc, p, v):
    from sys1_amd import _lib
    return orc.gelu_tanh(v) if p.epi & _lib.EPI_GELU_TANH else v


def _oracle_chain(orc, cfg, x, ws, bs, bf16):
    """f32 end to end (bf16=False), or rounded where the GPU rounds: the
    projection -> bf16, + bias -> bf16, gelu -> bf16, + residual -> bf16."""
    rb = orc.round_bf16 if bf16 else (lambda a: np.asarray(a, np.float32))
    h = rb(x)
    mix = {}
    for li, layer in enumerate(cfg.layers):
        for pi, p in enumerate(layer):
            src = h if p.src == "h" else np.ascontiguousarray(mix[p.src][:, p.src_off:p.src_off + p.K])
            out = rb(orc.linear_f32(src, rb(ws[li][pi])))
            out = rb(out + rb(bs[li][pi]))
            out = rb(_act(orc, p, out))
            if p.resid:
                out = rb(out + h)
            if p.dst == "h":
                h = out
            else:
                mix[p.dst] = out
    return h


def test_vision_block_projections_against_the_oracle(dev, orc):
    from sys1_amd.linear import Linear
    from sys1_amd.stacks import qwen35_vision
    cfg = qwen35_vision(1152, 4304, 1, "vision-1")
    M = 1000
    x = orc.fill_normal((M, 1152), 21)
    ws, bs = _params(orc, cfg, 300)
    h = to_gpu_bf16(x, torch)
    mix = {}
    print(f"[gpu] vision block projections M={M}", flush=True)
    for pi, p in enumerate(cfg.layers[0]):
        src = h if p.src == "h" else mix[p.src][:, p.src_off:p.src_off + p.K]
        lin = Linear(to_gpu_bf16(ws[0][pi], torch), to_gpu_bf16(bs[0][pi], torch), device=dev, blocked=True)
        gelu = "tanh" if "gelu_tanh" in p.name else False
        out = lin(src, residual=h if p.resid else None, gelu=gelu)
        ref = orc.linear_f32(to_np(src), ws[0][pi]) + orc.round_bf16(bs[0][pi])
        ref = _act(orc, p, ref)
        if p.resid:
            ref = ref + to_np(h)
        assert_parity(to_np(out), ref, f"vision {p.name}")
        if p.dst == "h":
            h = out
        else:
            mix[p.dst] = out


@pytest.mark.parametrize("M", [200, 3001])
def test_vision_stack_against_the_oracle_chain(dev, orc, M):
    from sys1_amd.stacks import ProjectionStack, qwen35_vision
    cfg = qwen35_vision(1152, 4304, 4, "vision-4")
    x = orc.fill_normal((M, 1152), 31 + M)
    ws, bs = _params(orc, cfg, 700)
    print(f"[gpu] vision stack 4 blocks M={M}", flush=True)
    stack = ProjectionStack(cfg, dev, M, weights=[[to_gpu_bf16(w, torch) for w in l] for l in ws],
                            biases=[[to_gpu_bf16(b, torch) for b in l] for l in bs], blocked=True)
    out = to_np(stack.forward(to_gpu_bf16(x, torch), M))
    emul = _oracle_chain(orc, cfg, x, ws, bs, True)
    f32 = _oracle_chain(orc, cfg, x, ws, bs, False)
    rel, _ = parity(out, emul)
    spread, _ = parity(emul, f32)
    print(f"[gpu]   vs bf16-rounding oracle chain {rel:.3e}; oracle chains differ by {spread:.3e}", flush=True)
    assert rel < max(4 * spread, 1e-3)
    assert_parity(out, f32, f"vision stack M={M} vs f32 chain")


def test_vision_stack_from_safetensors_checkpoint(dev, orc, tmp_path):
    """load_stack on a synthetic checkpoint in the reference's vision names
    (model.visual.blocks.{i}...; src/models/clef.rs:197): the stack runs the
    checkpoint's weights and biases, against the oracle chain of the same
    tensors."""
    st = pytest.importorskip("safetensors.torch")
    from sys1_amd import weights as W
    cfgj = {"vision_config": {"depth": 2, "hidden_size": 128, "intermediate_size": 344}}
    cfg = W.vision_config(cfgj)
    ws, bs = _params(orc, cfg, 900)
    leaves = ["attn.qkv", "attn.proj", "mlp.linear_fc1", "mlp.linear_fc2"]
    t = {}
    for i in range(2):
        for leaf, w, b in zip(leaves, ws[i], bs[i]):
            t[f"model.visual.blocks.{i}.{leaf}.weight"] = torch.from_numpy(w).to(torch.bfloat16)
            t[f"model.visual.blocks.{i}.{leaf}.bias"] = torch.from_numpy(b).to(torch.bfloat16)
    path = str(tmp_path / "vision.safetensors")
    st.save_file(t, path)
    M = 777
    print(f"[gpu] vision stack from a checkpoint M={M}", flush=True)
    stack = W.load_stack(path, "qwen35_vision", cfgj, dev, M)
    x = orc.fill_normal((M, 128), 5)
    out = to_np(stack.forward(to_gpu_bf16(x, torch), M))
    emul = _oracle_chain(orc, cfg, x, ws, bs, True)
    f32 = _oracle_chain(orc, cfg, x, ws, bs, False)
    rel, _ = parity(out, emul)
    spread, _ = parity(emul, f32)
    assert rel < max(4 * spread, 1e-3)
    assert_parity(out, f32, "vision checkpoint stack vs f32 chain")


def test_vision_merger_projections(dev, orc):
    """The tower's merger (src/archs/qwen35_vision.rs:261-268): LayerNorm,
    2x2 patches merged into rows of 4H, linear_fc1 4H->4H with bias and the
    exact GELU (candle gelu_erf), linear_fc2 4H->out with bias -- the bias +
    GELU and bias epilogues on merged rows, against the oracle."""
    from sys1_amd.linear import Linear
    H, out_h, M = 1152, 2048, 390
    W4 = 4 * H
    x = orc.round_bf16(orc.fill_normal((M, W4), 61))
    w1, b1 = orc.fill_normal((W4, W4), 62, 0.02), orc.fill_normal((W4,), 63, 0.02)
    w2, b2 = orc.fill_normal((out_h, W4), 64, 0.02), orc.fill_normal((out_h,), 65, 0.02)
    print(f"[gpu] vision merger M={M}", flush=True)
    fc1 = Linear(to_gpu_bf16(w1, torch), to_gpu_bf16(b1, torch), device=dev, blocked=True)
    fc2 = Linear(to_gpu_bf16(w2, torch), to_gpu_bf16(b2, torch), device=dev, blocked=True)
    a = fc1(to_gpu_bf16(x, torch), gelu=True)
    ref1 = orc.gelu_erf(orc.linear_f32(x, w1) + orc.round_bf16(b1))
    assert_parity(to_np(a), ref1, "merger fc1 + gelu")
    y = fc2(a)
    assert_parity(to_np(y), orc.linear_f32(to_np(a), w2) + orc.round_bf16(b2), "merger fc2")
    assert_parity(to_np(y), orc.linear_f32(ref1, w2) + b2, "merger chain vs f32")
