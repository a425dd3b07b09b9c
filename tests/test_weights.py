"""Checkpoint loading in the reference's tensor names (host side): tiny
synthetic safetensors checkpoints, written here, in ModernBERT and Qwen3.5
naming, some sharded."""
import json

import numpy as np
import pytest

torch = pytest.importorskip("torch")
st = pytest.importorskip("safetensors.torch")

from sys1_amd import weights as W  # noqa: E402

MB_CFG = {"hidden_size": 64, "intermediate_size": 96, "num_hidden_layers": 2, "num_attention_heads": 2}
QW_CFG = {"text_config": {"hidden_size": 64, "num_hidden_layers": 2, "num_attention_heads": 2,
                          "num_key_value_heads": 1, "head_dim": 16, "intermediate_size": 96,
                          "linear_num_key_heads": 2, "linear_key_head_dim": 8,
                          "linear_num_value_heads": 4, "linear_value_head_dim": 8,
                          "layer_types": ["linear_attention", "full_attention"]}}


def _t(g, *shape):
    return torch.randn(*shape, generator=g)


def _modernbert_ckpt(tmp_path, shards=1):
    g = torch.Generator().manual_seed(0)
    t = {"model.embeddings.tok_embeddings.weight": _t(g, 10, 64)}
    for i in range(2):
        p = f"model.layers.{i}."
        t[p + "attn.Wqkv.weight"] = _t(g, 192, 64)
        t[p + "attn.Wo.weight"] = _t(g, 64, 64)
        t[p + "mlp.Wi.weight"] = _t(g, 192, 64)
        t[p + "mlp.Wo.weight"] = _t(g, 64, 96)
        t[p + "mlp_norm.weight"] = _t(g, 64)
        if i > 0:  # ModernBERT's layer 0 has no attn_norm
            t[p + "attn_norm.weight"] = _t(g, 64)
    names = sorted(t)
    paths = []
    for s in range(shards):
        path = str(tmp_path / f"mb-{s}.safetensors")
        st.save_file({n: t[n].contiguous() for n in names[s::shards]}, path)
        paths.append(path)
    return t, paths


def test_modernbert_names_and_cast(tmp_path):
    t, paths = _modernbert_ckpt(tmp_path, shards=2)
    cfg = W.modernbert_config(MB_CFG)
    ws = W.read_projection_weights(paths, "modernbert", cfg)
    for i in range(2):
        p = f"model.layers.{i}."
        for got, n in zip(ws[i], ["attn.Wqkv", "attn.Wo", "mlp.Wi", "mlp.Wo"]):
            assert got.dtype == torch.bfloat16
            assert torch.equal(got, t[p + n + ".weight"].to(torch.bfloat16))


def test_modernbert_shape_and_missing_errors(tmp_path):
    t, _ = _modernbert_ckpt(tmp_path)
    bad = dict(t)
    bad["model.layers.1.attn.Wo.weight"] = torch.zeros(64, 32)
    path = str(tmp_path / "bad.safetensors")
    st.save_file(bad, path)
    with pytest.raises(ValueError, match="attn.Wo"):
        W.read_projection_weights(path, "modernbert", W.modernbert_config(MB_CFG))
    del bad["model.layers.1.attn.Wo.weight"]
    st.save_file(bad, path)
    with pytest.raises(KeyError):
        W.read_projection_weights(path, "modernbert", W.modernbert_config(MB_CFG))


def test_qwen35_concatenations_follow_layer_types(tmp_path):
    g = torch.Generator().manual_seed(1)
    c = QW_CFG["text_config"]
    kw, vw, nv = 16, 32, 4
    t = {}
    p0, p1 = "model.language_model.layers.0.", "model.language_model.layers.1."
    t[p0 + "linear_attn.in_proj_qkv.weight"] = _t(g, 2 * kw + vw, 64)
    t[p0 + "linear_attn.in_proj_z.weight"] = _t(g, vw, 64)
    t[p0 + "linear_attn.in_proj_b.weight"] = _t(g, nv, 64)
    t[p0 + "linear_attn.in_proj_a.weight"] = _t(g, nv, 64)
    t[p0 + "linear_attn.out_proj.weight"] = _t(g, 64, vw)
    t[p1 + "self_attn.q_proj.weight"] = _t(g, 2 * 2 * 16, 64)
    t[p1 + "self_attn.k_proj.weight"] = _t(g, 16, 64)
    t[p1 + "self_attn.v_proj.weight"] = _t(g, 16, 64)
    t[p1 + "self_attn.o_proj.weight"] = _t(g, 64, 2 * 16)
    for p in (p0, p1):
        t[p + "input_layernorm.weight"] = _t(g, 64)
        t[p + "post_attention_layernorm.weight"] = _t(g, 64)
        t[p + "mlp.gate_proj.weight"] = _t(g, 96, 64)
        t[p + "mlp.up_proj.weight"] = _t(g, 96, 64)
        t[p + "mlp.down_proj.weight"] = _t(g, 64, 96)
    path = str(tmp_path / "qwen.safetensors")
    st.save_file(t, path)
    cfgpath = tmp_path / "config.json"
    cfgpath.write_text(json.dumps(QW_CFG))
    cfg = W.qwen35_config(json.loads(cfgpath.read_text()))
    assert [l[0].name for l in cfg.layers] == ["in_proj_qkvzba", "q_k_v"]
    ws = W.read_projection_weights(path, "qwen35", cfg)
    b = lambda n: t[n].to(torch.bfloat16)
    assert torch.equal(ws[0][0], torch.cat([b(p0 + f"linear_attn.in_proj_{n}.weight") for n in ("qkv", "z", "b", "a")]))
    assert torch.equal(ws[0][1], b(p0 + "linear_attn.out_proj.weight"))
    assert torch.equal(ws[1][0], torch.cat([b(p1 + f"self_attn.{n}_proj.weight") for n in "qkv"]))
    assert torch.equal(ws[1][1], b(p1 + "self_attn.o_proj.weight"))
    for i, p in enumerate((p0, p1)):
        assert torch.equal(ws[i][2], torch.cat([b(p + "mlp.gate_proj.weight"), b(p + "mlp.up_proj.weight")]))
        assert torch.equal(ws[i][3], b(p + "mlp.down_proj.weight"))
    nw = W.read_norm_weights(path, "qwen35", cfg)
    for i, p in enumerate((p0, p1)):
        assert torch.equal(nw[i][0], t[p + "input_layernorm.weight"])
        assert nw[i][1] is None and nw[i][3] is None
        assert torch.equal(nw[i][2], t[p + "post_attention_layernorm.weight"])


def test_modernbert_norm_weights(tmp_path):
    t, paths = _modernbert_ckpt(tmp_path, shards=2)
    cfg = W.modernbert_config(MB_CFG)
    nw = W.read_norm_weights(paths, "modernbert", cfg)
    assert nw[0][0] is None  # layer 0: no attn_norm, the input passes through
    assert torch.equal(nw[1][0], t["model.layers.1.attn_norm.weight"])
    for i in range(2):
        assert torch.equal(nw[i][2], t[f"model.layers.{i}.mlp_norm.weight"])
        assert nw[i][1] is None and nw[i][3] is None
    bad = dict(t)
    del bad["model.layers.1.attn_norm.weight"]
    path = str(tmp_path / "nonorm.safetensors")
    st.save_file(bad, path)
    with pytest.raises(KeyError, match="attn_norm"):
        W.read_norm_weights(path, "modernbert", cfg)


VI_CFG = {"vision_config": {"depth": 2, "hidden_size": 32, "intermediate_size": 72, "num_heads": 2,
                            "in_channels": 3, "patch_size": 16, "temporal_patch_size": 2,
                            "spatial_merge_size": 2, "out_hidden_size": 64,
                            "num_position_embeddings": 64}}


def test_vision_weights_and_biases(tmp_path):
    """The vision tower's block Linears under model.visual.blocks.{i}
    (src/models/clef.rs:197, src/archs/qwen35_vision.rs:37-50): weights and
    biases in the stack's order and shapes, cast to bf16; a missing bias and
    a wrong bias shape raise."""
    g = torch.Generator().manual_seed(3)
    t = {}
    for i in range(2):
        p = f"model.visual.blocks.{i}."
        for leaf, (n, k) in {"attn.qkv": (96, 32), "attn.proj": (32, 32), "mlp.linear_fc1": (72, 32),
                             "mlp.linear_fc2": (32, 72)}.items():
            t[p + leaf + ".weight"] = _t(g, n, k)
            t[p + leaf + ".bias"] = _t(g, n)
        t[p + "norm1.weight"] = _t(g, 32)
    path = str(tmp_path / "v.safetensors")
    st.save_file(t, path)
    cfg = W.vision_config(VI_CFG)
    assert [p.name for p in cfg.layers[0]] == ["attn.qkv", "attn.proj", "mlp.fc1+gelu_tanh", "mlp.fc2"]
    ws = W.read_projection_weights(path, "qwen35_vision", cfg)
    bs = W.read_projection_biases(path, "qwen35_vision", cfg)
    for i in range(2):
        for q, w, b, leaf in zip(cfg.layers[i], ws[i], bs[i],
                                 ["attn.qkv", "attn.proj", "mlp.linear_fc1", "mlp.linear_fc2"]):
            ref = t[f"model.visual.blocks.{i}.{leaf}.weight"]
            assert w.dtype == torch.bfloat16 and torch.equal(w, ref.to(torch.bfloat16))
            assert torch.equal(b, t[f"model.visual.blocks.{i}.{leaf}.bias"].to(torch.bfloat16))
            assert tuple(w.shape) == (q.N, q.K) and tuple(b.shape) == (q.nout,)
    del t["model.visual.blocks.1.mlp.linear_fc2.bias"]
    st.save_file(t, path)
    with pytest.raises(KeyError, match="linear_fc2.bias"):
        W.read_projection_biases(path, "qwen35_vision", cfg)
    t["model.visual.blocks.1.mlp.linear_fc2.bias"] = _t(g, 33)
    st.save_file(t, path)
    with pytest.raises(ValueError, match="expected \\[32\\]"):
        W.read_projection_biases(path, "qwen35_vision", cfg)
    with pytest.raises(ValueError, match="unknown family"):
        W.read_norm_weights(path, "qwen35_vision", cfg)
