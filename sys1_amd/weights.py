"""Projection weights from safetensors checkpoints, in the reference's names.

The reference memory-maps safetensors shards into a VarBuilder
(src/models/laya.rs:210-216, src/models/clef.rs:176-192) and builds each
projection with `Linear::new(weight[out,in], None)` cast to the compute dtype
(linear_no_bias_dtype, src/archs/modernbert.rs:1036-1046; linear,
src/archs/qwen35_text.rs:174-176).  This module reads the same tensors by
the same names, casts them to bf16 [out, in], and concatenates the row
blocks the projection stacks fuse into one GEMM:

  ModernBERT  model.layers.{i}.attn.Wqkv | attn.Wo | mlp.Wi | mlp.Wo
              (src/archs/modernbert.rs:156-167,503-514,922)
  Qwen3.5     model.language_model.layers.{i}.
                linear_attn.in_proj_qkv|in_proj_z|in_proj_b|in_proj_a -> one
                linear_attn.out_proj
                self_attn.q_proj|k_proj|v_proj -> one, self_attn.o_proj
                mlp.gate_proj|up_proj -> one (gate rows first), mlp.down_proj
              (src/archs/qwen35_text.rs:205-240,266-285,441-478,905-928)
  Vision      model.visual.blocks.{i}.attn.qkv | attn.proj | mlp.linear_fc1 |
              mlp.linear_fc2, each with its .bias
              (src/models/clef.rs:197, src/archs/qwen35_vision.rs:8-13,37-50)

Pre-norm weights (for a stack with its norms fused) by the same names:
  ModernBERT  layers.{i}.attn_norm (before Wqkv; absent in layer 0),
              layers.{i}.mlp_norm (before Wi)  (src/archs/modernbert.rs:846-852)
  Qwen3.5     layers.{i}.input_layernorm (before in_proj / q,k,v),
              layers.{i}.post_attention_layernorm (before gate/up)
              (src/archs/qwen35_text.rs:916-927)

`read_projection_weights` / `read_projection_biases` / `read_norm_weights` are host-only (CPU tensors,
shapes validated against the stack); `load_stack` puts them on the device as
a ProjectionStack (gated weights pre-packed and norm weights folded once
there).
"""
from __future__ import annotations

import json
import os

import torch

from .stacks import StackConfig, modernbert, qwen35, qwen35_vision

MODERNBERT_PREFIX = "model."
QWEN35_PREFIX = "model.language_model."
VISION_PREFIX = "model.visual."  # src/models/clef.rs:197
FAMILIES = ("modernbert", "qwen35", "qwen35_vision")
_PREFIX = {"modernbert": MODERNBERT_PREFIX, "qwen35": QWEN35_PREFIX, "qwen35_vision": VISION_PREFIX}


def modernbert_config(config: dict, name: str = "modernbert") -> StackConfig:
    """Stack of a ModernBERT config.json (hidden_size, intermediate_size,
    num_hidden_layers)."""
    return modernbert(config["hidden_size"], config["intermediate_size"],
                      config["num_hidden_layers"], name)


def qwen35_config(config: dict, name: str = "qwen35") -> StackConfig:
    """Stack of a Qwen3.5 config.json (its text_config when nested), with the
    reference's widths: o_proj reads heads*head_dim (src/archs/qwen35_text.rs:281-285)."""
    c = config.get("text_config", config)
    return qwen35(c["hidden_size"], c["num_hidden_layers"], c["num_attention_heads"],
                  c["num_key_value_heads"], c["head_dim"], c["intermediate_size"],
                  c["linear_num_key_heads"] * c["linear_key_head_dim"],
                  c["linear_num_value_heads"] * c["linear_value_head_dim"],
                  c["linear_num_value_heads"], c["num_attention_heads"] * c["head_dim"], name,
                  layer_types=c["layer_types"])


def vision_config(config: dict, name: str = "qwen35-vision") -> StackConfig:
    """Stack of a Qwen3.5 config.json's vision_config (hidden_size,
    intermediate_size, depth: src/archs/qwen35_text.rs:63-75)."""
    c = config.get("vision_config", config)
    return qwen35_vision(c["hidden_size"], c["intermediate_size"], c["depth"], name)


def _vision_leaf(i: int, name: str) -> str:
    leaf = {"attn.qkv": "attn.qkv", "attn.proj": "attn.proj", "mlp.fc1+gelu_tanh": "mlp.linear_fc1",
            "mlp.fc2": "mlp.linear_fc2"}[name]
    return f"blocks.{i}.{leaf}"  # src/archs/qwen35_vision.rs:37-50


def _names(family: str, cfg: StackConfig, prefix: str) -> list[list[list[str]]]:
    """Per layer, per projection of the stack: the checkpoint tensors whose
    rows it concatenates."""
    out = []
    for i, layer in enumerate(cfg.layers):
        p = f"{prefix}layers.{i}."
        if family == "qwen35_vision":
            out.append([[f"{prefix}{_vision_leaf(i, q.name)}.weight"] for q in layer])
            continue
        if family == "modernbert":
            out.append([[p + "attn.Wqkv.weight"], [p + "attn.Wo.weight"], [p + "mlp.Wi.weight"],
                        [p + "mlp.Wo.weight"]])
            continue
        mlp = [[p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight"], [p + "mlp.down_proj.weight"]]
        if layer[0].name == "q_k_v":
            out.append([[p + f"self_attn.{n}_proj.weight" for n in "qkv"],
                        [p + "self_attn.o_proj.weight"]] + mlp)
        else:
            out.append([[p + f"linear_attn.in_proj_{n}.weight" for n in ("qkv", "z", "b", "a")],
                        [p + "linear_attn.out_proj.weight"]] + mlp)
    return out


def _index(paths: list[str]) -> dict[str, str]:
    from safetensors import safe_open
    where = {}
    for path in paths:
        with safe_open(path, framework="pt", device="cpu") as f:
            for k in f.keys():
                where[k] = path
    return where


def read_projection_weights(paths: str | list[str], family: str, cfg: StackConfig,
                            prefix: str | None = None) -> list[list[torch.Tensor]]:
    """bf16 [N, K] CPU tensors per layer and projection of `cfg`, read from
    safetensors shards (names as the reference loads them).  Raises KeyError
    for a missing tensor and ValueError for a shape that does not match the
    stack."""
    from safetensors import safe_open
    if family not in FAMILIES:
        raise ValueError(f"unknown family {family!r}")
    paths = [paths] if isinstance(paths, (str, os.PathLike)) else list(paths)
    prefix = prefix if prefix is not None else _PREFIX[family]
    where = _index(paths)
    handles = {p: safe_open(p, framework="pt", device="cpu") for p in paths}
    weights = []
    for layer, names in zip(cfg.layers, _names(family, cfg, prefix)):
        ws = []
        for proj, parts in zip(layer, names):
            blocks = []
            for n in parts:
                if n not in where:
                    raise KeyError(f"checkpoint has no tensor {n}")
                blocks.append(handles[where[n]].get_tensor(n).to(torch.bfloat16))
            w = torch.cat(blocks, 0) if len(blocks) > 1 else blocks[0]
            if tuple(w.shape) != (proj.N, proj.K):
                raise ValueError(f"{'+'.join(parts)}: shape {tuple(w.shape)}, the stack's {proj.name} "
                                 f"expects [{proj.N}, {proj.K}]")
            ws.append(w.contiguous())
        weights.append(ws)
    return weights


def read_projection_biases(paths: str | list[str], family: str, cfg: StackConfig,
                           prefix: str | None = None) -> list[list[torch.Tensor | None]]:
    """bf16 [nout] CPU tensors of the projections with a bias (Proj.bias;
    the vision tower's `dense` Linears, src/archs/qwen35_vision.rs:8-13),
    None elsewhere.  KeyError / ValueError as above."""
    from safetensors import safe_open
    if family not in FAMILIES:
        raise ValueError(f"unknown family {family!r}")
    paths = [paths] if isinstance(paths, (str, os.PathLike)) else list(paths)
    prefix = prefix if prefix is not None else _PREFIX[family]
    where = _index(paths)
    handles = {p: safe_open(p, framework="pt", device="cpu") for p in paths}
    out = []
    for layer, names in zip(cfg.layers, _names(family, cfg, prefix)):
        row = []
        for proj, parts in zip(layer, names):
            if not proj.bias:
                row.append(None)
                continue
            if len(parts) != 1 or not parts[0].endswith(".weight"):
                raise ValueError(f"{proj.name}: no single Linear to read a bias of")
            n = parts[0][: -len("weight")] + "bias"
            if n not in where:
                raise KeyError(f"checkpoint has no tensor {n}")
            b = handles[where[n]].get_tensor(n).to(torch.bfloat16)
            if tuple(b.shape) != (proj.nout,):
                raise ValueError(f"{n}: shape {tuple(b.shape)}, expected [{proj.nout}]")
            row.append(b.contiguous())
        out.append(row)
    return out


def read_norm_weights(paths: str | list[str], family: str, cfg: StackConfig,
                      prefix: str | None = None) -> list[list[torch.Tensor | None]]:
    """f32 [K] CPU tensors of the pre-norm of each projection with one
    (Proj.norm), None elsewhere.  KeyError / ValueError as above."""
    from safetensors import safe_open
    if family not in ("modernbert", "qwen35"):
        raise ValueError(f"norm weights: unknown family {family!r} (the vision stack has no fused norms)")
    paths = [paths] if isinstance(paths, (str, os.PathLike)) else list(paths)
    prefix = prefix if prefix is not None else _PREFIX[family]
    where = _index(paths)
    handles = {p: safe_open(p, framework="pt", device="cpu") for p in paths}
    out = []
    for i, layer in enumerate(cfg.layers):
        row = []
        for proj in layer:
            if not proj.norm:
                row.append(None)
                continue
            if family == "modernbert":
                leaf = "attn_norm" if proj.name == "Wqkv" else "mlp_norm"
            else:
                leaf = "post_attention_layernorm" if proj.name.startswith("gate_up") else "input_layernorm"
            n = f"{prefix}layers.{i}.{leaf}.weight"
            if n not in where:
                raise KeyError(f"checkpoint has no tensor {n}")
            g = handles[where[n]].get_tensor(n).to(torch.float32)
            if tuple(g.shape) != (proj.K,):
                raise ValueError(f"{n}: shape {tuple(g.shape)}, expected [{proj.K}]")
            row.append(g.contiguous())
        out.append(row)
    return out


def load_stack(paths: str | list[str], family: str, config: dict | str, dev, max_tokens: int,
               prefix: str | None = None, norms: bool = False):
    """ProjectionStack on `dev` with a checkpoint's projection weights (and,
    with norms=True, its pre-norm weights fused, with the config's eps)."""
    from .stacks import ProjectionStack
    if isinstance(config, (str, os.PathLike)):
        with open(config) as f:
            config = json.load(f)
    if family not in FAMILIES:
        raise ValueError(f"unknown family {family!r}")
    cfg = (modernbert_config(config) if family == "modernbert" else qwen35_config(config)
           if family == "qwen35" else vision_config(config))
    weights = read_projection_weights(paths, family, cfg, prefix)
    biases = read_projection_biases(paths, family, cfg, prefix) if family == "qwen35_vision" else None
    nw, eps = None, None
    if norms:
        nw = read_norm_weights(paths, family, cfg, prefix)
        c = config.get("text_config", config)
        eps = ({"layer": float(c.get("layer_norm_eps", 1e-5))} if family == "modernbert"
               else {"rms": float(c.get("rms_norm_eps", 1e-6))})
    return ProjectionStack(cfg, dev, max_tokens, weights=weights, norms=norms, norm_weights=nw,
                           norm_eps=eps, biases=biases)
