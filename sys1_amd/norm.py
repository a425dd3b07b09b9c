"""Pre-norm projections: the norm in front of a projection, fused into it.

The reference normalises the residual stream and then projects it:
  ModernBERT  `xs.apply(&attn_norm)` -> Wqkv, `xs.apply(&mlp_norm)` -> Wi
              (src/archs/modernbert.rs:865-868,884; the norm is a bias-free
              LayerNorm, :1005-1034)
  Qwen3.5     `input_norm.forward(x)` -> in_proj / q,k,v, `post_norm.forward`
              -> gate/up (src/archs/qwen35_text.rs:933,939; RMSNorm with
              alpha = 1 + weight, :178-203)
`NormLinear` does both in one call of `sys1hip_norm_linear_bf16`: the norm
weight is folded into the projection weight once here, and every call
computes the rows' statistics and projects the raw activations, applying
r_m (acc - mu_m c_n) (LayerNorm) or r_m acc (RMSNorm) to the accumulators.
A gated projection (Wi + GeGLU, gate/up + SwiGLU) is packed first and then
folded, so the column sums follow the packed order.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .device import HipDevice, load as load_device
from .linear import _check_operand, _rows, pack_blocked_weight, pack_gated_weight

_vp = ctypes.c_void_p
KINDS = {"layer": _lib.NORM_LAYER, "rms": _lib.NORM_RMS}


def fold_norm_weight(weight: torch.Tensor, gamma: torch.Tensor, kind: str,
                     device: HipDevice | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
    """bf16 weight [N, K] and norm weight [K] -> (folded weight, column sums
    [N] f32 for LayerNorm, None for RMSNorm)."""
    dev = device or load_device(weight.device.index or 0)
    if kind not in KINDS:
        raise ValueError(f"norm kind must be one of {sorted(KINDS)}, got {kind!r}")
    _check_operand(weight, "weight", dev)
    if weight.dim() != 2 or gamma.shape != (weight.shape[1],):
        raise ValueError(f"gamma must be [{weight.shape[-1]}], got {tuple(gamma.shape)}")
    w = weight.contiguous()
    g = gamma.to(device=w.device, dtype=torch.float32).contiguous()
    out = torch.empty_like(w)
    colsum = torch.empty(w.shape[0], dtype=torch.float32, device=w.device) if kind == "layer" else None
    dev.follow_torch_stream()
    _lib.check(dev._L.sys1hip_fold_norm_weight(
        dev.ctx, _vp(w.data_ptr()), _vp(g.data_ptr()), KINDS[kind], _vp(out.data_ptr()),
        _vp(colsum.data_ptr()) if colsum is not None else None, w.shape[0], w.shape[1]), dev.ctx)
    return out, colsum


class NormLinear:
    """y = proj(norm(x)) with the norm fused.

    weight: [N, K] bf16 ([out, in]); for gated=... [2I, K] with the gate rows
    first.  gamma: the norm's weight [K] (LayerNorm weight, or the RMSNorm
    weight w of alpha = 1 + w).  kind: "layer" or "rms".  gated: None,
    "gelu" (GeGLU, with LayerNorm) or "silu" (SwiGLU, with RMSNorm).
    blocked=True stores the folded weight in the blocked layout
    (pack_blocked_weight); the results are those of the row-major weight."""

    def __init__(self, weight: torch.Tensor, gamma: torch.Tensor, kind: str, eps: float,
                 gated: str | None = None, device: HipDevice | None = None, blocked: bool = False):
        self.device = device or load_device(weight.device.index or 0)
        if kind not in KINDS:
            raise ValueError(f"norm kind must be one of {sorted(KINDS)}, got {kind!r}")
        epi = {None: _lib.EPI_NONE, "gelu": _lib.EPI_GEGLU, "silu": _lib.EPI_SWIGLU}.get(gated, -1)
        if epi < 0:
            raise ValueError(f"gated must be None, 'gelu' or 'silu', got {gated!r}")
        self.kind, self.eps, self.epilogue = kind, float(eps), epi
        w = pack_gated_weight(weight, self.device) if gated else weight
        self.weight, self.colsum = fold_norm_weight(w, gamma, kind, self.device)
        self.rows = self.weight.shape[0]
        self.blocked = blocked
        if blocked:  # fold (and gate/up interleave) first, then the blocked layout of that
            self.weight = pack_blocked_weight(self.weight, self.device)
        self.in_features = weight.shape[1]
        self.out_features = weight.shape[0] // 2 if gated else weight.shape[0]

    def forward_into(self, x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        _check_operand(x, "x", self.device)
        if x.shape[-1] != self.in_features:
            raise ValueError(f"shape mismatch: x[..., {x.shape[-1]}] vs K={self.in_features}")
        x2, _ = _rows(x, "x")
        o2, _ = _rows(out, "out")
        M, K = x2.shape
        if o2.shape != (M, self.out_features):
            raise ValueError(f"out must be [{M}, {self.out_features}]")
        dev = self.device
        dev.follow_torch_stream()
        _lib.check(dev._L.sys1hip_norm_linear_bf16(
            dev.ctx, _vp(x2.data_ptr()), x2.stride(0) if M > 1 else K,
            _vp(self.weight.data_ptr()), K if self.blocked else self.weight.stride(0),
            _vp(self.colsum.data_ptr()) if self.colsum is not None else None,
            KINDS[self.kind], self.eps,
            _vp(o2.data_ptr()), o2.stride(0) if M > 1 else o2.shape[1],
            M, self.rows, K, self.epilogue | (_lib.EPI_BLOCKED_W if self.blocked else 0)), dev.ctx)
        return out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out = torch.empty(*x.shape[:-1], self.out_features, dtype=torch.bfloat16, device=x.device)
        return self.forward_into(x, out)

    __call__ = forward
