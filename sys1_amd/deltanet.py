"""Qwen3.5 DeltaNet input projection with its causal conv + SiLU fused.

The reference projects the layer input to q|k|v (then z, b, a), runs a
depthwise causal conv of kernel 4 along each sequence over the q|k|v
channels, and applies SiLU (`project_and_mix`, src/archs/qwen35_text.rs:515-526;
`causal_conv_silu` :632-650; CUDA `qwen35_conv`, src/kernels/qwen35.cu:3-29).
`InProjConv` does that in one call of `sys1hip_linear_conv_silu_bf16` on
packed ragged rows: the conv reads earlier rows of the same sequence from
the GEMM's own output tile, and `positions` marks where sequences start.
With `norm_weight` the layer's input RMSNorm (:933) is fused as well.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .device import HipDevice, load as load_device
from .linear import _check_operand, _rows
from .norm import fold_norm_weight

_vp = ctypes.c_void_p


class InProjConv:
    """y = [silu(conv(x.Wqkv^T)) | x.Wzba^T] for the DeltaNet in_proj.

    weight: [N, K] bf16, rows q|k|v first (conv_channels of them), then any
    z, b, a rows.  conv_weight: [conv_channels, 1, 4] or [conv_channels, 4].
    norm_weight: the RMSNorm weight w (alpha = 1 + w) to fuse, or None."""

    def __init__(self, weight: torch.Tensor, conv_weight: torch.Tensor, conv_channels: int,
                 norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                 device: HipDevice | None = None):
        self.device = device or load_device(weight.device.index or 0)
        _check_operand(weight, "weight", self.device)
        if weight.dim() != 2 or not (0 < conv_channels <= weight.shape[0]) or conv_channels % 8:
            raise ValueError(f"conv_channels must be a multiple of 8 in (0, {weight.shape[0]}], "
                             f"got {conv_channels}")
        cw = conv_weight.reshape(conv_channels, -1)
        if cw.shape[1] != 4:
            raise ValueError(f"conv weight must have 4 taps, got shape {tuple(conv_weight.shape)}")
        self.conv_weight = cw.to(device=weight.device, dtype=torch.bfloat16).contiguous()
        self.conv_channels = conv_channels
        self.eps = float(eps)
        self.norm = _lib.NORM_RMS if norm_weight is not None else 0
        self.weight = (fold_norm_weight(weight, norm_weight, "rms", self.device)[0]
                       if norm_weight is not None else weight.contiguous())
        self.out_features, self.in_features = weight.shape

    def forward_into(self, x: torch.Tensor, positions: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        _check_operand(x, "x", self.device)
        if x.shape[-1] != self.in_features:
            raise ValueError(f"shape mismatch: x[..., {x.shape[-1]}] vs K={self.in_features}")
        x2, _ = _rows(x, "x")
        o2, _ = _rows(out, "out")
        M, K = x2.shape
        if o2.shape != (M, self.out_features):
            raise ValueError(f"out must be [{M}, {self.out_features}]")
        if positions.shape != (M,) or positions.dtype != torch.int32 or positions.device != x.device:
            raise ValueError("positions must be int32 [M] on the input's device")
        dev = self.device
        dev.follow_torch_stream()
        _lib.check(dev._L.sys1hip_linear_conv_silu_bf16(
            dev.ctx, _vp(x2.data_ptr()), x2.stride(0) if M > 1 else K,
            _vp(self.weight.data_ptr()), self.weight.stride(0), self.norm, self.eps,
            _vp(self.conv_weight.data_ptr()), self.conv_channels, _vp(positions.data_ptr()),
            _vp(o2.data_ptr()), o2.stride(0) if M > 1 else o2.shape[1],
            M, self.out_features, K), dev.ctx)
        return out

    def forward(self, x: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        out = torch.empty(*x.shape[:-1], self.out_features, dtype=torch.bfloat16, device=x.device)
        return self.forward_into(x, positions, out)

    __call__ = forward
