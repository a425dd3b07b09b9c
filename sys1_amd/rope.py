"""Wqkv with the rotary embedding fused into the epilogue.

The reference projects Wqkv (src/archs/modernbert.rs:184-187) and then runs
its fused RoPE + q/k/v split (src/archs/modernbert.rs:112-120, CUDA op
src/kernels/modernbert.cu:31-74): q and k rotated pairwise over columns
(c, c + head_dim/2) with f32 cos/sin tables at the token's position, v
passed through, the three written as separate planes.  `RopeQkvLinear` does
both in one launch (`sys1hip_linear_rope_qkv_bf16`), on packed tokens whose
positions come from `batching.positions` instead of the padded rectangle's
token % length.

`rope_tables` builds the tables as RotaryEmbedding::new does
(src/archs/modernbert.rs:67-83): inv_freq[i] = 1 / theta^(2i / dim) computed
in f64 and stored as f32, frequencies = position x inv_freq in f32, and
cos/sin of them as f32 (evaluated in f64, rounded once).  Building them is set-up work, done once per model on the
device with torch.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .device import HipDevice, load as load_device

_vp = ctypes.c_void_p
HEAD_DIM = 64


def rope_tables(theta: float, head_dim: int, max_positions: int,
                device: torch.device | str = "cuda") -> tuple[torch.Tensor, torch.Tensor]:
    """f32 cos, sin [max_positions, head_dim/2] on `device`."""
    idx = torch.arange(0, head_dim, 2, dtype=torch.float64)
    # theta^(2i/dim) in f64, rounded to f32, then the reciprocal in f32 -- the
    # reference's `1f32 / theta.powf(..) as f32`.
    inv_freq = 1.0 / torch.pow(torch.tensor(float(theta), dtype=torch.float64), idx / head_dim).float()
    pos = torch.arange(max_positions, dtype=torch.float32)
    freqs = pos[:, None] * inv_freq[None, :]
    # cos/sin of the f32 frequencies evaluated in f64 and rounded once: f32
    # library trig loses accuracy in its argument reduction at the 8192 rad
    # of the longest positions.
    f = freqs.double()
    return f.cos().float().contiguous().to(device), f.sin().float().contiguous().to(device)


class RopeQkvLinear:
    """Wqkv [3H, hidden] (q | k | v row blocks, H = heads * 64) with RoPE.

    forward(x [M, hidden] bf16, positions [M] int32) -> [3, M, H] bf16:
    planes q, k, v, each [M, heads, 64] -- the packed (varlen) layout the
    attention call consumes.  Positions must index rows of the tables; the
    kernel clamps any that do not (no out-of-table reads)."""

    def __init__(self, weight: torch.Tensor, heads: int, cos: torch.Tensor, sin: torch.Tensor,
                 device: HipDevice | None = None):
        self.device = device or load_device(weight.device.index or 0)
        if weight.dtype != torch.bfloat16 or weight.dim() != 2 or not weight.is_cuda:
            raise ValueError("weight must be a bf16 [3H, hidden] device tensor")
        if weight.shape[0] != 3 * heads * HEAD_DIM:
            raise ValueError(f"weight rows {weight.shape[0]} != 3 * heads * {HEAD_DIM}")
        for t, name in ((cos, "cos"), (sin, "sin")):
            if t.dtype != torch.float32 or t.dim() != 2 or t.shape[1] != HEAD_DIM // 2 or not t.is_cuda:
                raise ValueError(f"{name} must be an f32 [positions, {HEAD_DIM // 2}] device tensor")
        self.weight = weight.contiguous()
        self.heads = heads
        self.cos, self.sin = cos.contiguous(), sin.contiguous()
        self.hidden = weight.shape[1]

    def forward_into(self, x: torch.Tensor, positions: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] != self.hidden or x.stride(1) != 1:
            raise ValueError(f"x must be bf16 [M, {self.hidden}] with unit column stride")
        M = x.shape[0]
        if positions.dtype != torch.int32 or positions.shape != (M,) or not positions.is_contiguous():
            raise ValueError("positions must be a contiguous int32 [M] tensor")
        H = self.heads * HEAD_DIM
        if out.dtype != torch.bfloat16 or tuple(out.shape) != (3, M, H) or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous bf16 [3, {M}, {H}] tensor")
        self.device.follow_torch_stream()
        rc = self.device._L.sys1hip_linear_rope_qkv_bf16(
            self.device.ctx, _vp(x.data_ptr()), x.stride(0), _vp(self.weight.data_ptr()),
            self.weight.stride(0), _vp(self.cos.data_ptr()), _vp(self.sin.data_ptr()),
            self.cos.shape[0], _vp(positions.data_ptr()), _vp(out.data_ptr()), M, self.heads, HEAD_DIM, self.hidden)
        _lib.check(rc, self.device.ctx)
        return out

    def forward(self, x: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        out = torch.empty(3, x.shape[0], self.heads * HEAD_DIM, dtype=torch.bfloat16, device=x.device)
        return self.forward_into(x, positions, out)

    __call__ = forward
