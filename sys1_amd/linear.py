"""The projection modules sys1's model code calls, on the gfx950 kernels.

`Linear` mirrors `candle_nn::Linear` as the reference builds and applies it:
`Linear::new(weight[out,in], bias?)` (src/archs/modernbert.rs:1036-1046,
src/archs/qwen35_text.rs:174-176, src/models/laya.rs:620-630) and
`xs.apply(&linear)` -> `Linear::forward` -> y = x.W^T (+ b) with the leading
dimensions of a contiguous input flattened.  The output is allocated fresh,
as candle's backend does; `forward_into` writes into a caller buffer instead.

`GatedLinear` is the Wi/gate-up projection with its gating fused in the
epilogue: ModernBERT's Wi + GeGLU (src/archs/modernbert.rs:521-533, CUDA op
src/kernels/modernbert.cu:4-29) and Qwen's gate/up + SwiGLU
(src/archs/qwen35_text.rs:232-240).  The optional `residual` argument fuses
the residual adds of src/archs/modernbert.rs:883,886 and
src/archs/qwen35_text.rs:938-939 into a projection.

Errors: shape/dtype/layout problems raise ValueError before any launch (the
reference bails through candle's Result); anything the library rejects
raises `Sys1HipError` with its message.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .device import HipDevice, load as load_device

_vp = ctypes.c_void_p


def _check_operand(t: torch.Tensor, name: str, dev: HipDevice) -> None:
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name}: expected bf16, got {t.dtype}")
    if t.device != dev.torch_device:
        raise ValueError(f"{name}: expected a tensor on {dev.torch_device}, got {t.device}")
    if t.dim() >= 1 and t.shape[-1] > 1 and t.stride(-1) != 1:
        raise ValueError(f"{name}: last dimension must be contiguous")


def _rows(t: torch.Tensor, name: str) -> tuple[torch.Tensor, int]:
    """View t as [rows, cols] and return it with its row stride (elements)."""
    if t.dim() == 2:
        return t, (t.stride(0) if t.shape[0] > 1 else t.shape[1])
    if not t.is_contiguous():
        raise ValueError(f"{name}: inputs with more than 2 dims must be contiguous")
    t2 = t.reshape(-1, t.shape[-1])
    return t2, t.shape[-1]


def linear_bf16(dev: HipDevice, x: torch.Tensor, w: torch.Tensor, out: torch.Tensor,
                epilogue: int = _lib.EPI_NONE, bias: torch.Tensor | None = None,
                residual: torch.Tensor | None = None, n: int | None = None) -> torch.Tensor:
    """Raw call of sys1hip_linear_bf16 on 2-D views: out = epi(x . w^T).
    With EPI_BLOCKED_W in `epilogue`, w is a blocked weight (BlockedWeight
    storage) of `n` rows."""
    M, K = x.shape
    blocked = bool(epilogue & _lib.EPI_BLOCKED_W)
    N = n if blocked else w.shape[0]
    dev.follow_torch_stream()
    _lib.check(dev._L.sys1hip_linear_bf16(
        dev.ctx,
        _vp(x.data_ptr()), x.stride(0) if M > 1 else K,
        _vp(w.data_ptr()), K if blocked else w.stride(0),
        _vp(bias.data_ptr()) if bias is not None else None,
        _vp(residual.data_ptr()) if residual is not None else None,
        (residual.stride(0) if M > 1 else residual.shape[1]) if residual is not None else 0,
        _vp(out.data_ptr()), out.stride(0) if M > 1 else out.shape[1],
        M, N, K, epilogue), dev.ctx)
    return out


def pack_blocked_weight(weight: torch.Tensor, device: HipDevice | None = None) -> torch.Tensor:
    """[N, K] row-major -> the blocked layout (sys1hip_pack_blocked_weight):
    32-row x 64-column blocks of 4 KB, so the weight-streaming kernels read
    4 KB of contiguous memory per 32 rows and k-step.  Returns a flat bf16
    tensor; calls on it pass EPI_BLOCKED_W and the row count."""
    dev = device or load_device(weight.device.index or 0)
    _check_operand(weight, "weight", dev)
    w = weight.contiguous()
    N, K = w.shape
    nbytes = dev._L.sys1hip_blocked_weight_bytes(N, K)
    if nbytes < 0:
        raise ValueError(f"bad weight shape {tuple(w.shape)}")
    packed = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=w.device)
    dev.follow_torch_stream()
    _lib.check(dev._L.sys1hip_pack_blocked_weight(dev.ctx, _vp(w.data_ptr()), K, _vp(packed.data_ptr()),
                                                   N, K), dev.ctx)
    return packed


class Linear:
    """y = x.W^T (+ b), weight [out, in] bf16 on the device.  blocked=True
    stores the weight in the blocked layout (pack_blocked_weight) instead of
    candle's row-major [out, in]: same results, read as contiguous 4 KB
    blocks by the weight-streaming kernels."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None = None,
                 device: HipDevice | None = None, blocked: bool = False):
        self.device = device or load_device(weight.device.index or 0)
        if weight.dim() != 2:
            raise ValueError(f"weight must be [out, in], got shape {tuple(weight.shape)}")
        _check_operand(weight, "weight", self.device)
        self.blocked = blocked
        self.weight = pack_blocked_weight(weight, self.device) if blocked else weight.contiguous()
        if bias is not None:
            _check_operand(bias, "bias", self.device)
            if bias.shape != (weight.shape[0],):
                raise ValueError(f"bias must be [{weight.shape[0]}], got {tuple(bias.shape)}")
            bias = bias.contiguous()
        self.bias = bias
        self.out_features, self.in_features = weight.shape

    def _epilogue(self, residual, gelu: bool | str) -> int:
        """gelu: False, True or "erf" (exact GELU, candle's gelu_erf: Laya
        scorer_in), or "tanh" (the tanh approximation, candle's gelu: the
        Qwen3.5 vision tower's fc1); either needs the bias."""
        e = _lib.EPI_BLOCKED_W if self.blocked else _lib.EPI_NONE
        if self.bias is not None:
            e |= _lib.EPI_BIAS
        if gelu not in (False, True, "erf", "tanh"):
            raise ValueError(f"gelu must be False, True, 'erf' or 'tanh', got {gelu!r}")
        if gelu:
            if self.bias is None:
                raise ValueError("the fused gelu epilogues need a bias (Laya scorer_in, vision fc1)")
            e |= _lib.EPI_GELU_TANH if gelu == "tanh" else _lib.EPI_GELU
        if residual is not None:
            e |= _lib.EPI_RESIDUAL
        return e

    def forward_into(self, x: torch.Tensor, out: torch.Tensor,
                     residual: torch.Tensor | None = None, gelu: bool | str = False) -> torch.Tensor:
        _check_operand(x, "x", self.device)
        if x.shape[-1] != self.in_features:
            raise ValueError(f"shape mismatch: x[..., {x.shape[-1]}] vs weight "
                             f"[{self.out_features}, {self.in_features}]")
        x2, _ = _rows(x, "x")
        o2, _ = _rows(out, "out")
        if o2.shape != (x2.shape[0], self.out_features):
            raise ValueError(f"out must be [{x2.shape[0]}, {self.out_features}], got {tuple(out.shape)}")
        r2 = None
        if residual is not None:
            _check_operand(residual, "residual", self.device)
            r2, _ = _rows(residual, "residual")
            if r2.shape != o2.shape:
                raise ValueError(f"residual must match the output shape {tuple(o2.shape)}")
        linear_bf16(self.device, x2, self.weight, o2, self._epilogue(residual, gelu),
                    self.bias, r2, n=self.out_features)
        return out

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None,
                gelu: bool | str = False) -> torch.Tensor:
        out = torch.empty(*x.shape[:-1], self.out_features, dtype=torch.bfloat16, device=x.device)
        return self.forward_into(x, out, residual, gelu)

    __call__ = forward


def pack_gated_weight(weight: torch.Tensor, device: HipDevice | None = None) -> torch.Tensor:
    """[2I, K] (gate rows then up rows) -> the interleaved layout the gated
    epilogue reads (groups of 16 gate rows followed by their 16 up rows)."""
    dev = device or load_device(weight.device.index or 0)
    _check_operand(weight, "weight", dev)
    w = weight.contiguous()
    packed = torch.empty_like(w)
    dev.follow_torch_stream()
    _lib.check(dev._L.sys1hip_pack_gated_weight(dev.ctx, _vp(w.data_ptr()), _vp(packed.data_ptr()),
                                                 w.shape[0], w.shape[1]), dev.ctx)
    return packed


class GatedLinear:
    """act(x.Wg^T) * (x.Wu^T) in one GEMM with the gate fused in the epilogue.

    `weight` is [2I, K] with the gate rows first (ModernBERT's Wi, chunked in
    two at src/archs/modernbert.rs:531-532) -- or pass gate and up separately
    (Qwen's gate_proj / up_proj, src/archs/qwen35_text.rs:205-231).
    activation: "gelu" (GeGLU, gelu_erf) or "silu" (SwiGLU)."""

    def __init__(self, weight: torch.Tensor | None = None, activation: str = "gelu",
                 gate: torch.Tensor | None = None, up: torch.Tensor | None = None,
                 device: HipDevice | None = None, packed: bool = False, blocked: bool = False):
        if weight is None:
            if gate is None or up is None:
                raise ValueError("pass either weight [2I, K] or both gate and up")
            weight = torch.cat([gate, up], 0)
        self.device = device or load_device(weight.device.index or 0)
        if activation not in ("gelu", "silu"):
            raise ValueError(f"activation must be 'gelu' or 'silu', got {activation!r}")
        if weight.dim() != 2 or weight.shape[0] % (2 * _lib.GATE_GROUP):
            raise ValueError(f"gated weight must be [2I, K] with I % {_lib.GATE_GROUP} == 0, "
                             f"got {tuple(weight.shape)}")
        self.epilogue = _lib.EPI_GEGLU if activation == "gelu" else _lib.EPI_SWIGLU
        self.weight = weight.contiguous() if packed else pack_gated_weight(weight, self.device)
        if blocked:  # the gate/up interleave first, then the blocked layout of that
            self.weight = pack_blocked_weight(self.weight, self.device)
            self.epilogue |= _lib.EPI_BLOCKED_W
        self.rows = weight.shape[0]
        self.in_features = weight.shape[1]
        self.out_features = weight.shape[0] // 2

    def forward_into(self, x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        _check_operand(x, "x", self.device)
        if x.shape[-1] != self.in_features:
            raise ValueError(f"shape mismatch: x[..., {x.shape[-1]}] vs K={self.in_features}")
        x2, _ = _rows(x, "x")
        o2, _ = _rows(out, "out")
        if o2.shape != (x2.shape[0], self.out_features):
            raise ValueError(f"out must be [{x2.shape[0]}, {self.out_features}]")
        return linear_bf16(self.device, x2, self.weight, o2, self.epilogue, n=self.rows)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out = torch.empty(*x.shape[:-1], self.out_features, dtype=torch.bfloat16, device=x.device)
        self.forward_into(x, out)
        return out

    __call__ = forward


def linear_no_bias_dtype(input: int, output: int, weight: torch.Tensor,
                         device: HipDevice | None = None) -> Linear:
    """src/archs/modernbert.rs:1036-1046: weight [output, input] cast to bf16."""
    if tuple(weight.shape) != (output, input):
        raise ValueError(f"expected weight [{output}, {input}], got {tuple(weight.shape)}")
    return Linear(weight.to(torch.bfloat16), None, device)
