"""Projection stacks of the model families the reference serves, run layer by
layer on the gfx950 kernels -- the callers of the hot path.

Each stack issues exactly the projections of one transformer layer, in the
reference's order, with the fusions this build makes (gating in the Wi /
gate-up epilogue, residual adds in the output projections).  Everything that
is not a projection -- norms, attention, RoPE, the DeltaNet conv/recurrence --
is out of scope and replaced by a fixed stand-in: the output projection reads
a column slice of the input projection's output (the V block for ModernBERT,
the z block for DeltaNet, the q block for gated attention).  The oracle
chain in tests applies the same stand-in, so the comparison covers the whole
projection chain.

Layer structure followed:
  ModernBERT  src/archs/modernbert.rs:857-887 (Layer::forward), :176-192
              (Wqkv -> attention -> Wo), :521-533 (Wi -> GeGLU -> Wo)
  Qwen3.5     src/archs/qwen35_text.rs:932-940 (Layer::forward), :491-629
              (DeltaNet in_proj_qkv/z/b/a, out_proj), :312-411 (gated GQA
              q/k/v/o), :232-240 (SwiGLU MLP)
The DeltaNet in_proj_qkv|z|b|a and the attention q|k|v are each one GEMM over
concatenated weights (same input, row-independent outputs).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import torch

from . import _lib
from .device import HipDevice


@dataclass(frozen=True)
class Proj:
    """One projection: y = epi(x . W^T), W [N, K]."""
    name: str
    K: int
    N: int          # weight rows (2I for gated)
    epi: int
    src: str        # input buffer name
    src_off: int    # first input column
    dst: str        # output buffer name
    resid: str | None = None
    norm: str | None = None  # pre-norm of the input ("layer" / "rms"), fused when the stack has norms
    conv_ch: int = 0         # leading output columns under the DeltaNet causal conv + SiLU
    mixes_rows: bool = False  # its input comes from a row-mixing op (attention, the DeltaNet recurrence)
    bias: bool = False        # a bias vector [nout] (epi carries EPI_BIAS)

    @property
    def nout(self) -> int:
        return self.N // 2 if self.epi in (_lib.EPI_GEGLU, _lib.EPI_SWIGLU) else self.N

    def flops(self, M: int) -> int:
        return 2 * M * self.N * self.K

    def bytes(self, M: int) -> int:
        """Algorithmic HBM bytes: read x and W once, write y, read residual."""
        b = 2 * (M * self.K + self.N * self.K + M * self.nout)
        if self.bias:
            b += 2 * self.nout
        if self.resid:
            b += 2 * M * self.nout
        return b


@dataclass
class StackConfig:
    name: str
    hidden: int
    layers: list[list[Proj]] = field(default_factory=list)
    description: str = ""

    def flops_per_token(self) -> int:
        return sum(p.flops(1) for layer in self.layers for p in layer)

    def weight_bytes(self) -> int:
        return sum(2 * p.N * p.K for layer in self.layers for p in layer)


def modernbert(hidden: int, intermediate: int, layers: int, name: str) -> StackConfig:
    """Pre-norms: attn_norm before Wqkv in every layer but the first (whose
    attn_norm weight is absent, so `Norm::load(..).ok()` is None and the
    input passes through, src/archs/modernbert.rs:846-851,865-868), mlp_norm
    before Wi (:884)."""
    H, I = hidden, intermediate

    def layer(i: int) -> list[Proj]:
        return [
            Proj("Wqkv", H, 3 * H, _lib.EPI_NONE, "h", 0, "qkv", norm="layer" if i > 0 else None),
            Proj("attn.Wo", H, H, _lib.EPI_RESIDUAL, "qkv", 2 * H, "h", resid="h", mixes_rows=True),
            Proj("Wi+geglu", H, 2 * I, _lib.EPI_GEGLU, "h", 0, "act", norm="layer"),
            Proj("mlp.Wo", I, H, _lib.EPI_RESIDUAL, "act", 0, "h", resid="h"),
        ]
    return StackConfig(name, H, [layer(i) for i in range(layers)],
                       f"ModernBERT H={H} I={I} x{layers}: Wqkv {H}->{3 * H}, Wo {H}->{H}, "
                       f"Wi {H}->2x{I} (GeGLU), Wo {I}->{H}")


def qwen35(hidden: int, layers: int, heads: int, kv_heads: int, head_dim: int,
           intermediate: int, dn_qk: int, dn_v: int, dn_heads: int, o_in: int,
           name: str, layer_types: list[str] | None = None) -> StackConfig:
    """Hybrid decoder: gated GQA attention layers and DeltaNet layers, in the
    order of `layer_types` ("full_attention" / "linear_attention", the
    reference's config field, src/archs/qwen35_text.rs:45,905-912), by
    default every 4th layer attention (3:1).  o_in is the o_proj input width
    (BASELINE states heads*hd*2 for the small config where the reference
    builds heads*hd; src/archs/qwen35_text.rs:281-285)."""
    H = hidden
    mlp = [
        Proj("gate_up+swiglu", H, 2 * intermediate, _lib.EPI_SWIGLU, "h", 0, "act", norm="rms"),
        Proj("down", intermediate, H, _lib.EPI_RESIDUAL, "act", 0, "h", resid="h"),
    ]
    dn_in = 2 * dn_qk + 2 * dn_v + 2 * dn_heads  # qkv | z | b | a
    deltanet = [
        Proj("in_proj_qkvzba", H, dn_in, _lib.EPI_NONE, "h", 0, "mix", norm="rms",
             conv_ch=2 * dn_qk + dn_v),
        Proj("out_proj", dn_v, H, _lib.EPI_RESIDUAL, "mix", 2 * dn_qk + dn_v, "h", resid="h", mixes_rows=True),
    ] + mlp
    q_w = 2 * heads * head_dim
    attn_in = q_w + 2 * kv_heads * head_dim
    attention = [
        Proj("q_k_v", H, attn_in, _lib.EPI_NONE, "h", 0, "mix", norm="rms"),
        Proj("o_proj", o_in, H, _lib.EPI_RESIDUAL, "mix", 0, "h", resid="h", mixes_rows=True),
    ] + mlp
    if layer_types is None:
        layer_types = ["full_attention" if (i + 1) % 4 == 0 else "linear_attention" for i in range(layers)]
    if len(layer_types) != layers:
        raise ValueError(f"{len(layer_types)} layer types for {layers} layers")
    stack = [list(attention if t == "full_attention" else deltanet) for t in layer_types]
    return StackConfig(name, H, stack,
                       f"Qwen3.5 hybrid H={H} x{layers} (3:1 DeltaNet:GQA), in_proj {H}->{dn_in}, "
                       f"out {dn_v}->{H}, qkv {H}->{attn_in}, o {o_in}->{H}, "
                       f"SwiGLU {H}->2x{intermediate}, down {intermediate}->{H}")


def qwen35_vision(hidden: int, intermediate: int, depth: int, name: str) -> StackConfig:
    """The Qwen3.5 vision tower's blocks (src/archs/qwen35_vision.rs:15-57,
    163-171): every Linear has a bias (`dense`, :8-13); attn.qkv H->3H,
    attn.proj H->H + residual, mlp.linear_fc1 H->I + tanh-approximate GELU
    (candle `gelu`, :169), mlp.linear_fc2 I->H + residual.  The pre-block
    LayerNorms (eps 1e-6) and the attention are glue outside the stack, and
    attn.proj reads the v block as the attention output's stand-in, as the
    text stacks do.  The merger (once per image, on merged rows) is not part
    of the per-block stack."""
    H, I = hidden, intermediate
    B = _lib.EPI_BIAS

    def block() -> list[Proj]:
        return [
            Proj("attn.qkv", H, 3 * H, B, "h", 0, "qkv", bias=True),
            Proj("attn.proj", H, H, B | _lib.EPI_RESIDUAL, "qkv", 2 * H, "h", resid="h", mixes_rows=True,
                 bias=True),
            Proj("mlp.fc1+gelu_tanh", H, I, B | _lib.EPI_GELU_TANH, "h", 0, "act", bias=True),
            Proj("mlp.fc2", I, H, B | _lib.EPI_RESIDUAL, "act", 0, "h", resid="h", bias=True),
        ]
    return StackConfig(name, H, [block() for _ in range(depth)],
                       f"Qwen3.5 vision tower H={H} I={I} x{depth}: qkv {H}->{3 * H}, proj {H}->{H}, "
                       f"fc1 {H}->{I} (bias + tanh GELU), fc2 {I}->{H}, every Linear with a bias")


CONFIGS = {
    "modernbert-base": lambda: modernbert(768, 1152, 22, "modernbert-base"),
    "modernbert-large": lambda: modernbert(1024, 2624, 28, "modernbert-large"),
    "qwen35-small": lambda: qwen35(2048, 24, 16, 2, 128, 6144, 2048, 4096, 16, 4096,
                                   "qwen35-small"),
    "qwen35-27b": lambda: qwen35(5120, 64, 24, 4, 256, 17408, 2048, 6144, 48, 6144,
                                 "qwen35-27b"),
    # The reference reads the vision tower's sizes from the checkpoint's
    # config.json (VisionConfig, src/archs/qwen35_text.rs:63-75); these are
    # the published Qwen3-VL-class tower's (hidden 1152, intermediate 4304,
    # 27 blocks), not values the reference fixes.
    "qwen35-vision": lambda: qwen35_vision(1152, 4304, 27, "qwen35-vision"),
}


# sys1hip_linear_chain_bf16 runs a chain as a weight stream (32-column items
# over the whole K on every CU) up to this many tokens when every K is within
# the second bound (csrc/chain.hip: kStreamChainKernel), and as 128 x 192
# tiles on row panels otherwise.
STREAM_CHAIN_MAX_M = 64
STREAM_CHAIN_MAX_K = 2688

NORM_EPS = {"layer": 1e-5, "rms": 1e-6}  # ModernBERT layer_norm_eps, Qwen3.5 rms_norm_eps


class ProjectionStack:
    """Weights and activation buffers of a stack on one GPU, and the layer
    loop that enqueues its projections.

    norms=True fuses each projection's pre-norm (Proj.norm) into it
    (sys1hip_norm_linear_bf16) with the norm weights of a fresh model --
    LayerNorm weight 1, RMSNorm weight 0 (alpha 1) -- or `norm_weights`
    [layer][projection] (f32 [K] or None), with eps per kind (NORM_EPS, or
    `norm_eps`).  norms=False runs the projections alone.

    conv=True fuses the DeltaNet causal conv + SiLU into each in_proj
    (Proj.conv_ch columns; conv weights N(0, 0.5^2) or `conv_weights`
    [layer] -> [conv_ch, 4]); the calls then need per-token positions.

    chain=True runs each row-local run of projections (from one row-mixing
    op to the next: attention, the DeltaNet recurrence) as one launch
    (sys1hip_linear_chain_bf16, at most 4 projections each), bit for bit the
    results of the per-projection calls; it applies to stacks without fused
    norms or conv, and projections the chain kernel does not take (K not a
    multiple of 64 or below 192) run as single calls.

    blocked=True stores the weights in the blocked layout
    (linear.pack_blocked_weight: contiguous 4 KB per 32 rows and k-step,
    what the weight-streaming kernels read best), after any gate/up packing
    and norm folding; the in_proj calls with the conv fused keep the
    row-major layout."""

    def __init__(self, cfg: StackConfig, dev: HipDevice, max_tokens: int, seed: int = 0,
                 weights: list[list[torch.Tensor]] | None = None, w_std: float = 0.02,
                 norms: bool = False, norm_weights: list[list[torch.Tensor | None]] | None = None,
                 norm_eps: dict[str, float] | None = None, conv: bool = False,
                 conv_weights: list[torch.Tensor | None] | None = None, blocked: bool = False,
                 chain: bool = False, biases: list[list[torch.Tensor | None]] | None = None):
        self.cfg = cfg
        self.dev = dev
        self.max_tokens = max_tokens
        d = dev.torch_device
        g = torch.Generator(device=d)
        g.manual_seed(seed)
        from .linear import pack_blocked_weight, pack_gated_weight
        from .norm import fold_norm_weight
        self.norms = norms
        self.blocked = blocked
        if chain and (norms or conv):
            raise ValueError("chain=True runs projections without fused norms or conv")
        if norms and any(p.bias and p.norm for layer in cfg.layers for p in layer):
            raise ValueError("the fused pre-norm projections take no bias")
        self.chain = chain
        self.conv = conv
        self.conv_w: list[torch.Tensor | None] = []
        self.norm_eps = dict(NORM_EPS, **(norm_eps or {}))
        self.weights: list[list[torch.Tensor]] = []
        self.colsums: list[list[torch.Tensor | None]] = []
        self.biases: list[list[torch.Tensor | None]] = []
        for li, layer in enumerate(cfg.layers):
            ws, cs, bs = [], [], []
            for pi, p in enumerate(layer):
                bvec = None
                if p.bias:
                    bvec = biases[li][pi] if biases is not None else None
                    if bvec is None:
                        bvec = torch.randn(p.nout, generator=g, device=d, dtype=torch.float32) * w_std
                    bvec = bvec.to(device=d, dtype=torch.bfloat16).contiguous()
                    if bvec.shape != (p.nout,):
                        raise ValueError(f"{p.name}: bias must be [{p.nout}], got {tuple(bvec.shape)}")
                bs.append(bvec)
                if weights is not None:
                    w = weights[li][pi].to(device=d, dtype=torch.bfloat16).contiguous()
                else:
                    w = (torch.randn(p.N, p.K, generator=g, device=d, dtype=torch.float32) * w_std
                         ).to(torch.bfloat16)
                if p.epi in (_lib.EPI_GEGLU, _lib.EPI_SWIGLU):
                    w = pack_gated_weight(w, dev)
                c = None
                if norms and p.norm:
                    gw = norm_weights[li][pi] if norm_weights is not None else None
                    if gw is None:
                        gw = torch.ones(p.K) if p.norm == "layer" else torch.zeros(p.K)
                    w, c = fold_norm_weight(w, gw, p.norm, dev)
                if blocked and not (conv and p.conv_ch):
                    w = pack_blocked_weight(w, dev)
                ws.append(w)
                cs.append(c)
            self.weights.append(ws)
            self.colsums.append(cs)
            self.biases.append(bs)
            cwt = None
            convs = [p for p in layer if p.conv_ch]
            if conv and convs:
                cwt = conv_weights[li] if conv_weights is not None else None
                if cwt is None:
                    cwt = torch.randn(convs[0].conv_ch, 4, generator=g, device=d) * 0.5
                cwt = cwt.reshape(convs[0].conv_ch, 4).to(device=d, dtype=torch.bfloat16).contiguous()
            self.conv_w.append(cwt)
        widths: dict[str, int] = {"h": cfg.hidden}
        for layer in cfg.layers:
            for p in layer:
                widths[p.dst] = max(widths.get(p.dst, 0), p.nout)
        # Widths rounded up to 8 elements so every row stays 16-byte aligned.
        self.buffers = {k: torch.zeros(max_tokens, (v + 7) // 8 * 8, dtype=torch.bfloat16, device=d)
                        for k, v in widths.items()}
        self._fn = dev._L.sys1hip_linear_bf16
        self._norm_fn = dev._L.sys1hip_norm_linear_bf16
        self._conv_fn = dev._L.sys1hip_linear_conv_silu_bf16
        self._chain_fn = dev._L.sys1hip_linear_chain_bf16

    def _calls(self, x: torch.Tensor, M: int, positions: torch.Tensor | None = None) -> list[tuple]:
        """Argument tuples of every launch for M tokens (prepared once per M,
        so the enqueue loop is a plain sequence of C calls)."""
        assert x.shape[1] == self.cfg.hidden and x.dtype == torch.bfloat16 and x.stride(1) == 1
        if M > self.max_tokens:
            raise ValueError(f"M={M} exceeds the stack's max_tokens={self.max_tokens}")
        bufs = self.buffers
        calls = []
        first_resid = True
        for li, layer in enumerate(self.cfg.layers):
            for pi, p in enumerate(layer):
                if p.src == "h" and li == 0 and pi == 0:
                    src, ldx = x.data_ptr(), x.stride(0)
                elif p.src == "h" and first_resid:
                    src, ldx = x.data_ptr(), x.stride(0)
                else:
                    b = bufs[p.src]
                    src, ldx = b.data_ptr() + 2 * p.src_off, b.stride(0)
                dst = bufs[p.dst]
                rptr, ldr = None, 0
                if p.resid:
                    # The first residual reads the input x; later ones run in place on h.
                    if first_resid:
                        rptr, ldr = x.data_ptr(), x.stride(0)
                        first_resid = False
                    else:
                        rptr, ldr = bufs["h"].data_ptr(), bufs["h"].stride(0)
                w = self.weights[li][pi]
                if self.conv and p.conv_ch:
                    if positions is None or positions.numel() < M or positions.dtype != torch.int32:
                        raise ValueError("a stack with the conv fused needs int32 positions for every row")
                    normed = self.norms and p.norm == "rms"
                    calls.append((p, self._conv_fn, (
                        src, ldx, w.data_ptr(), w.stride(0), _lib.NORM_RMS if normed else 0,
                        self.norm_eps["rms"], self.conv_w[li].data_ptr(), p.conv_ch,
                        positions.data_ptr(), dst.data_ptr(), dst.stride(0), M, p.N, p.K)))
                elif self.norms and p.norm:
                    c = self.colsums[li][pi]
                    calls.append((p, self._norm_fn, (
                        src, ldx, w.data_ptr(), p.K if self.blocked else w.stride(0),
                        c.data_ptr() if c is not None else None,
                        _lib.NORM_LAYER if p.norm == "layer" else _lib.NORM_RMS, self.norm_eps[p.norm],
                        dst.data_ptr(), dst.stride(0), M, p.N, p.K,
                        p.epi | (_lib.EPI_BLOCKED_W if self.blocked else 0))))
                else:
                    bvec = self.biases[li][pi]
                    calls.append((p, self._fn, (src, ldx, w.data_ptr(), p.K if self.blocked else w.stride(0),
                                                bvec.data_ptr() if bvec is not None else None, rptr, ldr,
                                                dst.data_ptr(), dst.stride(0), M, p.N, p.K,
                                                p.epi | (_lib.EPI_BLOCKED_W if self.blocked else 0))))
        return calls

    @staticmethod
    def _chainable(p: Proj) -> bool:
        return p.K % 64 == 0 and p.K >= 192 and p.epi in (
            _lib.EPI_NONE, _lib.EPI_RESIDUAL, _lib.EPI_GEGLU, _lib.EPI_SWIGLU)

    def _chain_calls(self, calls: list[tuple], M: int) -> list[tuple]:
        """Group the per-projection calls into chain launches: a run ends
        before a projection whose input is row-mixed, after CHAIN_MAX
        projections, and around a projection the chain kernel does not take
        (that one stays a single call)."""
        out, run = [], []

        def flush():
            if not run:
                return
            arr = (_lib.ChainProj * len(run))()
            for i, (p, _, a) in enumerate(run):
                src, ldx, w, ldw, _bias, rptr, ldr, dst, ldy, _M, N, K, epi = a
                arr[i] = _lib.ChainProj(src, ldx, w, ldw, rptr, ldr, dst, ldy, N, K, epi)
            out.append((tuple(p for p, _, _ in run), self._chain_fn, (self.dev.ctx, arr, len(run), M)))
            run.clear()

        for p, fn, a in calls:
            if fn is not self._fn or not self._chainable(p):
                flush()
                out.append((p, fn, a))
                continue
            if p.mixes_rows or len(run) == _lib.CHAIN_MAX:
                flush()
            run.append((p, fn, a))
        flush()
        return out

    def prepare(self, x: torch.Tensor, M: int, positions: torch.Tensor | None = None):
        """[(projection, C function, argument tuple)] of every launch (a chain
        launch carries the tuple of its projections)."""
        ctx = self.dev.ctx
        out = []
        calls = self._calls(x, M, positions)
        if self.chain:
            calls = self._chain_calls(calls, M)
        for p, fn, args in calls:
            if fn is self._chain_fn:
                out.append((p, fn, args))
                continue
            ptrs = ((0, 2, 4, 7) if fn is self._norm_fn else (0, 2, 6, 8, 9) if fn is self._conv_fn
                    else (0, 2, 4, 5, 7))
            out.append((p, fn, (ctx, *[ctypes.c_void_p(a) if i in ptrs and a is not None else a
                                      for i, a in enumerate(args)])))
        return out

    def run_prepared(self, prepared) -> None:
        for _, fn, args in prepared:
            rc = fn(*args)
            if rc:
                _lib.check(rc, self.dev.ctx)

    def forward(self, x: torch.Tensor, M: int, positions: torch.Tensor | None = None,
                check: bool | None = None) -> torch.Tensor:
        """Enqueue the whole stack for the first M rows of x; returns the
        hidden-state buffer (first M rows valid once the stream reaches it).

        check (default: on for a stack with chains) synchronises and reads
        the chain launches' error word (sys1hip_chain_status): a chain whose
        bounded dependency wait expired left invalid rows, and this raises
        RuntimeError instead of returning them.  Callers that enqueue
        without synchronising (run_prepared, graph capture) read it with
        HipDevice.chain_status themselves."""
        self.dev.follow_torch_stream()
        self.run_prepared(self.prepare(x, M, positions))
        if self.chain if check is None else check:
            flags = self.dev.chain_status()
            if flags:
                raise RuntimeError(f"projection chain launch failed (sys1hip_chain_status flags {flags}: "
                                   "1 = a dependency wait expired, 2 = a queue was not drained, "
                                   "4 = a workgroup on an unexpected XCD); the outputs are not valid")
        return self.buffers["h"][:M, :self.cfg.hidden]
