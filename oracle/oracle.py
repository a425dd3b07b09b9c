"""numpy front end of the C oracle (oracle/oracle.c) -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may
import this module, and only as the checker or the timed CPU baseline; the
shipped package never does.  Every function cites the reference lines it
restates (paths relative to the sys1 reference tree).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE, "liboracle.so"],
                       check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_linear_f32.argtypes = [_f32p, _i64, _f32p, _i64, _f32p, _f32p, _i64, _i64, _i64, _i64]
        L.orc_linear_f64.argtypes = [_f32p, _i64, _f32p, _i64, _f32p, _f64p, _i64, _i64, _i64, _i64]
        L.orc_gelu_erf.argtypes = [ctypes.c_float]
        L.orc_gelu_erf.restype = ctypes.c_float
        L.orc_silu.argtypes = [ctypes.c_float]
        L.orc_silu.restype = ctypes.c_float
        L.orc_geglu.argtypes = [_f32p, _i64, _f32p, _i64, _i64, _i64]
        L.orc_swiglu.argtypes = [_f32p, _i64, _f32p, _i64, _f32p, _i64, _i64, _i64]
        L.orc_layer_norm.argtypes = [_f32p, _i64, _f32p, _f32p, ctypes.c_float, _f32p, _i64, _i64, _i64]
        L.orc_rms_norm.argtypes = [_f32p, _i64, _f32p, ctypes.c_float, _f32p, _i64, _i64, _i64]
        L.orc_conv_silu.argtypes = [_f32p, _i64, _f32p, ctypes.POINTER(ctypes.c_int32), _i64, _i64, _i64,
                                    ctypes.c_int, _f32p, _i64]
        L.orc_argmax.argtypes = [_f32p, _i64]
        L.orc_argmax.restype = _i64
        L.orc_round_bf16.argtypes = [ctypes.c_float]
        L.orc_round_bf16.restype = ctypes.c_float
        L.orc_round_bf16_array.argtypes = [_f32p, _i64]
        L.orc_fill_normal.argtypes = [_f32p, _i64, ctypes.c_uint64, ctypes.c_float]
        L.orc_pack_ragged.argtypes = [ctypes.c_uint64, _i64, _i64, _i64, ctypes.c_int,
                                      ctypes.POINTER(ctypes.c_int64), _i64]
        L.orc_pack_ragged.restype = _i64
        L.orc_gelu_erf_array.argtypes = [_f32p, _f32p, _i64]
        L.orc_silu_array.argtypes = [_f32p, _f32p, _i64]
        L.orc_gelu_tanh_array.argtypes = [_f32p, _f32p, _i64]
        L.orc_rope_tables.argtypes = [ctypes.c_double, _i64, _i64, _f32p, _f32p]
        L.orc_rope_qkv.argtypes = [_f32p, _i64, _f32p, _f32p, ctypes.POINTER(ctypes.c_int32),
                                   _i64, _i64, _i64, _f32p]
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray, t=_f32p):
    return a.ctypes.data_as(t)


def linear_f32(x, w, bias=None) -> np.ndarray:
    """y = x.W^T (+ b) in f32 -- candle_nn::Linear::forward as built by
    src/archs/modernbert.rs:1036-1046 (no bias) and src/models/laya.rs:620-630
    (bias).  x may be [..., K]; leading dims are flattened as candle does for a
    contiguous input."""
    x = _f32(x)
    w = _f32(w)
    lead = x.shape[:-1]
    K = x.shape[-1]
    N = w.shape[0]
    assert w.shape[1] == K, (x.shape, w.shape)
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    y = np.empty((M, N), np.float32)
    b = _f32(bias) if bias is not None else None
    if M and N:
        lib().orc_linear_f32(_p(x2), K, _p(w), K, _p(b) if b is not None else None,
                             _p(y), N, M, N, K)
    return y.reshape(*lead, N)


def linear_f64(x, w, bias=None) -> np.ndarray:
    """Same contract as linear_f32, accumulated and returned in float64."""
    x = _f32(x)
    w = _f32(w)
    lead = x.shape[:-1]
    K = x.shape[-1]
    N = w.shape[0]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    y = np.empty((M, N), np.float64)
    b = _f32(bias) if bias is not None else None
    if M and N:
        lib().orc_linear_f64(_p(x2), K, _p(w), K, _p(b) if b is not None else None,
                             _p(y, _f64p), N, M, N, K)
    return y.reshape(*lead, N)


def gelu_erf(v) -> np.ndarray:
    """0.5 v (1 + erf(v/sqrt2)) (src/kernels/modernbert.cu:9-14, candle gelu_erf)."""
    v = _f32(v)
    out = np.empty_like(v)
    lib().orc_gelu_erf_array(_p(v), _p(out), v.size)
    return out


def gelu_tanh(v) -> np.ndarray:
    """0.5 v (1 + tanh(sqrt(2/pi)(v + 0.044715 v^3))) (candle gelu, the
    Qwen3.5 vision tower's fc1: src/archs/qwen35_vision.rs:166-169)."""
    v = _f32(v)
    out = np.empty_like(v)
    lib().orc_gelu_tanh_array(_p(v), _p(out), v.size)
    return out


def silu(v) -> np.ndarray:
    """v / (1 + e^-v) (src/archs/qwen35_text.rs:239)."""
    v = _f32(v)
    out = np.empty_like(v)
    lib().orc_silu_array(_p(v), _p(out), v.size)
    return out


def geglu(projected) -> np.ndarray:
    """[M, 2I] -> gelu_erf(first I) * (second I) (src/archs/modernbert.rs:531-532)."""
    p = _f32(projected)
    M, two_i = p.reshape(-1, p.shape[-1]).shape
    I = two_i // 2
    out = np.empty((M, I), np.float32)
    lib().orc_geglu(_p(p), two_i, _p(out), I, M, I)
    return out.reshape(*p.shape[:-1], I)


def swiglu(gate, up) -> np.ndarray:
    """silu(gate) * up (src/archs/qwen35_text.rs:232-240)."""
    g = _f32(gate)
    u = _f32(up)
    I = g.shape[-1]
    M = g.size // I
    out = np.empty((M, I), np.float32)
    lib().orc_swiglu(_p(g), I, _p(u), I, _p(out), I, M, I)
    return out.reshape(g.shape)


def layer_norm(x, weight, bias, eps=1e-5) -> np.ndarray:
    """candle layer_norm with weight and bias (src/models/laya.rs:258)."""
    x = _f32(x)
    H = x.shape[-1]
    x2 = x.reshape(-1, H)
    y = np.empty_like(x2)
    g = _f32(weight)
    b = _f32(bias) if bias is not None else None
    lib().orc_layer_norm(_p(x2), H, _p(g), _p(b) if b is not None else None, eps, _p(y), H,
                         x2.shape[0], H)
    return y.reshape(x.shape)


def layer_norm_bf16(x, weight, eps=1e-5) -> np.ndarray:
    """ModernBERT's bias-free LayerNorm on bf16 activations
    (src/archs/modernbert.rs:1005-1034, `LayerNorm::new_no_bias`), as
    candle-nn 0.11.0's LayerNorm::forward computes it for a bf16 input
    without bias: in f32, centre by the mean, divide by sqrt(mean of squared
    deviations + eps), cast the normalised value to bf16, then multiply by
    the weight in bf16 (rounded)."""
    H = _f32(x).shape[-1]
    normed = round_bf16(layer_norm(x, np.ones(H, np.float32), None, eps))
    return round_bf16(normed * round_bf16(_f32(weight)))


def rms_norm(x, weight, eps=1e-6) -> np.ndarray:
    """Qwen3.5 RMSNorm, f32 result before the cast back to the input dtype
    (src/archs/qwen35_text.rs:178-203; alpha = 1 + weight)."""
    x = _f32(x)
    H = x.shape[-1]
    x2 = x.reshape(-1, H)
    y = np.empty_like(x2)
    w = _f32(weight)
    lib().orc_rms_norm(_p(x2), H, _p(w), eps, _p(y), H, x2.shape[0], H)
    return y.reshape(x.shape)


def conv_silu(projected, weight, positions, bf16=True) -> np.ndarray:
    """Qwen3.5 DeltaNet causal conv + SiLU over packed rows
    (src/archs/qwen35_text.rs:632-650): projected [M, C], weight [C, k]
    (the conv1d weight [C, 1, k] squeezed), positions [M] (each token's
    position within its sequence).  bf16=True follows the reference's bf16
    arithmetic (rounded products and partial sums)."""
    p = _f32(projected)
    w = _f32(weight)
    M, C = p.shape
    k = w.shape[1]
    pos = np.ascontiguousarray(positions, np.int32)
    out = np.empty((M, C), np.float32)
    lib().orc_conv_silu(_p(p), C, _p(w), pos.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), M, C, k,
                        1 if bf16 else 0, _p(out), C)
    return out


def argmax(v) -> int:
    """Lowest index among maxima (src/models/laya.rs:909-916)."""
    v = _f32(v)
    return int(lib().orc_argmax(_p(v), v.size))


def round_bf16(a) -> np.ndarray:
    """Round-to-nearest-even to bf16, returned as f32 values."""
    a = np.array(a, dtype=np.float32, copy=True)
    lib().orc_round_bf16_array(_p(a), a.size)
    return a


def to_bf16_bits(a) -> np.ndarray:
    """bf16 bit patterns (uint16) of RNE-rounded f32 values."""
    r = round_bf16(a)
    return (r.view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def fill_normal(shape, seed: int, std: float = 1.0) -> np.ndarray:
    """Seeded N(0, std^2) via SplitMix64 + Box-Muller (oracle.c:orc_fill_normal)."""
    out = np.empty(shape, np.float32)
    lib().orc_fill_normal(_p(out), out.size, seed & 0xFFFFFFFFFFFFFFFF, std)
    return out


def pack_ragged(seed: int, lo: int, hi: int, budget: int, exact: bool = False) -> np.ndarray:
    """Sequence lengths ~ U[lo,hi] drawn until the next would exceed `budget`."""
    cap = budget // max(lo, 1) + 2
    out = np.empty(cap, np.int64)
    n = lib().orc_pack_ragged(seed & 0xFFFFFFFFFFFFFFFF, lo, hi, budget, int(exact),
                              out.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), cap)
    return out[:n].copy()


# ----------------------------------------------------------------- chains ---

def modernbert_layer_f32(h, wqkv, wo, wi, wo2):
    """One ModernBERT layer's projection chain in f32, with the attention
    stand-in used throughout this build (attention is not on the projection
    path): the V block of the Wqkv output feeds Wo.
    Follows src/archs/modernbert.rs:857-887 (Layer::forward: residual adds at
    :883 and :886), :176-192 (Wqkv/Wo), :521-533 (Wi -> GeGLU -> Wo).  Norms are
    left out (not projections)."""
    H = h.shape[-1]
    qkv = linear_f32(h, wqkv)
    attn = qkv[:, 2 * H:3 * H]
    h1 = linear_f32(attn, wo) + h
    g = geglu(linear_f32(h1, wi))
    return linear_f32(g, wo2) + h1


def laya_scorer_f32(hidden_rows, ln_w, ln_b, w_in, b_in, w_out, b_out):
    """Decision logits: LN -> Linear(+b) -> gelu_erf -> Linear(+b)
    (src/models/laya.rs:510-520, norm eps 1e-5 at :258)."""
    z = layer_norm(hidden_rows, ln_w, ln_b, 1e-5)
    z = gelu_erf(linear_f32(z, w_in, b_in))
    return linear_f32(z, w_out, b_out)[:, 0]


def rope_tables(theta: float, dim: int, positions: int):
    """cos, sin [positions, dim/2] f32 of src/archs/modernbert.rs:67-83."""
    half = dim // 2
    c = np.empty((positions, half), np.float32)
    s = np.empty((positions, half), np.float32)
    lib().orc_rope_tables(float(theta), dim, positions, _p(c), _p(s))
    return c, s


def rope_qkv(qkv, cos, sin, positions, heads: int, dim: int) -> np.ndarray:
    """Fused RoPE + q/k/v split (src/kernels/modernbert.cu:31-74) on packed
    tokens: qkv [M, 3*heads*dim] -> planes [3, M, heads*dim]; positions[m] is
    token m's rotary position within its sequence."""
    qkv = _f32(qkv)
    M = qkv.shape[0]
    pos = np.ascontiguousarray(positions, np.int32)
    assert pos.shape == (M,) and qkv.shape[1] == 3 * heads * dim
    out = np.empty((3, M, heads * dim), np.float32)
    lib().orc_rope_qkv(_p(qkv), qkv.shape[1], _p(_f32(cos)), _p(_f32(sin)),
                       pos.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), M, heads, dim, _p(out))
    return out
