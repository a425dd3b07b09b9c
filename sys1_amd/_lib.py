"""ctypes binding of libsys1hip.so (include/sys1hip.h).

The shared library is the product: there is no Python or CPU fallback.  If
it is missing, importing this module raises, naming the build command.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsys1hip.so")

# Epilogue flags (include/sys1hip.h).
EPI_NONE = 0
EPI_BIAS = 1
EPI_GEGLU = 2
EPI_SWIGLU = 4
EPI_RESIDUAL = 8
EPI_GELU = 16
EPI_GELU_TANH = 64   # bias + tanh-approximate GELU
EPI_BLOCKED_W = 32   # not an epilogue: the weight is in the blocked layout
GATE_GROUP = 16

# Pre-norm kinds (include/sys1hip.h).
NORM_LAYER = 1
NORM_RMS = 2

OK = 0
EINVAL = -22
EALIGN = -14
EDEVICE = -19
ERANGE = -34

# Every symbol the header declares; the ABI test checks the library exports them.
EXPORTS = (
    "sys1hip_version", "sys1hip_init", "sys1hip_destroy", "sys1hip_set_stream",
    "sys1hip_sync", "sys1hip_last_error", "sys1hip_linear_bf16",
    "sys1hip_pack_gated_weight", "sys1hip_query_kernel", "sys1hip_set_kernel",
    "sys1hip_kernel_count", "sys1hip_kernel_name", "sys1hip_set_grid",
    "sys1hip_set_dp_tiles", "sys1hip_linear_rope_qkv_bf16", "sys1hip_fold_norm_weight",
    "sys1hip_norm_linear_bf16", "sys1hip_linear_conv_silu_bf16", "sys1hip_linear_bf16_noalloc",
    "sys1hip_blocked_weight_bytes", "sys1hip_pack_blocked_weight", "sys1hip_plan_kernel",
    "sys1hip_plan_kernel_strided", "sys1hip_linear_chain_bf16", "sys1hip_chain_status",
    "sys1hip_set_chain_wait", "sys1hip_chain_queue", "sys1hip_set_chain_trace",
)


class ChainProj(ctypes.Structure):
    """sys1hip_chain_proj: one projection of a chain launch."""
    _fields_ = [("x", ctypes.c_void_p), ("ldx", ctypes.c_int64),
                ("w", ctypes.c_void_p), ("ldw", ctypes.c_int64),
                ("residual", ctypes.c_void_p), ("ldr", ctypes.c_int64),
                ("y", ctypes.c_void_p), ("ldy", ctypes.c_int64),
                ("N", ctypes.c_int64), ("K", ctypes.c_int64),
                ("epilogue", ctypes.c_int32)]


CHAIN_MAX = 4  # projections per chain launch


class Sys1HipError(RuntimeError):
    """A failing sys1hip call: the return code and the library's message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"sys1hip error {code}: {message}")
        self.code = code


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m sys1_amd.build` "
            "(there is no fallback path)")
    L = ctypes.CDLL(LIB_PATH)
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    L.sys1hip_version.restype = ctypes.c_int
    L.sys1hip_version.argtypes = []
    L.sys1hip_init.argtypes = [ctypes.c_int, ctypes.POINTER(vp)]
    L.sys1hip_destroy.argtypes = [vp]
    L.sys1hip_set_stream.argtypes = [vp, vp]
    L.sys1hip_sync.argtypes = [vp]
    L.sys1hip_last_error.argtypes = [vp]
    L.sys1hip_last_error.restype = ctypes.c_char_p
    L.sys1hip_linear_bf16.argtypes = [vp, vp, i64, vp, i64, vp, vp, i64, vp, i64, i64, i64, i64, i32]
    L.sys1hip_linear_bf16_noalloc.argtypes = [vp, vp, i64, vp, i64, vp, vp, i64, vp, i64, i64, i64, i64,
                                              i32]
    L.sys1hip_pack_gated_weight.argtypes = [vp, vp, vp, i64, i64]
    L.sys1hip_blocked_weight_bytes.argtypes = [i64, i64]
    L.sys1hip_blocked_weight_bytes.restype = i64
    L.sys1hip_pack_blocked_weight.argtypes = [vp, vp, i64, vp, i64, i64]
    L.sys1hip_query_kernel.argtypes = [vp, i64, i64, i64, i32, ctypes.c_char_p, i64]
    L.sys1hip_plan_kernel.argtypes = [i32, i64, i64, i64, i32, ctypes.POINTER(i64), ctypes.c_char_p, i64]
    L.sys1hip_plan_kernel_strided.argtypes = [i32, i64, i64, i64, i64, i64, i32, ctypes.POINTER(i64),
                                              ctypes.c_char_p, i64]
    L.sys1hip_set_kernel.argtypes = [vp, i32]
    L.sys1hip_set_grid.argtypes = [vp, i32]
    L.sys1hip_set_dp_tiles.argtypes = [vp, i32]
    L.sys1hip_linear_rope_qkv_bf16.argtypes = [vp, vp, i64, vp, i64, vp, vp, i64, vp, vp, i64, i64, i64, i64]
    L.sys1hip_fold_norm_weight.argtypes = [vp, vp, vp, i32, vp, vp, i64, i64]
    L.sys1hip_norm_linear_bf16.argtypes = [vp, vp, i64, vp, i64, vp, i32, ctypes.c_float, vp, i64,
                                           i64, i64, i64, i32]
    L.sys1hip_linear_conv_silu_bf16.argtypes = [vp, vp, i64, vp, i64, i32, ctypes.c_float, vp, i64, vp,
                                                vp, i64, i64, i64, i64]
    L.sys1hip_linear_chain_bf16.argtypes = [vp, ctypes.POINTER(ChainProj), i32, i64]
    L.sys1hip_chain_status.argtypes = [vp, ctypes.POINTER(i32)]
    L.sys1hip_set_chain_wait.argtypes = [vp, i32, i32]
    L.sys1hip_set_chain_trace.argtypes = [vp, vp, i64]
    L.sys1hip_chain_queue.argtypes = [i32, i64, i32, ctypes.POINTER(i64), ctypes.POINTER(i32), i64]
    L.sys1hip_kernel_count.argtypes = []
    L.sys1hip_kernel_name.argtypes = [i32]
    L.sys1hip_kernel_name.restype = ctypes.c_char_p
    for name in ("sys1hip_init", "sys1hip_destroy", "sys1hip_set_stream", "sys1hip_sync",
                 "sys1hip_linear_bf16", "sys1hip_pack_gated_weight", "sys1hip_query_kernel",
                 "sys1hip_set_kernel", "sys1hip_set_grid", "sys1hip_set_dp_tiles",
                 "sys1hip_linear_rope_qkv_bf16", "sys1hip_fold_norm_weight",
                 "sys1hip_norm_linear_bf16", "sys1hip_linear_conv_silu_bf16", "sys1hip_kernel_count",
                 "sys1hip_linear_bf16_noalloc", "sys1hip_pack_blocked_weight", "sys1hip_plan_kernel",
                 "sys1hip_plan_kernel_strided", "sys1hip_linear_chain_bf16", "sys1hip_chain_status",
                 "sys1hip_set_chain_wait", "sys1hip_chain_queue", "sys1hip_set_chain_trace"):
        getattr(L, name).restype = ctypes.c_int
    _lib = L
    return L


def check(code: int, ctx=None) -> int:
    if code < 0:
        msg = load().sys1hip_last_error(ctx)
        raise Sys1HipError(code, msg.decode() if msg else "")
    return code


def plan_kernel(M: int, N: int, K: int, epilogue: int = 0, cus: int = 256,
                ldx: int | None = None, ldw: int | None = None) -> tuple[int, int, str]:
    """(kernel id, workgroups, plan name) that the library would choose for a
    projection on a GPU with `cus` compute units (no device needed); ldx /
    ldw default to K (contiguous rows)."""
    L = load()
    grid = ctypes.c_int64()
    buf = ctypes.create_string_buffer(96)
    kid = check(L.sys1hip_plan_kernel_strided(cus, M, N, K, ldx or K, ldw or K, epilogue,
                                              ctypes.byref(grid), buf, 96))
    return kid, grid.value, buf.value.decode()


def chain_queue(xcc: int, M: int, Ns: list[int]) -> list[tuple[int, int, int]]:
    """The chain kernel's tile queue of one XCD: (projection, row panel,
    column tile) in the order its workgroups take them."""
    L = load()
    n_arr = (ctypes.c_int64 * len(Ns))(*Ns)
    total = check(L.sys1hip_chain_queue(xcc, M, len(Ns), n_arr, None, 0))
    buf = (ctypes.c_int32 * (3 * total))()
    check(L.sys1hip_chain_queue(xcc, M, len(Ns), n_arr, buf, 3 * total))
    return [(buf[3 * i], buf[3 * i + 1], buf[3 * i + 2]) for i in range(total)]


def kernel_names() -> list[str]:
    L = load()
    return [L.sys1hip_kernel_name(i).decode() for i in range(L.sys1hip_kernel_count())]
