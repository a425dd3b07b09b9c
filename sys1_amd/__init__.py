"""MI355X (gfx950) projection-GEMM path for sys1's model projections.

The compute is libsys1hip.so (hand-written HIP/MFMA kernels behind the C ABI
in include/sys1hip.h).  Importing this package does not touch the GPU; the
library loads on first use and raises if it has not been built.
"""
from ._lib import (EPI_BIAS, EPI_GEGLU, EPI_GELU, EPI_GELU_TANH, EPI_NONE, EPI_RESIDUAL, EPI_SWIGLU,
                   Sys1HipError, kernel_names)
from .batching import cu_seqlens, draw_lengths, pack_rows, unpack_rows

__all__ = ["EPI_BIAS", "EPI_GEGLU", "EPI_GELU", "EPI_GELU_TANH", "EPI_NONE", "EPI_RESIDUAL", "EPI_SWIGLU",
           "Sys1HipError", "kernel_names", "cu_seqlens", "draw_lengths", "pack_rows",
           "unpack_rows", "HipDevice", "Linear", "GatedLinear", "pack_gated_weight"]


def __getattr__(name):
    # torch-dependent modules load lazily so the package imports without torch.
    if name == "HipDevice":
        from .device import HipDevice
        return HipDevice
    if name in ("Linear", "GatedLinear", "pack_gated_weight", "linear_no_bias_dtype"):
        from . import linear
        return getattr(linear, name)
    raise AttributeError(name)
