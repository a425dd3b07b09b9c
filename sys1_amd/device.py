"""HIP device context: the counterpart of sys1's `device::load()`
(src/device.rs:43-65), which returns the one candle Device the process uses
(`Device::new_cuda(0)` at :49-51).  Here the device is a sys1hip context on
one GPU; its kernels run on the torch stream that is current when a
projection is called, so they order naturally with the torch ops that own
the buffers.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


class HipDevice:
    def __init__(self, index: int = 0):
        L = _lib.load()
        ctx = ctypes.c_void_p()
        _lib.check(L.sys1hip_init(int(index), ctypes.byref(ctx)))
        self._L = L
        self.ctx = ctx
        self.index = int(index)
        self.torch_device = torch.device("cuda", self.index)
        self._stream = None
        self.follow_torch_stream()

    def follow_torch_stream(self) -> int:
        """Point the context at torch's current stream on this device."""
        s = torch.cuda.current_stream(self.torch_device).cuda_stream
        if s != self._stream:
            _lib.check(self._L.sys1hip_set_stream(self.ctx, ctypes.c_void_p(s)), self.ctx)
            self._stream = s
        return s

    def synchronize(self) -> None:
        _lib.check(self._L.sys1hip_sync(self.ctx), self.ctx)

    def set_kernel(self, kernel_id: int) -> None:
        """Force one kernel id (-1: automatic choice)."""
        _lib.check(self._L.sys1hip_set_kernel(self.ctx, int(kernel_id)), self.ctx)

    def set_grid(self, workgroups: int) -> None:
        """Force the persistent grid size (0: automatic)."""
        _lib.check(self._L.sys1hip_set_grid(self.ctx, int(workgroups)), self.ctx)

    def set_dp_tiles(self, tiles: int) -> None:
        """Force the tiles a stream-K kernel runs whole before its stream
        phase (-1 = automatic)."""
        _lib.check(self._L.sys1hip_set_dp_tiles(self.ctx, int(tiles)), self.ctx)

    def chain_status(self) -> int:
        """Synchronise and return (then clear) the error bits of the chain
        launches since the last call (sys1hip_chain_status); 0 = all fine."""
        v = ctypes.c_int32()
        _lib.check(self._L.sys1hip_chain_status(self.ctx, ctypes.byref(v)), self.ctx)
        return v.value

    def set_chain_wait(self, wait_us: int = 20000, extra: int = 0) -> None:
        """Real time a chain dependency wait may take before it gives up, and
        an amount added to every dependency target (a test knob: > 0 makes
        every wait expire)."""
        _lib.check(self._L.sys1hip_set_chain_wait(self.ctx, int(wait_us), int(extra)), self.ctx)

    def query_kernel(self, M: int, N: int, K: int, epilogue: int = 0) -> tuple[int, str]:
        buf = ctypes.create_string_buffer(96)
        kid = _lib.check(self._L.sys1hip_query_kernel(self.ctx, M, N, K, epilogue, buf, 96), self.ctx)
        return kid, buf.value.decode()

    def close(self) -> None:
        if self.ctx:
            _lib.check(self._L.sys1hip_destroy(self.ctx))
            self.ctx = ctypes.c_void_p()

    def __del__(self):
        try:
            if self.ctx:
                self._L.sys1hip_destroy(self.ctx)
        except Exception:
            pass


_default: HipDevice | None = None


def load(index: int = 0) -> HipDevice:
    """The process-wide device (mirrors `device::load()`): created on first use."""
    global _default
    if _default is None or _default.index != index:
        _default = HipDevice(index)
    return _default
