"""The context-free, allocation-free entry point (sys1hip_linear_bf16_noalloc)
through the C ABI: its output equals sys1hip_linear_bf16's on the same
inputs (same kernel plan, so bit for bit), on two calls in a row, the second
with a smaller input -- the static workspace keeps the first call's
contents, and its arrival counters must come back re-armed."""
import ctypes

import numpy as np
import pytest

from gpu_helpers import assert_parity, to_gpu_bf16, to_np

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _call(L, fn, first, x, w, y, bias=None, res=None, epi=0):
    M, K = x.shape
    N = w.shape[0]
    rc = fn(first, _ptr(x), x.stride(0), _ptr(w), w.stride(0), _ptr(bias), _ptr(res),
            res.stride(0) if res is not None else 0, _ptr(y), y.stride(0), M, N, K, epi)
    return rc


def test_noalloc_matches_the_context_entry_point(orc):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from sys1_amd import _lib
    from sys1_amd.device import HipDevice
    L = _lib.load()
    dev = HipDevice(0)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    dev.follow_torch_stream()
    # Two calls in a row, the second smaller: stream-K plans (weights above
    # the skinny kernels' 32 MB, so the static workspace and its counters
    # are used), then tile and skinny plans, with and without epilogues.
    cases = [(96, 8192, 4096, 0), (48, 4096, 5120, 0), (40, 6144, 4096, _lib.EPI_RESIDUAL),
             (600, 768, 768, _lib.EPI_RESIDUAL), (33, 3072, 1024, 0), (64, 4096, 2048, _lib.EPI_GEGLU)]
    for (M, N, K, epi) in cases:
        print(f"[gpu] noalloc M={M} N={N} K={K} epi={epi} plan={dev.query_kernel(M, N, K, epi)[1]}", flush=True)
        x = to_gpu_bf16(orc.fill_normal((M, K), 3 + M), torch)
        w = to_gpu_bf16(orc.fill_normal((N, K), 4 + N, 0.02), torch)
        nout = N // 2 if epi == _lib.EPI_GEGLU else N
        if epi == _lib.EPI_GEGLU:
            wp = torch.empty_like(w)
            _lib.check(L.sys1hip_pack_gated_weight(dev.ctx, _ptr(w), _ptr(wp), N, K), dev.ctx)
            w = wp
        res = to_gpu_bf16(orc.fill_normal((M, nout), 5), torch) if epi == _lib.EPI_RESIDUAL else None
        y_ctx = torch.empty(M, nout, dtype=torch.bfloat16, device="cuda:0")
        y_static = torch.full((M, nout), float("nan"), dtype=torch.bfloat16, device="cuda:0")
        _lib.check(_call(L, L.sys1hip_linear_bf16, dev.ctx, x, w, y_ctx, res=res, epi=epi), dev.ctx)
        _lib.check(_call(L, L.sys1hip_linear_bf16_noalloc, stream, x, w, y_static, res=res, epi=epi))
        torch.cuda.synchronize()
        assert torch.equal(y_ctx, y_static), f"M={M} N={N} K={K} epi={epi}"
        if epi == 0:
            assert_parity(to_np(y_static), orc.linear_f32(to_np(x), to_np(w)), f"noalloc M={M} N={N} K={K}")
    # the refused call: a bad shape reports an error, not a launch
    x = to_gpu_bf16(orc.fill_normal((8, 64), 1), torch)
    w = to_gpu_bf16(orc.fill_normal((64, 64), 2), torch)
    y = torch.empty(8, 64, dtype=torch.bfloat16, device="cuda:0")
    rc = L.sys1hip_linear_bf16_noalloc(stream, _ptr(x), 64, _ptr(w), 64, None, None, 0, _ptr(y), 64,
                                       8, 64, 60, 0)
    assert rc == _lib.EALIGN


def test_noalloc_under_graph_capture(orc):
    """The entry point inside a captured HIP graph: each replay, with eager
    calls of the same entry point (which overwrite the static workspace) and
    synchronisations between replays, equals the eager result bit for bit.
    Covers a stream-K plan (workspace and counters) and a skinny plan."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from sys1_amd import _lib
    L = _lib.load()
    for (M, N, K, epi) in [(64, 8192, 4096, _lib.EPI_RESIDUAL), (48, 3072, 1024, 0)]:
        print(f"[gpu] noalloc graph M={M} N={N} K={K} epi={epi}", flush=True)
        x = to_gpu_bf16(orc.fill_normal((M, K), 7 + M), torch)
        w = to_gpu_bf16(orc.fill_normal((N, K), 8 + N, 0.02), torch)
        res = to_gpu_bf16(orc.fill_normal((M, N), 9), torch) if epi == _lib.EPI_RESIDUAL else None
        x2 = to_gpu_bf16(orc.fill_normal((M, K), 11), torch)
        y_eager = torch.empty(M, N, dtype=torch.bfloat16, device="cuda:0")
        y_graph = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda:0")
        y_other = torch.empty(M, N, dtype=torch.bfloat16, device="cuda:0")
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(_call(L, L.sys1hip_linear_bf16_noalloc, s, x, w, y_eager, res=res, epi=epi))
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            cs = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            _lib.check(_call(L, L.sys1hip_linear_bf16_noalloc, cs, x, w, y_graph, res=res, epi=epi))
        torch.cuda.synchronize()
        for r in range(4):
            y_graph.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y_graph, y_eager), f"replay {r}: M={M} N={N} K={K} epi={epi}"
            # eager work between replays, on the same static workspace
            _lib.check(_call(L, L.sys1hip_linear_bf16_noalloc, s, x2, w, y_other, res=res, epi=epi))
            torch.cuda.synchronize()
        del g


_FIRST_CALL_UNDER_CAPTURE = r"""
import ctypes, sys
import torch
sys.path.insert(0, sys.argv[1])
from sys1_amd import _lib
L = _lib.load()
torch.manual_seed(0)
M, N, K = 64, 8192, 4096  # a stream-K plan: the static workspace and its counters
x = torch.randn(M, K).to(torch.bfloat16).cuda()
w = (torch.randn(N, K) * 0.02).to(torch.bfloat16).cuda()
r = torch.randn(M, N).to(torch.bfloat16).cuda()
y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
p = lambda t: ctypes.c_void_p(t.data_ptr())
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.sys1hip_linear_bf16_noalloc(s, p(x), K, p(w), K, None, p(r), N, p(y), N, M, N, K, _lib.EPI_RESIDUAL)
print("first call under capture: rc", rc, flush=True)
assert rc == 0, L.sys1hip_last_error(None)
from sys1_amd.device import HipDevice
dev = HipDevice(0)
ref = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
dev.follow_torch_stream()
_lib.check(L.sys1hip_linear_bf16(dev.ctx, p(x), K, p(w), K, None, p(r), N, p(ref), N, M, N, K,
                                 _lib.EPI_RESIDUAL), dev.ctx)
torch.cuda.synchronize()
for i in range(3):
    y.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, ref), f"replay {i}"
print("replays equal sys1hip_linear_bf16", flush=True)
"""


def test_noalloc_first_call_under_capture_in_a_fresh_process():
    """A process whose very first call of the entry point is inside a graph
    capture (set-up then runs under capture: symbol address and occupancy
    queries, no counter-clearing kernel, counters zero from the module
    load).  Run in a child process so that no earlier call did the set-up;
    its replays must equal sys1hip_linear_bf16."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("[gpu] noalloc first call under capture (child process)", flush=True)
    out = subprocess.run([sys.executable, "-c", _FIRST_CALL_UNDER_CAPTURE, root], capture_output=True,
                         text=True, timeout=100)
    print(out.stdout[-2000:], out.stderr[-2000:], flush=True)
    assert out.returncode == 0
    assert "replays equal" in out.stdout
