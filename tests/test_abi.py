"""Host-side checks of the C ABI: the library loads, exports every symbol
include/sys1hip.h declares, and rejects bad arguments with the documented
codes before touching a device (so these run without a GPU)."""
import ctypes
import os
import re

import pytest

from sys1_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sys1hip.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"SYS1HIP_API\s+[\w\s\*]+?\b(sys1hip_\w+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    assert _declared() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    for name in _declared():
        assert hasattr(L, name), name
    nm = os.popen(f"nm -D --defined-only {_lib.LIB_PATH}").read()
    exported = set(re.findall(r"\bT (sys1hip_\w+)", nm))
    assert exported == set(_declared())


def test_version_and_kernel_table():
    L = _lib.load()
    assert L.sys1hip_version() == 100
    names = _lib.kernel_names()
    assert len(names) == L.sys1hip_kernel_count() >= 6
    assert any(n.startswith("tile_") for n in names) and any(n.startswith("stream_") for n in names)
    assert L.sys1hip_kernel_name(-1) is None and L.sys1hip_kernel_name(len(names)) is None


def test_flag_values_match_header():
    text = open(HEADER).read()
    for name in ("NONE", "BIAS", "GEGLU", "SWIGLU", "RESIDUAL", "GELU", "GELU_TANH", "BLOCKED_W"):
        m = re.search(rf"#define SYS1HIP_EPI_{name} (\d+)", text)
        assert int(m.group(1)) == getattr(_lib, f"EPI_{name}")
    for name in ("EINVAL", "EALIGN", "EDEVICE", "ERANGE"):
        m = re.search(rf"#define SYS1HIP_{name} \((-\d+)\)", text)
        assert int(m.group(1)) == getattr(_lib, name)
    for name in ("LAYER", "RMS"):
        m = re.search(rf"#define SYS1HIP_NORM_{name} (\d+)", text)
        assert int(m.group(1)) == getattr(_lib, f"NORM_{name}")


def _no_gpu():
    try:
        import torch
        return not torch.cuda.is_available()
    except Exception:
        return True


@pytest.mark.skipif(not _no_gpu(), reason="checks the no-device error path")
def test_init_without_device_fails_loudly():
    L = _lib.load()
    ctx = ctypes.c_void_p()
    rc = L.sys1hip_init(0, ctypes.byref(ctx))
    assert rc == _lib.EDEVICE
    assert b"no HIP device" in L.sys1hip_last_error(None)
    with pytest.raises(_lib.Sys1HipError):
        _lib.check(rc)


# Argument validation runs before the context is dereferenced, so a dummy
# non-null context is enough to force every error path from the host.
_DUMMY = ctypes.create_string_buffer(256)
_ctx = ctypes.cast(_DUMMY, ctypes.c_void_p)
_P = 1 << 20  # a 16-byte-aligned fake device address (never dereferenced)


def _call(x=_P, ldx=64, w=_P, ldw=64, bias=None, res=None, ldr=0, y=_P, ldy=64, M=4, N=64,
          K=64, epi=0, ctx=_ctx):
    L = _lib.load()
    return L.sys1hip_linear_bf16(ctx, x, ldx, w, ldw, bias, res, ldr, y, ldy, M, N, K, epi)


@pytest.mark.parametrize("kwargs,code", [
    (dict(ctx=None), _lib.EINVAL),
    (dict(epi=128), _lib.EINVAL),                     # unknown flag
    (dict(epi=_lib.EPI_GELU), _lib.EINVAL),           # gelu needs bias
    (dict(epi=_lib.EPI_GELU_TANH), _lib.EINVAL),      # so does the tanh gelu
    (dict(epi=_lib.EPI_GELU | _lib.EPI_GELU_TANH | _lib.EPI_BIAS), _lib.EINVAL),  # one gelu at most
    (dict(epi=_lib.EPI_GEGLU | _lib.EPI_SWIGLU), _lib.EINVAL),
    (dict(N=0), _lib.EINVAL),
    (dict(K=0), _lib.EINVAL),
    (dict(M=-1), _lib.EINVAL),
    (dict(x=None), _lib.EINVAL),
    (dict(y=None), _lib.EINVAL),
    (dict(epi=_lib.EPI_BIAS), _lib.EINVAL),           # bias flag, no pointer
    (dict(bias=_P), _lib.EINVAL),                     # pointer, no flag
    (dict(epi=_lib.EPI_RESIDUAL), _lib.EINVAL),       # residual flag, no pointer
    (dict(epi=_lib.EPI_GEGLU, N=80), _lib.EINVAL),    # gated needs N % 32 == 0
    (dict(ldx=32), _lib.EINVAL),                      # ldx < K
    (dict(ldy=32), _lib.EINVAL),                      # ldy < N
    (dict(K=60, ldx=64, ldw=64), _lib.EALIGN),        # K % 8
    (dict(ldx=68), _lib.EALIGN),
    (dict(x=_P + 2), _lib.EALIGN),
    (dict(w=_P + 8), _lib.EALIGN),
    (dict(M=(1 << 30) + 1), _lib.ERANGE),
])
def test_linear_rejects_bad_arguments(kwargs, code):
    rc = _call(**kwargs)
    assert rc == code, (kwargs, rc, _lib.load().sys1hip_last_error(None))
    assert _lib.load().sys1hip_last_error(None)


def test_empty_batch_is_a_noop():
    assert _call(M=0, x=None, y=None) == _lib.OK


def test_gated_output_width_drives_ldy_rule():
    # Gated: Nout = N/2 = 32, so ldy = 30 is too small.
    assert _call(M=4, N=64, ldy=30, epi=_lib.EPI_GEGLU) == _lib.EINVAL


def _rope(ctx=_ctx, x=_P, ldx=64, w=_P, ldw=64, cos=_P, sin=_P, rows=16, pos=_P, y=_P, M=4, heads=2,
          dim=64, K=64):
    L = _lib.load()
    return L.sys1hip_linear_rope_qkv_bf16(ctx, x, ldx, w, ldw, cos, sin, rows, pos, y, M, heads, dim, K)


@pytest.mark.parametrize("kwargs,code", [
    (dict(ctx=None), _lib.EINVAL),
    (dict(dim=128), _lib.EINVAL),        # head_dim 64 only
    (dict(heads=0), _lib.EINVAL),
    (dict(rows=0), _lib.EINVAL),
    (dict(M=-1), _lib.EINVAL),
    (dict(cos=None), _lib.EINVAL),
    (dict(pos=None), _lib.EINVAL),
    (dict(ldx=32), _lib.EINVAL),
    (dict(K=60, ldx=64, ldw=64), _lib.EALIGN),
    (dict(sin=_P + 4), _lib.EALIGN),
    (dict(M=(1 << 30) + 1), _lib.ERANGE),
])
def test_rope_qkv_rejects_bad_arguments(kwargs, code):
    rc = _rope(**kwargs)
    assert rc == code, (kwargs, rc, _lib.load().sys1hip_last_error(None))


def test_rope_qkv_empty_batch_is_a_noop():
    assert _rope(M=0, x=None, y=None, cos=None, sin=None, pos=None) == _lib.OK


def _norm(ctx=_ctx, x=_P, ldx=64, w=_P, ldw=64, colsum=_P, norm=1, eps=1e-5, y=_P, ldy=64, M=4, N=64,
          K=64, epi=0):
    L = _lib.load()
    return L.sys1hip_norm_linear_bf16(ctx, x, ldx, w, ldw, colsum, norm, eps, y, ldy, M, N, K, epi)


@pytest.mark.parametrize("kwargs,code", [
    (dict(ctx=None), _lib.EINVAL),
    (dict(norm=3), _lib.EINVAL),                                   # unknown norm
    (dict(norm=_lib.NORM_LAYER, epi=_lib.EPI_SWIGLU), _lib.EINVAL),  # pairs the reference has only
    (dict(norm=_lib.NORM_RMS, epi=_lib.EPI_GEGLU), _lib.EINVAL),
    (dict(epi=_lib.EPI_RESIDUAL), _lib.EINVAL),
    (dict(eps=-1.0), _lib.EINVAL),
    (dict(eps=float("nan")), _lib.EINVAL),
    (dict(M=-1), _lib.EINVAL),
    (dict(epi=_lib.EPI_GEGLU, N=80), _lib.EINVAL),
    (dict(colsum=None), _lib.EINVAL),                              # LayerNorm needs colsum
    (dict(x=None), _lib.EINVAL),
    (dict(ldy=32), _lib.EINVAL),
    (dict(K=60, ldx=64, ldw=64), _lib.EALIGN),
    (dict(colsum=_P + 4), _lib.EALIGN),
    (dict(M=(1 << 20) + 1), _lib.ERANGE),
])
def test_norm_linear_rejects_bad_arguments(kwargs, code):
    rc = _norm(**kwargs)
    assert rc == code, (kwargs, rc, _lib.load().sys1hip_last_error(None))


def test_norm_linear_rms_needs_no_colsum_and_empty_is_noop():
    assert _norm(M=0, x=None, y=None) == _lib.OK
    # RMSNorm without colsum passes validation up to the (dummy) device step,
    # so only the empty batch can be checked here without a GPU.
    assert _norm(M=0, norm=_lib.NORM_RMS, colsum=None, x=None, y=None) == _lib.OK


def test_fold_norm_rejects_bad_arguments():
    L = _lib.load()
    f = L.sys1hip_fold_norm_weight
    assert f(None, _P, _P, 1, _P, _P, 64, 64) == _lib.EINVAL
    assert f(_ctx, _P, _P, 0, _P, _P, 64, 64) == _lib.EINVAL        # unknown norm
    assert f(_ctx, _P, _P, 1, _P, None, 64, 64) == _lib.EINVAL      # LayerNorm needs colsum
    assert f(_ctx, _P, None, 2, _P, None, 64, 64) == _lib.EINVAL    # gamma
    assert f(_ctx, _P, _P, 1, _P, _P, 0, 64) == _lib.EINVAL
    assert f(_ctx, _P, _P, 1, _P, _P, 64, 12) == _lib.EALIGN
    assert f(_ctx, _P, _P + 4, 1, _P, _P, 64, 64) == _lib.EALIGN


def _conv(ctx=_ctx, x=_P, ldx=64, w=_P, ldw=64, norm=0, eps=1e-6, cw=_P, C=64, pos=_P, y=_P, ldy=128,
          M=4, N=128, K=64):
    L = _lib.load()
    return L.sys1hip_linear_conv_silu_bf16(ctx, x, ldx, w, ldw, norm, eps, cw, C, pos, y, ldy, M, N, K)


@pytest.mark.parametrize("kwargs,code", [
    (dict(ctx=None), _lib.EINVAL),
    (dict(norm=_lib.NORM_LAYER), _lib.EINVAL),     # RMSNorm only (Qwen3.5)
    (dict(C=0), _lib.EINVAL),
    (dict(C=130), _lib.EINVAL),                    # more conv channels than N
    (dict(C=60), _lib.EINVAL),                     # multiple of 8
    (dict(M=-1), _lib.EINVAL),
    (dict(pos=None), _lib.EINVAL),
    (dict(cw=None), _lib.EINVAL),
    (dict(ldy=64), _lib.EINVAL),
    (dict(K=60, ldx=64, ldw=64), _lib.EALIGN),
    (dict(cw=_P + 8), _lib.EALIGN),
    (dict(ldy=132), _lib.EALIGN),
    (dict(M=(1 << 20) + 1), _lib.ERANGE),
])
def test_conv_rejects_bad_arguments(kwargs, code):
    rc = _conv(**kwargs)
    assert rc == code, (kwargs, rc, _lib.load().sys1hip_last_error(None))


def test_conv_empty_batch_is_a_noop():
    assert _conv(M=0, x=None, y=None, pos=None, cw=None) == _lib.OK


def test_pack_rejects_bad_arguments():
    L = _lib.load()
    f = L.sys1hip_pack_gated_weight
    assert f(None, _P, _P + 4096, 64, 64) == _lib.EINVAL
    assert f(_ctx, _P, _P, 64, 64) == _lib.EINVAL          # aliasing
    assert f(_ctx, _P, _P + 4096, 80, 64) == _lib.EINVAL    # N % 32
    assert f(_ctx, _P, _P + 4096, 64, 12) == _lib.EALIGN    # K % 8
    assert f(_ctx, _P + 2, _P + 4096, 64, 64) == _lib.EALIGN


def test_query_and_set_kernel_validate():
    L = _lib.load()
    assert L.sys1hip_set_kernel(None, 0) == _lib.EINVAL
    assert L.sys1hip_set_grid(None, 0) == _lib.EINVAL
    assert L.sys1hip_set_grid(_ctx, -1) == _lib.EINVAL
    assert L.sys1hip_set_dp_tiles(None, 0) == _lib.EINVAL
    assert L.sys1hip_set_dp_tiles(_ctx, -2) == _lib.EINVAL
    assert L.sys1hip_query_kernel(None, 1, 1, 8, 0, None, 0) == _lib.EINVAL
