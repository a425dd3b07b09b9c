"""Shared helpers of the GPU parity tests: seeded inputs from the oracle's
generator, bf16 transfer, and the parity metrics of the projection path
(relative Frobenius error <= 1e-2 and max-abs error <= 2e-2 * max|ref| per
projection output)."""
import numpy as np

REL_FRO_TOL = 1e-2
MAX_ABS_TOL = 2e-2


def to_gpu_bf16(a, torch):
    """f32 numpy -> bf16 tensor on cuda:0 (RNE, torch's cast)."""
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).to("cuda:0")


def to_np(t):
    return t.float().cpu().numpy()


def parity(out, ref):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    rel = np.linalg.norm(out - ref) / max(np.linalg.norm(ref), 1e-30)
    mx = np.abs(out - ref).max() / max(np.abs(ref).max(), 1e-30) if ref.size else 0.0
    return float(rel), float(mx)


def assert_parity(out, ref, what=""):
    rel, mx = parity(out, ref)
    assert rel <= REL_FRO_TOL and mx <= MAX_ABS_TOL, f"{what}: rel_fro={rel:.3e} max_abs/max={mx:.3e}"
    return rel, mx


def bf16_ulp(v):
    """Spacing of bf16 numbers at |v| (8 significant bits)."""
    v = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(v, 2.0 ** -126)))
    return 2.0 ** (e - 7)
