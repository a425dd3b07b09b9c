"""Build libsys1hip.so (the gfx950 projection kernels + C ABI) in-tree.

Run as ``python -m sys1_amd.build``.  hipcc cross-compiles for gfx950 without
a GPU, so this works on the build host; the .so then travels with the tree.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libsys1hip.so")
SOURCES = [os.path.join(CSRC, "sys1hip.hip")]
HEADERS = [os.path.join(CSRC, f) for f in ("common.hpp", "gemm_tile.hpp", "norm.hpp", "conv.hpp")] + [
    os.path.join(ROOT, "include", "sys1hip.h")]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    # Packed-FP32 VALU ops are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def build(verbose: bool = False) -> str:
    cmd = [HIPCC, *FLAGS, *SOURCES, "-o", LIB + ".tmp"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building libsys1hip.so")
    if verbose:
        noise = "is not a recognized feature for this target"
        msgs = [l for l in (res.stdout + res.stderr).splitlines() if noise not in l]
        if msgs:
            print("\n".join(msgs))
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
