"""Writes tests/golden/projection_golden.json.

The expected outputs come from numpy float64 / scipy / torch, not from the
oracle, so the fixture pins the oracle and the GPU path independently:
  - linear: y = x.W^T (+ b), candle_nn::Linear's contract (weight [out,in]),
    in float64 over float32 inputs, for small ragged shapes;
  - geglu: the reference's 16-value vector (src/archs/modernbert.rs:746-757),
    gelu_erf(first half) * second half with scipy's normal CDF;
  - swiglu: first 64 values of the reference generator
    (src/archs/qwen35_text.rs:1097-1104) with scipy's logistic;
  - bf16: round-to-nearest-even bit patterns from torch's bf16 cast.
Run: python tests/golden/make_golden.py
"""
import json
import os

import numpy as np
import scipy.special
import scipy.stats
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "projection_golden.json")


def main():
    rng = np.random.default_rng(20261201)
    cases = []
    for (M, N, K, bias) in [(1, 8, 8, False), (3, 5, 16, True), (7, 12, 24, False),
                            (16, 33, 40, True), (5, 64, 72, False)]:
        x = rng.standard_normal((M, K)).astype(np.float32)
        w = (0.02 * rng.standard_normal((N, K))).astype(np.float32)
        b = rng.standard_normal(N).astype(np.float32) if bias else None
        y = x.astype(np.float64) @ w.astype(np.float64).T
        if b is not None:
            y = y + b.astype(np.float64)
        cases.append({"x": x.tolist(), "w": w.tolist(), "bias": None if b is None else b.tolist(),
                      "y": y.tolist()})
    vals = np.array([-4.0, -1.5, -0.25, 0.0, 0.5, 1.25, 3.0, 5.0, 2.0, -0.75, 0.125, -3.5, 1.0,
                     0.5, -2.0, 4.5]).reshape(2, 8)
    a, u = vals[:, :4], vals[:, 4:]
    geglu = a * scipy.stats.norm.cdf(a) * u
    i = np.arange(64)
    g = (((i * 97) % 1601).astype(np.float32) - 800.0) / 73.0
    up = (-0.5 * g + 0.25).astype(np.float32)
    g64 = g.astype(np.float64)
    swi = g64 * scipy.special.expit(g64) * up.astype(np.float64)
    r = (1000 * rng.standard_normal(256)).astype(np.float32)
    r[:4] = [1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 0.0]
    bits = torch.from_numpy(r).to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)
    gold = {"linear": cases,
            "geglu": {"input": vals.tolist(), "output": geglu.tolist()},
            "swiglu": {"gate": g.tolist(), "up": up.tolist(), "output": swi.tolist()},
            "bf16": {"input": r.tolist(), "bits": bits.tolist()}}
    with open(OUT, "w") as f:
        json.dump(gold, f)
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
