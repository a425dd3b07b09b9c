"""Packed ragged token batches: the M the projections see.

The reference pads Laya's sequences to a rectangle [batch, max_len]
(src/models/laya.rs:396-431), so M includes pad rows.  A projection is
row-independent, so packing the real tokens back to back (cu_seqlens
bookkeeping, as the varlen attention path at src/archs/modernbert.rs:430-477
already uses) gives the same outputs for the real rows with no pad work.

Lengths for the synthetic benchmark batches are drawn from the SplitMix64
stream (Steele, Lea & Flood 2014) so that the host, the tests and the CPU
checker produce the same batches for a seed.
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, index: np.ndarray) -> np.ndarray:
    """Element `index` of the SplitMix64 stream started at `seed`."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + (index.astype(np.uint64) + np.uint64(1)) * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def draw_lengths(seed: int, lo: int, hi: int, budget: int, exact: bool = False) -> np.ndarray:
    """Lengths ~ U[lo, hi] drawn until the next would exceed `budget` tokens;
    with `exact`, the last sequence is truncated to fill the budget exactly."""
    if lo < 1 or hi < lo or budget < 0:
        raise ValueError(f"bad length range [{lo}, {hi}] or budget {budget}")
    n = budget // lo + 2
    draws = lo + (splitmix64(seed, np.arange(n)) % np.uint64(hi - lo + 1)).astype(np.int64)
    total = np.cumsum(draws)
    count = int(np.searchsorted(total, budget, side="right"))
    lengths = draws[:count].copy()
    used = int(lengths.sum())
    if exact and used < budget:
        lengths = np.append(lengths, budget - used)
    return lengths


def cu_seqlens(lengths) -> np.ndarray:
    """Prefix offsets [0, l0, l0+l1, ...] of the packed sequences."""
    lengths = np.asarray(lengths, dtype=np.int64)
    if (lengths < 0).any():
        raise ValueError("negative sequence length")
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)


def positions(lengths) -> np.ndarray:
    """Per packed token, its position within its sequence (int32): the
    rotary position the reference reads as token % length on its padded
    rectangle (src/kernels/modernbert.cu:31-74)."""
    lengths = np.asarray(lengths, dtype=np.int64)
    if (lengths < 0).any():
        raise ValueError("negative sequence length")
    starts = np.repeat(cu_seqlens(lengths)[:-1], lengths)
    return (np.arange(int(lengths.sum()), dtype=np.int64) - starts).astype(np.int32)


def pack_rows(padded: np.ndarray, lengths) -> np.ndarray:
    """[batch, max_len, H] padded rectangle -> [sum(lengths), H] packed rows."""
    return np.concatenate([padded[b, :l] for b, l in enumerate(lengths)], 0)


def unpack_rows(packed: np.ndarray, lengths, max_len: int, fill=0.0) -> np.ndarray:
    """Inverse of pack_rows; pad rows take `fill`."""
    lengths = list(lengths)
    out = np.full((len(lengths), max_len, packed.shape[-1]), fill, dtype=packed.dtype)
    off = cu_seqlens(lengths)
    for b, l in enumerate(lengths):
        out[b, :l] = packed[off[b]:off[b + 1]]
    return out
