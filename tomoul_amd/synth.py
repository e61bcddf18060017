"""Seeded synthetic inputs: SplitMix64 -> 53-bit uniform -> Box-Muller in f64
-> f32.  Normals come in (cos, sin) pairs from two consecutive uniforms, the
first mapped to (0, 1] so the logarithm is finite.  Seeds used by the bench:
X = 1001, W = 2002 (+ layer index), bias = 3003.
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, count: int, skip: int = 0) -> np.ndarray:
    """Outputs skip + 1 .. skip + count of SplitMix64 started at `seed` (uint64)."""
    with np.errstate(over="ignore"):
        i = np.arange(skip + 1, skip + count + 1, dtype=np.uint64)
        z = np.uint64(seed) + i * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0, offset: int = 0) -> np.ndarray:
    """n float32 samples of N(mean, std^2): elements offset .. offset + n - 1
    of the stream started at `seed` (offset even: normals come in pairs), so a
    long stream can be drawn in pieces."""
    if offset % 2:
        raise ValueError("offset must be even")
    pairs = (n + 1) // 2
    r = splitmix64(seed, 2 * pairs, offset)
    u = (r >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    u1 = 1.0 - u[0::2]
    u2 = u[1::2]
    rad = np.sqrt(-2.0 * np.log(u1))
    ang = 2.0 * np.pi * u2
    z = np.empty(2 * pairs, dtype=np.float64)
    z[0::2] = rad * np.cos(ang)
    z[1::2] = rad * np.sin(ang)
    return (mean + std * z[:n]).astype(np.float32)


def normal_matrix(seed: int, rows: int, cols: int, std: float = 1.0) -> np.ndarray:
    return normal(seed, rows * cols, 0.0, std).reshape(rows, cols)
