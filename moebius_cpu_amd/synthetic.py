"""Seeded synthetic inputs for the benchmark workloads and parity tests.

One documented generator: splitmix64 -> 53-bit uniforms -> Box-Muller in f64
-> f32. Every tensor is generated once on the host; the identical bytes go to
the CPU oracle and to HBM.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs start..start+n-1 of splitmix64 seeded with `seed` (state += golden; mix)."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + _GOLDEN * np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, start: int = 0) -> np.ndarray:
    """n f64 uniforms in [0, 1) from the top 53 bits (outputs start..start+n-1)."""
    return (splitmix64(seed, n, start) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


_BLOCK = 1 << 22  # pairs generated per pass (bounds the f64 temporaries)


def normal(seed: int, shape, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    """Box-Muller normals (f64) -> f32, `mean + std * z`: pair i uses uniforms
    2i (radius) and 2i+1 (angle) and yields (r cos t, r sin t)."""
    n = int(np.prod(shape, dtype=np.int64))
    m = (n + 1) // 2
    out = np.empty(2 * m, np.float32)
    for p0 in range(0, m, _BLOCK):
        pm = min(_BLOCK, m - p0)
        u = uniform(seed, 2 * pm, 2 * p0).reshape(pm, 2)
        r = np.sqrt(-2.0 * np.log1p(-u[:, 0]))
        t = 2.0 * np.pi * u[:, 1]
        out[2 * p0:2 * (p0 + pm):2] = (mean + std * (r * np.cos(t))).astype(np.float32)
        out[2 * p0 + 1:2 * (p0 + pm):2] = (mean + std * (r * np.sin(t))).astype(np.float32)
    return out[:n].reshape(shape)


def kaiming(seed: int, shape, fan_in: int) -> np.ndarray:
    """Kaiming-normal weights: std = sqrt(2 / fan_in) (torch kaiming_normal_ default)."""
    return normal(seed, shape, std=float(np.sqrt(2.0 / fan_in)))


def uniform_range(seed: int, shape, lo: float, hi: float) -> np.ndarray:
    n = int(np.prod(shape, dtype=np.int64))
    return (lo + (hi - lo) * uniform(seed, n)).astype(np.float32).reshape(shape)
