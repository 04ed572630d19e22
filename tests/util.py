"""Shared helpers for the parity tests: the reference's error measures and
deterministic input formulas (moebius-cpu tests/kernels.rs), and fixture
access."""
from __future__ import annotations

import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fixtures():
    """tests/fixtures/kernels.safetensors of the reference (format tag
    `moebius-cpu-fixture/1`), copied to tests/golden/ as data."""
    from safetensors.numpy import load_file

    return load_file(os.path.join(GOLDEN, "kernels.safetensors"))


def max_scaled_err(got, want) -> float:
    """tests/kernels.rs:28-38: max |g - w| / (1 + |w|)."""
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, f"shape {got.shape} vs {want.shape}"
    return float(np.max(np.abs(got - want) / (1.0 + np.abs(want)))) if got.size else 0.0


def assert_close(got, want, tol):
    err = max_scaled_err(got, want)
    assert err <= tol, f"max scaled error {err:e} > {tol:e}"


def rel_l2(got, want) -> float:
    """tests/kernels.rs:223-231"""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    assert g.shape == w.shape
    return float(np.sqrt(np.sum((g - w) ** 2) / np.sum(w ** 2)))


def max_abs_rel(got, want) -> float:
    """max |g - w| / max |w|: the f32 parity measure (tolerance 1e-4)."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    assert g.shape == w.shape, f"shape {g.shape} vs {w.shape}"
    if g.size == 0:
        return 0.0
    return float(np.max(np.abs(g - w)) / max(np.max(np.abs(w)), 1e-30))


def hashed(n, mul, mod, div, off):
    """((i * mul) % mod) / div - off for i in 0..n (tests/kernels.rs input formulas)."""
    i = np.arange(n, dtype=np.int64)
    return (((i * mul) % mod).astype(np.float32) / np.float32(div) - np.float32(off)).astype(np.float32)


_LCG_A = np.uint64(6364136223846793005)
_LCG_C = np.uint64(1442695040888963407)


class Lcg:
    """tests/kernels.rs:215-221: s = s*a + c (mod 2^64); ((s >> 40) / 2^24) * 2 - 1."""

    def __init__(self, seed: int):
        self.s = np.uint64(seed)

    def take(self, n: int) -> np.ndarray:
        with np.errstate(over="ignore"):
            block = 1024
            first = np.empty(min(n, block), np.uint64)
            s = self.s
            for i in range(first.size):
                s = s * _LCG_A + _LCG_C
                first[i] = s
            if n <= block:
                states = first
            else:
                # Jump `block` steps at once: s' = A s + C with A = a^block, C = c (a^(block-1) + ... + 1).
                A, C = np.uint64(1), np.uint64(0)
                for _ in range(block):
                    A, C = A * _LCG_A, C * _LCG_A + _LCG_C
                rows = (n + block - 1) // block
                states = np.empty((rows, block), np.uint64)
                states[0] = first
                for r in range(1, rows):
                    states[r] = states[r - 1] * A + C
                states = states.reshape(-1)[:n]
            self.s = states[-1]
        return ((states >> np.uint64(40)).astype(np.float32) / np.float32(1 << 24) * np.float32(2.0)
                - np.float32(1.0)).astype(np.float32)
