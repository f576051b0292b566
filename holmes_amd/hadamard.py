"""Randomized Hadamard right-rotation of a weight matrix (QuaRot-style).

The reference converts checkpoints by right-multiplying each projection weight with a seeded
randomized Hadamard matrix (tools/convert/hadamard/numpy.py:54-91); the C3 configuration quotes its
q_proj on such a weight.  Here W' = W (diag(s) H / sqrt(n)) with s a seeded +-1 vector and H the
Sylvester Hadamard matrix, computed by an in-place fast Walsh-Hadamard transform over the last axis
(n log n additions instead of a dense product).
"""

from __future__ import annotations

import numpy as np


def randomized_hadamard_right(w: np.ndarray, seed: int) -> np.ndarray:
    n = w.shape[-1]
    if n <= 0 or n & (n - 1):
        raise ValueError("Hadamard size must be a power of two")
    signs = np.random.default_rng(seed).choice(np.array([-1.0, 1.0]), size=n)
    x = np.asarray(w, dtype=np.float64) * signs
    h = 1
    while h < n:
        x = x.reshape(*x.shape[:-1], n // (2 * h), 2, h)
        a, b = x[..., 0, :].copy(), x[..., 1, :].copy()
        x[..., 0, :], x[..., 1, :] = a + b, a - b
        x = x.reshape(*x.shape[:-3], n)
        h *= 2
    return x / np.sqrt(n)


__all__ = ["randomized_hadamard_right"]
