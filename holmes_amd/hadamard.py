"""Hadamard right-rotations of weight matrices (QuaRot-style).

The reference converts checkpoints by right-multiplying projection weights with a normalised
Hadamard matrix: ``matmul_had_u`` (tools/convert/hadamard/numpy.py:77-91) rotates the last axis by
H_n / sqrt(n), with H_n the Sylvester matrix for n a power of two and H_K (x) H_{n/K} for
n = K 2^k -- for Llama-3-8B's down_proj input, n = 14336 = 28 x 512 (numpy.py:22-52, fuse.py:40-52).
Its 28 x 28 block is a vendored table (numpy.py:5-18); here it is built by Paley's second
construction over GF(13) (13 = 1 mod 4, order 2(13 + 1) = 28).  Any Hadamard matrix of order 28
gives an orthogonal rotation of the same kind; a checkpoint converted with the reference's table
must be rotated with that table, which these functions do not claim to reproduce.

The last axis, index a * (n/K) + b, is split into the K block's index a and the power-of-two
index b, itself split into Sylvester factors of at most 128; each factor is one dense product.
"""

from __future__ import annotations

import functools

import numpy as np


def _is_pow2(n: int) -> bool:
    return n > 0 and not n & (n - 1)


@functools.lru_cache(maxsize=None)
def paley2_hadamard(q: int) -> np.ndarray:
    """Hadamard matrix of order 2(q + 1) for a prime q = 1 mod 4 (Paley construction II).

    The Jacobsthal matrix Q[i, j] = chi(j - i) (chi the quadratic character mod q) bordered by
    ones gives a symmetric conference matrix C of order q + 1 (C C^T = q I, zero diagonal); then
    H = C (x) [[1, 1], [1, -1]] + I (x) [[1, -1], [-1, -1]].
    """

    if q < 5 or q % 4 != 1 or any(q % d == 0 for d in range(2, int(q**0.5) + 1)):
        raise ValueError("Paley construction II needs a prime q = 1 mod 4")
    squares = {(i * i) % q for i in range(1, q)}
    chi = np.array([0] + [1 if d in squares else -1 for d in range(1, q)], dtype=np.int64)
    idx = np.arange(q)
    conf = np.zeros((q + 1, q + 1), dtype=np.int64)
    conf[0, 1:] = 1
    conf[1:, 0] = 1
    conf[1:, 1:] = chi[(idx[None, :] - idx[:, None]) % q]
    h = np.kron(conf, np.array([[1, 1], [1, -1]])) + np.kron(np.eye(q + 1, dtype=np.int64),
                                                             np.array([[1, -1], [-1, -1]]))
    return h


def hadamard_block(n: int) -> tuple[np.ndarray | None, int]:
    """(H_K, K) with n = K 2^k: K = 1 (no block) for a power of two, K = 28 when n / 28 is one."""

    if _is_pow2(n):
        return None, 1
    if n % 28 == 0 and _is_pow2(n // 28):
        return paley2_hadamard(13), 28
    raise ValueError(f"Hadamard size must be 2^k or 28 * 2^k, got {n}")


def _sylvester(m: int) -> np.ndarray:
    h = np.ones((1, 1))
    while h.shape[0] < m:
        h = np.block([[h, h], [h, -h]])
    return h


def _factors(n: int) -> list[np.ndarray]:
    """H_n as a Kronecker product of small dense factors, outermost first: the K block (if any)
    and Sylvester factors of at most 128 (H_{2^(a+b)} = H_{2^a} (x) H_{2^b})."""

    block, k = hadamard_block(n)
    out = [block.astype(np.float64)] if block is not None else []
    e = (n // k).bit_length() - 1
    parts = max(1, -(-e // 7))
    for i in range(parts):
        out.append(_sylvester(1 << (e // parts + (1 if i < e % parts else 0))))
    return out


def hadamard_right(w: np.ndarray, signs: np.ndarray | None = None) -> np.ndarray:
    """W (diag(signs)) (H_K (x) H_{n/K}) / sqrt(n) over the last axis, in float64.

    The last axis is split into the Kronecker factors' indices and each factor is applied to its
    own axis as one dense product (a GEMM each, instead of log n strided passes)."""

    n = w.shape[-1]
    factors = _factors(n)
    x = np.array(w, dtype=np.float64)
    if signs is not None:
        x *= signs
    post = n
    for f in factors:
        s = f.shape[0]
        post //= s
        if post == 1:
            x = x.reshape(-1, s) @ f.T
        else:
            x = np.matmul(f, x.reshape(-1, s, post))
    return x.reshape(w.shape) / np.sqrt(n)


def randomized_hadamard_right(w: np.ndarray, seed: int) -> np.ndarray:
    """hadamard_right with a seeded +-1 sign vector in front (the randomized rotation)."""

    n = w.shape[-1]
    hadamard_block(n)
    signs = np.random.default_rng(seed).choice(np.array([-1.0, 1.0]), size=n)
    return hadamard_right(w, signs)


def rotate_mlp_weights(gate: np.ndarray, up: np.ndarray, down: np.ndarray, seed: int):
    """Gate / up ([I, D]) right-rotated on their D-wide input axis by a seeded randomized Hadamard
    (the residual-stream rotation), down ([D, I]) on its I-wide input axis by H_I / sqrt(I) --
    the reference's fused online down_proj Hadamard (fuse.py:40-52), H_28 (x) H_512 at I = 14336."""

    return (randomized_hadamard_right(gate, seed), randomized_hadamard_right(up, seed),
            hadamard_right(down))


__all__ = ["hadamard_block", "hadamard_right", "paley2_hadamard", "randomized_hadamard_right",
           "rotate_mlp_weights"]
