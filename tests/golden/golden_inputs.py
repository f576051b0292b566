"""Seeded inputs of the committed golden vectors (numpy only, no product code).

Both the generator (make_golden.py, which runs the CPU oracle) and the tests that check the
oracle and the GPU path against the committed files build their inputs here, so a vector is
identified by (parameter set, seed) alone."""

from __future__ import annotations

import hashlib

import numpy as np

# parameter sets: (log_n, prime bits, num_q, num_p, alpha)
SMALL = dict(log_n=8, bits=50, L=4, K=2, alpha=2)
PROD = dict(log_n=16, bits=50, L=24, K=8, alpha=8)
SEED = 20261201


def rng(seed: int, tag: str) -> np.random.Generator:
    h = hashlib.blake2b(f"{seed}/{tag}".encode(), digest_size=8).digest()
    return np.random.default_rng(int.from_bytes(h, "little"))


def uniform(r: np.random.Generator, primes, prefix, n: int) -> np.ndarray:
    out = np.empty(tuple(prefix) + (len(primes), n), dtype=np.uint64)
    for i, q in enumerate(primes):
        out[..., i, :] = r.integers(0, int(q), size=tuple(prefix) + (n,), dtype=np.uint64)
    return out


def ternary(r: np.random.Generator, n: int) -> np.ndarray:
    return r.integers(-1, 2, size=n, dtype=np.int64)


def gaussian(r: np.random.Generator, shape, sigma: float = 3.2) -> np.ndarray:
    e = np.rint(r.normal(0.0, sigma, size=shape))
    b = np.ceil(6.0 * sigma)
    return np.clip(e, -b, b).astype(np.int64)


def automorph_signed(s: np.ndarray, g: int) -> np.ndarray:
    """X^i -> X^(i g) mod (X^N + 1) on a signed coefficient vector."""

    n = s.size
    idx = (np.arange(n, dtype=np.int64) * int(g)) % (2 * n)
    out = np.zeros(n, dtype=np.int64)
    wrap = idx >= n
    out[idx[~wrap]] = s[~wrap]
    out[idx[wrap] - n] = -s[wrap]
    return out


def galois(rotation: int, log_n: int) -> int:
    return pow(5, int(rotation) % (1 << (log_n - 1)), 2 << log_n)


def key_inputs(params: dict, primes, rotation: int, seed: int = SEED):
    """(s_from, s_to, a, e, g) of the rotation key used by the golden key switch / rotation."""

    n = 1 << params["log_n"]
    beta = -(-params["L"] // params["alpha"])
    r = rng(seed, f"key/{rotation}")
    s = ternary(r, n)
    a = uniform(r, primes, (beta,), n)
    e = gaussian(r, (beta, n))
    g = galois(rotation, params["log_n"])
    return automorph_signed(s, g), s, a, e, g


def limb_hashes(x: np.ndarray) -> list[str]:
    """sha256 (hex, first 16 chars) of each limb's little-endian uint64 bytes; x is [..., limbs, N]."""

    x = np.ascontiguousarray(x, dtype="<u8")
    flat = x.reshape(-1, x.shape[-1])
    return [hashlib.sha256(row.tobytes()).hexdigest()[:16] for row in flat]
