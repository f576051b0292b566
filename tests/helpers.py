"""Independent Python big-integer math used to pin the oracle (no shared code with it)."""

from __future__ import annotations

import numpy as np


def bitrev(x: int, bits: int) -> int:
    return int(format(x, f"0{bits}b")[::-1], 2) if bits else 0


def small_primes(log_n: int, bits: int, count: int, skip=()) -> list[int]:
    """Primes = 1 mod 2N below 2^bits by trial with Python's pow-based Fermat + MR bases."""

    step = 2 << log_n
    out = []
    c = (1 << bits) + 1 - step
    skip = set(skip)
    while len(out) < count:
        if c not in skip and is_prime_py(c):
            out.append(c)
        c -= step
    return out


def is_prime_py(n: int) -> bool:
    if n < 2:
        return False
    for p in (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37, 41, 43, 47):
        if n % p == 0:
            return n == p
    d, s = n - 1, 0
    while d % 2 == 0:
        d //= 2
        s += 1
    # a different base set from the oracle's, so a shared mistake would have to be coincidental
    for a in (41, 43, 47, 53, 59, 61, 67, 71, 73, 79, 83, 89):
        x = pow(a, d, n)
        if x in (1, n - 1):
            continue
        for _ in range(s - 1):
            x = x * x % n
            if x == n - 1:
                break
        else:
            return False
    return True


def negacyclic_mul(a, b, q: int):
    """Schoolbook product mod (X^N + 1, q) on Python ints."""

    n = len(a)
    out = [0] * n
    for i, ai in enumerate(a):
        if ai == 0:
            continue
        for j, bj in enumerate(b):
            k = i + j
            if k < n:
                out[k] = (out[k] + ai * bj) % q
            else:
                out[k - n] = (out[k - n] - ai * bj) % q
    return out


def crt(residues, primes) -> int:
    Q = 1
    for p in primes:
        Q *= p
    x = 0
    for r, p in zip(residues, primes):
        qi = Q // p
        x += int(r) * qi * pow(qi, -1, p)
    return x % Q


def centered(x: int, Q: int) -> int:
    x %= Q
    return x - Q if x > Q // 2 else x


def to_residues(coeffs, primes) -> np.ndarray:
    return np.array([[int(c) % p for c in coeffs] for p in primes], dtype=np.uint64)
