"""CKKS parameter set: context spec and the RNS prime chain.

``CKKSContextSpec`` keeps the keyword surface of EasyFHE's spec as Holmes builds it
(llama3fhe/backend.py:574-588, llama3fhe/application/session.py:44-59: depth, log_n, dnum,
dcrt_bits, first_mod, secret_key_dist, scale_mode, rescale_policy, rotations, auto_load_keys,
rotation_key_limb_limits) plus the fields this backend adds (special_bits, scale_bits,
num_special, seed).
"""

from __future__ import annotations

from dataclasses import dataclass, field


def _mr_prime(n: int) -> bool:
    """Deterministic Miller-Rabin for n < 2^64."""

    if n < 2:
        return False
    small = (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37)
    for p in small:
        if n % p == 0:
            return n == p
    d, s = n - 1, 0
    while d % 2 == 0:
        d //= 2
        s += 1
    for a in small:
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


def ntt_primes(log_n: int, bits: int, count: int, exclude=()) -> list[int]:
    """The ``count`` largest primes below 2^bits that are 1 mod 2N, skipping ``exclude``.

    Candidates are 2^bits + 1 - k * 2N for k = 1, 2, ... in that order.
    """

    step = 2 << int(log_n)
    excl = set(int(v) for v in exclude)
    out: list[int] = []
    c = (1 << int(bits)) + 1 - step
    while len(out) < int(count):
        if c <= step:
            raise ValueError(f"not enough {bits}-bit NTT primes for N=2^{log_n}")
        if c not in excl and _mr_prime(c):
            out.append(c)
        c -= step
    return out


@dataclass(frozen=True)
class CKKSContextSpec:
    depth: int = 23
    log_n: int = 16
    dnum: int = 3
    dcrt_bits: int = 50
    first_mod: int = 50
    secret_key_dist: str = "UNIFORM_TERNARY"
    scale_mode: str = "fixed"
    rescale_policy: str = "manual"
    rotations: tuple = ()
    auto_load_keys: bool = True
    rotation_key_limb_limits: dict | None = None
    special_bits: int | None = None
    num_special: int | None = None
    scale_bits: int = 40
    seed: int = 20261201
    hamming_weight: int = 192
    error_sigma: float = 3.2
    # Key material (secret, key-switching keys) is generated from ``seed`` so that a context is
    # reproducible (the reference seeds its keys the same way, parallel/prefill/keys.py:49-53).
    # Encryption randomness (a, e) comes from the OS entropy source unless this is set: two
    # clients of one spec must not encrypt with the same (a, e).  Tests that need repeatable
    # ciphertexts set it.
    deterministic_encryption: bool = False

    @property
    def num_q(self) -> int:
        return int(self.depth) + 1

    @property
    def alpha(self) -> int:
        return -(-self.num_q // int(self.dnum))

    @property
    def num_p(self) -> int:
        return int(self.num_special) if self.num_special is not None else self.alpha

    def prime_chain(self) -> tuple[list[int], list[int]]:
        """(Q primes, P primes).  The special primes are the largest ``special_bits``-bit NTT
        primes; q_0 is the largest ``first_mod``-bit prime not used by P; the rest of Q are the
        next ``dcrt_bits``-bit primes."""

        sbits = int(self.special_bits) if self.special_bits is not None else max(
            int(self.dcrt_bits), int(self.first_mod)
        )
        P = ntt_primes(self.log_n, sbits, self.num_p)
        q0 = ntt_primes(self.log_n, int(self.first_mod), 1, exclude=P)
        rest = ntt_primes(self.log_n, int(self.dcrt_bits), self.num_q - 1, exclude=P + q0)
        return q0 + rest, P

    def validate(self) -> None:
        if int(self.log_n) != 16:
            raise ValueError("this backend's kernels are built for N = 2^16 (log_n = 16)")
        if self.num_q < 2 or int(self.dnum) < 1:
            raise ValueError("need depth >= 1 and dnum >= 1")
        for bits in (self.dcrt_bits, self.first_mod, self.special_bits or self.dcrt_bits):
            # primes below 2^50 run on the FP64-exact arithmetic; wider ones (the reference's 59/60-bit
            # chains) on the 64-bit integer path, which takes primes up to 2^61
            if not 32 <= int(bits) <= 60:
                raise ValueError(f"prime sizes from 32 to 60 bits are supported (got {bits}-bit primes)")
        if str(self.secret_key_dist).upper() not in ("UNIFORM_TERNARY", "SPARSE_TERNARY"):
            raise ValueError(f"unsupported secret key distribution {self.secret_key_dist!r}")
        if str(self.scale_mode) != "fixed":
            raise ValueError("only scale_mode='fixed' is supported")


__all__ = ["CKKSContextSpec", "ntt_primes"]
