"""Client side: secret key, key generation, encrypt / decrypt.

Key material is drawn on the host from NumPy generators seeded by (spec.seed, purpose), so a
context's keys are reproducible -- for benchmarks and tests only; Holmes seeds its keys from a
fixed Blake2 seed, one PRNG stream per rotation (llama3fhe/parallel/prefill/keys.py:49-53), and
this backend declares its own streams.  Encryption randomness (the uniform a and the error e of
every encryption) is keyed from the operating system's entropy source (a Philox stream per
encryption), unless the spec asks for deterministic encryption.  All ring arithmetic (NTTs,
products, key assembly) runs on the GPU through libholmes_ckks.
"""

from __future__ import annotations

import hashlib
import os

import numpy as np
import torch

from . import _native as nat
from . import encoding
from .context import Cipher, CipherState, CKKSContext


def _rng(seed: int, *purpose) -> np.random.Generator:
    tag = hashlib.blake2b(repr((int(seed),) + tuple(purpose)).encode(), digest_size=16).digest()
    return np.random.Generator(np.random.PCG64(int.from_bytes(tag, "little")))


def _fresh_rng() -> np.random.Generator:
    """A generator keyed by 128 bits of OS entropy (a new key per call)."""

    return np.random.Generator(np.random.Philox(key=int.from_bytes(os.urandom(16), "little")))


def sample_ternary(rng: np.random.Generator, n: int, dist: str, h: int) -> np.ndarray:
    if str(dist).upper() == "SPARSE_TERNARY":
        s = np.zeros(n, dtype=np.int64)
        pos = rng.choice(n, size=int(h), replace=False)
        s[pos] = rng.choice(np.array([-1, 1], dtype=np.int64), size=int(h))
        return s
    return rng.integers(-1, 2, size=n, dtype=np.int64)


def sample_gaussian(rng: np.random.Generator, shape, sigma: float) -> np.ndarray:
    """Rounded Gaussian, tails cut at 6 sigma."""

    e = np.rint(rng.normal(0.0, float(sigma), size=shape))
    bound = np.ceil(6.0 * float(sigma))
    return np.clip(e, -bound, bound).astype(np.int64)


def sample_uniform(rng: np.random.Generator, primes, shape_prefix, n: int) -> np.ndarray:
    """Uniform residues: out[..., i, :] uniform in [0, primes[i])."""

    out = np.empty(tuple(shape_prefix) + (len(primes), n), dtype=np.uint64)
    for i, q in enumerate(primes):
        out[..., i, :] = rng.integers(0, int(q), size=tuple(shape_prefix) + (n,), dtype=np.uint64)
    return out


def automorph_coeff_signed(s: np.ndarray, g: int) -> np.ndarray:
    """sigma_g(s) for a signed coefficient vector: X^i -> X^(i g) mod X^N + 1."""

    n = s.size
    idx = (np.arange(n, dtype=np.int64) * int(g)) % (2 * n)
    out = np.zeros(n, dtype=np.int64)
    wrap = idx >= n
    out[idx[~wrap]] = s[~wrap]
    out[idx[wrap] - n] = -s[wrap]
    return out


class Client:
    """Holds the secret key; encrypts, decrypts and generates evaluation keys."""

    def __init__(self, context: CKKSContext):
        self.context = context
        spec = context.spec
        self.secret = sample_ternary(_rng(spec.seed, "secret"), context.N, spec.secret_key_dist, spec.hamming_weight)
        idx = list(range(context.L + context.K))
        s = torch.from_numpy(self.secret).reshape(1, -1).to(context.device)
        self._s_ntt = context.from_signed(s, idx)  # [1][L+K][N], NTT domain after the transform below
        context.ntt(self._s_ntt, prime_idx=idx)
        self._enc_counter = 0

    # ------------------------------------------------------------------ keys
    def rotation_key(self, galois: int) -> torch.Tensor:
        ctx = self.context
        spec = ctx.spec
        rng = _rng(spec.seed, "rotation-key", int(galois))
        a = sample_uniform(rng, ctx.primes, (ctx.beta_max,), ctx.N)
        e = sample_gaussian(rng, (ctx.beta_max, ctx.N), spec.error_sigma)
        s_from = automorph_coeff_signed(self.secret, galois)
        return ctx.make_switching_key(s_from, self.secret, a, e)

    def key_inputs(self, galois: int):
        """(s_from, s_to, a, e) used for the key of ``galois`` (for checkers)."""

        ctx = self.context
        spec = ctx.spec
        rng = _rng(spec.seed, "rotation-key", int(galois))
        a = sample_uniform(rng, ctx.primes, (ctx.beta_max,), ctx.N)
        e = sample_gaussian(rng, (ctx.beta_max, ctx.N), spec.error_sigma)
        return automorph_coeff_signed(self.secret, galois), self.secret.copy(), a, e

    def secret_square(self) -> np.ndarray:
        """Coefficients of s^2 in Z[X]/(X^N + 1), int64: the NTT-domain square over q_0, inverse
        transformed and centered (exact, since every coefficient of s^2 is at most the number of
        nonzero coefficients of s, far below q_0 / 2)."""

        ctx = self.context
        s0 = self._s_ntt[:, :1].contiguous()
        sq = ctx.empty(1, 1, ctx.N)
        ctx.poly_op(nat.HCK_OP_MUL, sq, s0, s0, prime_idx=[0])
        ctx.ntt(sq, prime_idx=[0], inverse=True)
        r = sq[0, 0].cpu().numpy().astype(np.int64)
        q0 = int(ctx.primes[0])
        return np.where(r > q0 // 2, r - q0, r).astype(np.int64)

    def relin_key_inputs(self):
        """(s_from = s^2, s_to = s, a, e) of the relinearisation key (for checkers)."""

        ctx = self.context
        spec = ctx.spec
        rng = _rng(spec.seed, "relin-key")
        a = sample_uniform(rng, ctx.primes, (ctx.beta_max,), ctx.N)
        e = sample_gaussian(rng, (ctx.beta_max, ctx.N), spec.error_sigma)
        return self.secret_square(), self.secret.copy(), a, e

    def relin_key(self) -> torch.Tensor:
        """The s^2 -> s key-switching key that relinearises a ciphertext product."""

        return self.context.make_switching_key(*self.relin_key_inputs())

    def generate_rotation_keys(self, rotations) -> None:
        ctx = self.context
        for r in rotations:
            g = ctx.M - 1 if int(r) == ctx.M - 1 else ctx.galois_element(int(r))
            if g not in ctx.rotation_keys:
                ctx.rotation_keys[g] = self.rotation_key(g)

    # ------------------------------------------------------------------ encrypt / decrypt
    def encrypt_coeffs(self, m: np.ndarray, cur_limbs: int, state: CipherState, slots: int) -> Cipher:
        """Encrypt integer coefficient vectors m ([batch][N] int64) under the secret key."""

        ctx = self.context
        m = np.atleast_2d(np.asarray(m, dtype=np.int64))
        idx = ctx.q_prime_idx(cur_limbs)
        pt = ctx.from_signed(torch.from_numpy(m).to(ctx.device), idx)
        ctx.ntt(pt, prime_idx=idx)
        return self.encrypt_ntt(pt, cur_limbs, state, slots)

    def encrypt_ntt(self, pt: torch.Tensor, cur_limbs: int, state: CipherState, slots: int) -> Cipher:
        """Encrypt NTT-domain plaintexts pt ([batch][>= cur_limbs][N]): (pt + e - a s, a)."""

        ctx = self.context
        B = int(pt.shape[0])
        self._enc_counter += 1
        if getattr(ctx.spec, "deterministic_encryption", False):
            rng = _rng(ctx.spec.seed, "encrypt", self._enc_counter)
        else:
            rng = _fresh_rng()
        e = sample_gaussian(rng, (B, ctx.N), ctx.spec.error_sigma)
        idx = ctx.q_prime_idx(cur_limbs)
        mpe = ctx.from_signed(torch.from_numpy(e).to(ctx.device), idx)
        ctx.ntt(mpe, prime_idx=idx)
        ctx.poly_op(nat.HCK_OP_ADD, mpe, mpe, pt[:, :cur_limbs], prime_idx=idx)
        a = torch.from_numpy(sample_uniform(rng, ctx.primes[:cur_limbs], (B,), ctx.N)).to(ctx.device)
        s = self._s_ntt[:, :cur_limbs].expand(B, -1, -1)
        as_ = ctx.empty(B, cur_limbs, ctx.N)
        ctx.poly_op(nat.HCK_OP_MUL, as_, a, s.contiguous(), prime_idx=idx)
        c0 = ctx.empty(B, cur_limbs, ctx.N)
        ctx.poly_op(nat.HCK_OP_SUB, c0, mpe, as_, prime_idx=idx)
        return Cipher([c0, a], state, slots=slots, batch_size=B)

    def encrypt(self, values, *, device=None, slots: int | None = None, cur_limbs: int | None = None,
                scaling_factor: float | None = None) -> Cipher:
        """Encode + encrypt one vector (or a [batch][slots] array) of real/complex values."""

        ctx = self.context
        slots = ctx.max_slots if slots is None else int(slots)
        cur_limbs = ctx.L if cur_limbs is None else int(cur_limbs)
        scale = ctx.scale_at(cur_limbs) if scaling_factor is None else float(scaling_factor)
        re, im = ctx.slot_rows(values, slots)
        pt = ctx.encode(re, scale, cur_limbs, values_im=im)
        state = CipherState(cur_limbs=cur_limbs, scale_degree=1, scaling_factor=scale)
        return self.encrypt_ntt(pt, cur_limbs, state, slots)

    def decrypt_coeffs(self, cipher: Cipher) -> np.ndarray:
        """Centered integer coefficients of c0 + c1 s (object array of Python ints, [batch][N])."""

        ctx = self.context
        limbs = int(cipher.state.cur_limbs)
        if cipher.is_ext:
            raise ValueError("decrypt needs a non-extended ciphertext")
        idx = ctx.q_prime_idx(limbs)
        c0, c1 = cipher.cv
        B = c0.shape[0]
        s = self._s_ntt[:, :limbs].expand(B, -1, -1).contiguous()
        m = ctx.empty(B, limbs, ctx.N)
        ctx.poly_op(nat.HCK_OP_MUL, m, c1[:, :limbs].contiguous(), s, prime_idx=idx)
        ctx.poly_op(nat.HCK_OP_ADD, m, m, c0[:, :limbs].contiguous(), prime_idx=idx)
        use = min(limbs, 2)
        ctx.ntt(m, prime_idx=idx, inverse=True)
        res = m[:, :use].cpu().numpy()
        return crt_centered(res, ctx.q_primes[:use])

    def decrypt(self, cipher: Cipher) -> np.ndarray:
        coeffs = self.decrypt_coeffs(cipher)
        ctx = self.context
        out = [encoding.decode(c.astype(np.float64), cipher.state.scaling_factor, ctx.logN, cipher.slots)
               for c in coeffs]
        out = np.stack(out)
        return out[0] if out.shape[0] == 1 else out


def crt_centered(res: np.ndarray, primes) -> np.ndarray:
    """Centered CRT of residues res[batch][len(primes)][N] -> object array of Python ints."""

    primes = [int(p) for p in primes]
    Q = 1
    for p in primes:
        Q *= p
    B, _, n = res.shape
    out = np.empty((B, n), dtype=object)
    terms = []
    for i, p in enumerate(primes):
        qi = Q // p
        terms.append((qi, pow(qi % p, -1, p), p))
    for b in range(B):
        acc = np.zeros(n, dtype=object)
        for i, (qi, inv, p) in enumerate(terms):
            r = res[b, i].astype(object)
            acc = acc + ((r * inv) % p) * qi
        acc = acc % Q
        half = Q // 2
        out[b] = np.where(acc > half, acc - Q, acc)
    return out


__all__ = ["Client", "crt_centered", "automorph_coeff_signed"]
