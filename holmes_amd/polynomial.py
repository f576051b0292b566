"""Chebyshev series on ciphertexts with exact scales (the polynomial evaluator of
llama3fhe/operators/nonlinear/polynomial.py:140-562 and llama3fhe/approx/chebyshev.py, used by
SiLU, the RMSNorm inverse square root and the bootstrap's EvalMod).

Paterson-Stockmeyer over the Chebyshev basis: baby basis T_1..T_k (one batched product per depth),
giants T_k, T_2k, ..., and p = q T_M + r split recursively (``chebyshev_divide``).  Every ciphertext
at l limbs carries the canonical scale S_(l) of its level (``canonical_scales``): products of two
operands of one level land on the next level's scale, linear combinations encode each coefficient
at the ratio that lands its term on the target scale, so additions never mix scales.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import _native as _nat
from . import fhe
from .context import Cipher, CKKSContext, u64_cat

__all__ = ["PSEvaluator", "canonical_scales", "chebyshev_divide", "chebyshev_coefficients", "eval_chebyshev",
           "chebyshev_depth", "series_from_entry", "entry_coefficients"]


def chebyshev_divide(coeffs: np.ndarray, M: int) -> tuple[np.ndarray, np.ndarray]:
    """p = q T_M + r for a Chebyshev series p of length <= 2M: T_(M+a) = 2 T_M T_a - T_(M-a)."""

    c = np.asarray(coeffs, dtype=np.float64)
    if len(c) <= M:
        return np.zeros(1), c.copy()
    if len(c) > 2 * M:
        raise ValueError("chebyshev_divide needs len(coeffs) <= 2 M")
    q = np.zeros(len(c) - M)
    r = c[:M].copy()
    q[0] = c[M]
    for a in range(1, len(c) - M):
        q[a] = 2.0 * c[M + a]
        r[M - a] -= c[M + a]
    return q, r


def _baby_size(degree: int) -> int:
    return 1 << max(1, math.ceil(math.log2(math.sqrt(degree + 1))))


def canonical_scales(primes, top_limbs: int, top_scale: float) -> dict:
    """Scale of a ciphertext at each level below ``top_limbs`` when every product multiplies two
    operands of one level and rescales: S_(l) = S_(l+1)^2 / q_l (q_l the prime the rescale from
    l + 1 limbs drops)."""

    out = {int(top_limbs): float(top_scale)}
    for l in range(int(top_limbs) - 1, 0, -1):
        out[l] = out[l + 1] * out[l + 1] / float(primes[l])
    return out


class PSEvaluator:
    """Chebyshev series on a cipher batch with slots in [-1, 1], every scale exact.

    Paterson-Stockmeyer over the Chebyshev basis (the split of the reference's evaluator,
    llama3fhe/operators/nonlinear/polynomial.py:140-330): baby basis T_1 .. T_k, giants T_k, T_2k,
    ..., p = q T_M + r (``chebyshev_divide``) recursively.  Every ciphertext at l limbs carries the
    canonical scale S_(l) (``canonical_scales``): a product of two operands at one level lands on
    the next level's scale, a linear combination encodes each coefficient at the ratio that lands
    its term on the target scale (so it changes level and scale for free), and ``adjust`` (one
    scalar product and rescale) brings any other operand down to a level.  Additions therefore
    never mix scales.  With ``sim`` the operands are plain limb counts: the same schedule run for
    its levels only (the program's depth)."""

    def __init__(self, ctx: CKKSContext | None, x, limbs: int, scale: float, degree: int, primes,
                 sim: bool = False):
        self.ctx = ctx
        self.sim = bool(sim)
        self.primes = [int(p) for p in primes]
        self.canon = canonical_scales(self.primes, limbs, scale)
        self.k = _baby_size(degree)
        self._adj: dict = {}
        T = {1: (limbs if self.sim else self._fix(x, limbs))}
        j0 = 1
        while j0 < self.k:  # T_(j0+1) .. T_(2 j0) from T_(j/2) T_(j - j/2): one batched product per depth
            js = list(range(j0 + 1, min(2 * j0, self.k) + 1))
            pairs = [(T[j // 2], T[j - j // 2]) for j in js]
            subs = [None if j // 2 == j - j // 2 else T[j - 2 * (j // 2)] for j in js]
            for j, t in zip(js, self.mul_many_double(pairs, subs)):
                T[j] = t
            j0 *= 2
        M = 2 * self.k
        while M <= degree:
            T[M] = self.double_minus(T[M // 2], T[M // 2])
            M *= 2
        self.T = T

    # -- primitives (ciphertexts, or limb counts when simulating)
    def lv(self, x) -> int:
        return int(x) if self.sim else int(x.state.cur_limbs)

    def _fix(self, ct: Cipher, l: int) -> Cipher:
        want = self.canon[l]
        got = float(ct.state.scaling_factor)
        if abs(got - want) > 2.0**-40 * want:
            raise AssertionError(f"scale {got} at {l} limbs drifted from {want}")
        return ct.cipher_like(ct.cv, state=ct.state.replace(scaling_factor=want, scale_degree=1))

    def _combine(self, terms, limbs: int, weights: np.ndarray) -> list:
        """sum_t weights[t] * terms[t] (residue tables [terms][limbs]) for every component and item,
        each term read at its own level: one hck_lincomb launch."""

        ctx = self.ctx
        B = terms[0].batch_size
        out = fhe._alloc(ctx, 2, B, limbs)
        xs = [[x.cv[c][b] for x in terms] for c in range(2) for b in range(B)]
        ctx.lincomb(xs, limbs, [out[c][b] for c in range(2) for b in range(B)],
                    ctx.resident(np.asarray(weights, dtype=np.uint64)))
        return out

    def _combine_rescale(self, terms, limbs: int, weights: np.ndarray, c0: float = 0.0) -> list:
        """rescale(sum_t weights[t] * terms[t]) at ``limbs - 1`` limbs, plus c0 (encoded at that level's
        canonical scale) on the c0 component: one hck_lincomb_rescale, the combination never stored."""

        ctx = self.ctx
        B = terms[0].batch_size
        l = limbs - 1
        out = fhe._alloc(ctx, 2, B, l)
        xs = [[x.cv[c][b] for x in terms] for c in range(2) for b in range(B)]
        add = None if c0 == 0.0 else [int(v) for v in self._residues(float(c0), l, self.canon[l])]
        ctx.lincomb_rescale(xs, limbs, [out[c][b] for c in range(2) for b in range(B)],
                            ctx.resident(np.asarray(weights, dtype=np.uint64)), add=add,
                            add_groups=range(B) if add is not None else ())
        return out

    def _residues(self, value: float, limbs: int, scaling_factor: float, integer: bool = False) -> np.ndarray:
        return fhe._scalar_residues(value, limbs, scaling_factor, integer, self.ctx)[0]

    def adjust(self, x, l: int):
        lx = self.lv(x)
        if lx == l:
            return x
        if lx < l:
            raise AssertionError(f"cannot raise an operand from {lx} to {l} limbs")
        if self.sim:
            return l
        key = (id(x), l)
        hit = self._adj.get(key)
        if hit is not None and hit[0] is x:
            return hit[1]
        ratio = self.canon[l] * float(self.primes[l]) / self.canon[lx]
        out = self._combine_rescale([x], l + 1, self._residues(1.0, l + 1, ratio)[None])
        y = self._fix(x.cipher_like(out, state=x.state.replace(
            cur_limbs=l, scale_degree=1,
            scaling_factor=self.canon[l] * float(self.primes[l]) / float(self.ctx.rescale_divisor_at(l + 1)))), l)
        self._adj[key] = (x, y)
        return y

    def mul(self, a, b):
        l = min(self.lv(a), self.lv(b))
        if l < 2:
            raise ValueError("EvalMod ran out of levels")
        a, b = self.adjust(a, l), self.adjust(b, l)
        if self.sim:
            return l - 1
        return self._fix(fhe.homo_mul_relin_rescale(a, b, self.ctx), l - 1)

    def add(self, a, b):
        l = min(self.lv(a), self.lv(b))
        a, b = self.adjust(a, l), self.adjust(b, l)
        return l if self.sim else fhe.homo_add(a, b, self.ctx)

    def _add_const_inplace(self, x, c: float):
        """c added to every slot of ``x`` (a temporary this evaluator owns), in place on c0."""

        if self.sim or c == 0.0:
            return x
        l = self.lv(x)
        res = self._residues(float(c), l, self.canon[l])
        self.ctx.poly_op(_nat.HCK_OP_ADD_SCALAR, x.cv[0], x.cv[0], prime_idx=self.ctx.q_prime_idx(l),
                         scalar=[int(v) for v in res])
        return x

    def mul_many(self, pairs) -> list:
        """Products of several operand pairs (relinearised and rescaled), every operand first brought
        to the lowest level among them; small batches go as one batched call."""

        if len(pairs) == 1 or self.sim:
            return [self.mul(a, b) for a, b in pairs]
        l = min(self.lv(x) for pr in pairs for x in pr)
        if l < 2:
            raise ValueError("EvalMod ran out of levels")
        ops = [(self.adjust(a, l), self.adjust(b, l)) for a, b in pairs]
        B = ops[0][0].batch_size
        if B >= 16:  # a launch sequence per pair is already large: no operand copies
            return [self._fix(fhe.homo_mul_relin_rescale(a, b, self.ctx), l - 1) for a, b in ops]
        side = [[u64_cat([pr[k].cv[c][:, :l] for pr in ops]) for c in range(2)] for k in range(2)]
        both = self.ctx.mul_relin_rescale_raw(side[0][0], side[0][1], side[1][0], side[1][1], l, self.ctx.relin_key,
                                              stacked=True)
        x0 = ops[0][0]
        n = len(ops) * B
        r = self._fix(x0.cipher_like([both[0], both[1]], batch_size=n,
                                     state=x0.state.replace(cur_limbs=l - 1, scale_degree=1,
                                                            scaling_factor=self.canon[l] * self.canon[l]
                                                            / float(self.ctx.rescale_divisor_at(l)))), l - 1)
        return [r.cipher_like([c[i * B:(i + 1) * B] for c in r.cv], batch_size=B) for i in range(len(ops))]

    def _finish_double(self, p, sub=None):
        """2 p - sub (sub = None: - 1) for a product p on its canonical scale."""

        if self.sim:
            return p
        l = self.lv(p)
        terms = [p] if sub is None else [p, self.adjust(sub, l)]
        w = np.stack([self._residues(v, l, 1.0, integer=True) for v in ((2,) if sub is None else (2, -1))])
        out = p.cipher_like(self._combine(terms, l, w))
        return self._add_const_inplace(out, -1.0) if sub is None else out

    def _mul_double(self, a, b, sub, l: int):
        """2 a b - sub (sub = None: - 1) for a, b at l limbs: one hck_mul_relin_rescale_postop (the
        doubling, the subtraction and the constant ride on the product's last kernel)."""

        ctx = self.ctx
        pair = sc = None
        if sub is None:
            sc = [int(v) for v in self._residues(-1.0, l - 1, self.canon[l - 1])]
        else:
            s = self.adjust(sub, l - 1)
            pair = tuple(c[:, :l - 1] for c in s.cv)
        both = ctx.mul_relin_rescale_postop_raw(a.cv[0][:, :l], a.cv[1][:, :l], b.cv[0][:, :l], b.cv[1][:, :l], l,
                                                ctx.relin_key, apply_double=True, sub=pair, scalar=sc)
        state = a.state.replace(cur_limbs=l - 1, scale_degree=1,
                                scaling_factor=self.canon[l] * self.canon[l] / float(ctx.rescale_divisor_at(l)))
        return self._fix(a.cipher_like([both[0], both[1]], state=state), l - 1)

    def mul_many_double(self, pairs, subs) -> list:
        """2 a b - sub (sub None: - 1) for every pair, every operand first brought to the lowest
        level among them (as ``mul_many``)."""

        if self.sim:
            return [self._finish_double(p, s) for p, s in zip(self.mul_many(pairs), subs)]
        l = min(self.lv(x) for pr in pairs for x in pr)
        if l < 2:
            raise ValueError("EvalMod ran out of levels")
        B = pairs[0][0].batch_size
        if len(pairs) == 1 or B >= 16:
            return [self._mul_double(self.adjust(a, l), self.adjust(b, l), s, l) for (a, b), s in zip(pairs, subs)]
        return [self._finish_double(p, s) for p, s in zip(self.mul_many(pairs), subs)]

    def double_minus(self, a, b, sub=None):
        """2 a b - sub (sub = None: - 1)."""

        if self.sim:
            return self._finish_double(self.mul(a, b), sub)
        return self.mul_many_double([(a, b)], [sub])[0]

    def lincomb(self, terms, c0: float, cap: int | None):
        """c0 + sum c_j x_j over ``terms`` = [(c_j, x_j)], rescaled once, at min(level) - 1 or ``cap``:
        each coefficient is encoded at the ratio that lands its term on the target scale, and the
        terms are read at their own levels by one hck_lincomb_rescale (c0 added in its last kernel)."""

        l = min(self.lv(x) for _, x in terms) - 1
        if cap is not None:
            l = min(l, int(cap))
        if l < 1:
            raise ValueError("EvalMod ran out of levels")
        if self.sim:
            return l
        target = self.canon[l] * float(self.primes[l])
        w = np.stack([self._residues(float(c), l + 1, target / self.canon[self.lv(x)]) for c, x in terms])
        x0 = terms[0][1]
        out = self._combine_rescale([x for _, x in terms], l + 1, w, c0)
        return self._fix(x0.cipher_like(out, state=x0.state.replace(
            cur_limbs=l, scale_degree=1, scaling_factor=target / float(self.ctx.rescale_divisor_at(l + 1)))), l)

    # -- the series
    def evaluate(self, coeffs, cap: int | None = None):
        c = np.asarray(coeffs, dtype=np.float64)
        if len(c) <= self.k:
            terms = [(c[j], self.T[j]) for j in range(1, len(c)) if c[j] != 0.0] or [(0.0, self.T[1])]
            return self.lincomb(terms, float(c[0]), cap)
        M = self.k
        while 2 * M < len(c):
            M *= 2
        q, r = chebyshev_divide(c, M)
        TM = self.T[M]
        if len(q) == 1:
            prod = self.lincomb([(q[0], TM)], 0.0, cap)
        else:
            qe = self.evaluate(q, self.lv(TM) if cap is None else min(self.lv(TM), cap + 1))
            prod = self.mul(qe, TM)
            if cap is not None and self.lv(prod) > cap:
                prod = self.adjust(prod, cap)
        re = self.evaluate(r, self.lv(prod))
        return self.add(prod, re)


def chebyshev_coefficients(fn, degree: int, interval=(-1.0, 1.0)) -> np.ndarray:
    """Chebyshev interpolant of ``fn`` on ``interval`` at the Chebyshev points of the first kind,
    as a series in u = (2x - (a + b)) / (b - a) (np.polynomial.chebyshev.chebinterpolate)."""

    a, b = (float(v) for v in interval)
    if not b > a:
        raise ValueError("interval must be increasing")
    return np.polynomial.chebyshev.chebinterpolate(lambda u: fn(0.5 * (b - a) * u + 0.5 * (a + b)), int(degree))


def series_from_entry(entry: dict) -> np.ndarray:
    """The numpy-convention series (sum_j c_j T_j) of a reference coefficient dictionary, whose
    evaluator halves the constant term (llama3fhe/approx/chebyshev.py:136-163: c_0 / 2 +
    sum_(j>=1) c_j T_j)."""

    c = np.array(entry["coefficients"], dtype=np.float64)
    if len(c):
        c[0] *= 0.5
    return c


def entry_coefficients(series) -> np.ndarray:
    """Coefficients in the reference dictionary's convention for a numpy-convention series."""

    c = np.array(series, dtype=np.float64)
    if len(c):
        c[0] *= 2.0
    return c


def chebyshev_depth(degree: int) -> int:
    """Levels ``eval_chebyshev`` consumes for a series of ``degree`` (the affine map included)."""

    ev = PSEvaluator(None, None, 1024, 1.0, int(degree), [2] * 1025, sim=True)
    return 1 + 1024 - int(ev.evaluate(np.ones(int(degree) + 1)))


def eval_chebyshev(ct: Cipher, coeffs, ctx: CKKSContext, interval=(-1.0, 1.0)) -> Cipher:
    """sum_j c_j T_j(u(x)) slot-wise, u = (2x - (a + b)) / (b - a) taking ``interval`` to [-1, 1]
    (one scalar product + rescale), then the Paterson-Stockmeyer evaluation.  The output sits on
    the canonical scale of its level (exact bookkeeping in ``state.scaling_factor``)."""

    a, b = (float(v) for v in interval)
    limbs = int(ct.state.cur_limbs)
    if limbs < 3:
        raise ValueError("a Chebyshev series needs more limbs")
    alpha, beta = 2.0 / (b - a), -(a + b) / (b - a)
    q = float(ctx.rescale_divisor_at(limbs))
    enc = fhe.encode_scalar(alpha, cur_limbs=limbs, scale_degree=1, scaling_factor=q, context=ctx)
    u = fhe.homo_mul_scalar_rescale(ct, enc, ctx)
    S = float(ct.state.scaling_factor)
    u = u.cipher_like(u.cv, state=u.state.replace(scaling_factor=S, scale_degree=1))
    if beta != 0.0:
        u = fhe.homo_add_scalar(u, fhe.encode_scalar(beta, cur_limbs=limbs - 1, scale_degree=1, scaling_factor=S,
                                                      context=ctx), ctx)
    coeffs = np.asarray(coeffs, dtype=np.float64)
    ev = PSEvaluator(ctx, u, limbs - 1, S, len(coeffs) - 1, ctx.q_primes)
    return ev.evaluate(coeffs)
