"""Pins of the oracle's ModUp, ModDown, key switch, key generation, rescale and BSGS MAC.

ModUp must be an approximate CRT lift (residues of X + u Q_j for the centered digit value X and
one integer |u| <= (digit size + 1) / 2, the same for every target prime); ModDown must be
round(Z / P) - u with |u| <= (K + 1) / 2; rescale must be round(X / q_last) exactly; a key switch must satisfy b + a s = d s' + small noise
(mod Q); the MAC must equal the big-integer sum.  All checked with Python big integers on
small rings (N = 2^4 .. 2^10), so a dropped term, a wrong index or a transposed operand fails.
"""

from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import centered, crt


# Both chain widths the GPU tests run on: 50-bit primes (the FP64 path) and the reference's
# production shape (assets/feature_major.json:3-14): a 60-bit first modulus, 59-bit Q primes, 60-bit
# special primes (the wide path).  Every pin below runs on both.
pytestmark = pytest.mark.parametrize("chain", ["50", "60/59"])


def _ctx(log_n, L, K, alpha, chain="50"):
    if chain == "50":
        ps = O.gen_primes(log_n, 50, L + K)
        P, Q = ps[:K], ps[K:]
    else:
        P = O.gen_primes(log_n, 60, K)
        q0 = O.gen_primes(log_n, 60, 1, exclude=P)
        Q = q0 + O.gen_primes(log_n, 59, L - 1)
    return O.OracleContext(log_n, L, K, alpha, Q + P)


def _rand_ntt(ctx, rng, limbs, prime_idx=None):
    prime_idx = list(range(limbs)) if prime_idx is None else prime_idx
    return np.stack([rng.integers(0, ctx.primes[i], ctx.n, dtype=np.uint64) for i in prime_idx])


@pytest.mark.parametrize("ell,digit", [(6, 0), (6, 2), (5, 2), (4, 1)])
def test_modup_is_approximate_crt_lift(ell, digit, chain):
    ctx = _ctx(4, 6, 2, 2, chain=chain)
    rng = np.random.default_rng(ell * 10 + digit)
    d = _rand_ntt(ctx, rng, ell)
    ext = ctx.modup(ell, digit, d)
    coef_d = ctx.ntt_inv_limbs(d, list(range(ell)))
    ext_idx = list(range(ell)) + [ctx.L + k for k in range(ctx.K)]
    coef_e = ctx.ntt_inv_limbs(ext, ext_idx)
    lo, hi = digit * ctx.alpha, min((digit + 1) * ctx.alpha, ell)
    src = [ctx.primes[i] for i in range(lo, hi)]
    Qj = 1
    for p in src:
        Qj *= p
    all_primes = [ctx.primes[i] for i in ext_idx]
    big = 1
    for p in all_primes:
        big *= p
    for t in range(ctx.n):
        X = centered(crt([int(coef_d[i][t]) for i in range(lo, hi)], src), Qj)
        W = centered(crt([int(coef_e[e][t]) for e in range(len(ext_idx))], all_primes), big)
        u, r = divmod(W - X, Qj)
        assert r == 0 and abs(u) <= (len(src) + 1) // 2
        # with centered y_s = [x_s (Q_j/q_s)^-1]_{q_s}, u = sum_s y_s / q_s - X / Q_j exactly
        ys = [centered(int(coef_d[i][t]) * pow(Qj // ctx.primes[i], -1, ctx.primes[i]), ctx.primes[i])
              for i in range(lo, hi)]
        assert Fraction(u) == sum(Fraction(y, p) for y, p in zip(ys, src)) - Fraction(X, Qj)
    # the digit's own limbs pass through unchanged (NTT domain)
    assert np.array_equal(ext[lo:hi], d[lo:hi])


@pytest.mark.parametrize("ell", [6, 3])
def test_moddown_is_rounded_division_by_P(ell, chain):
    ctx = _ctx(4, 6, 3, 2, chain=chain)
    rng = np.random.default_rng(ell)
    ext_idx = list(range(ell)) + [ctx.L + k for k in range(ctx.K)]
    x = _rand_ntt(ctx, rng, len(ext_idx), ext_idx)
    out = ctx.moddown(ell, x)
    cx = ctx.ntt_inv_limbs(x, ext_idx)
    co = ctx.ntt_inv_limbs(out, list(range(ell)))
    qp = [ctx.primes[i] for i in ext_idx]
    q = ctx.primes[:ell]
    P = 1
    for p in ctx.primes[ctx.L:]:
        P *= p
    Q = 1
    for p in q:
        Q *= p
    for t in range(ctx.n):
        Z = crt([int(cx[e][t]) for e in range(len(ext_idx))], qp)
        Ov = crt([int(co[i][t]) for i in range(ell)], q)
        k = (Z - centered(Z, P)) // P  # round(Z / P)
        u = centered(k - Ov, Q)
        assert abs(u) <= (ctx.K + 1) // 2
    # ModDown(P * y) = y exactly
    y = _rand_ntt(ctx, rng, ell)
    py = np.zeros_like(x)
    for i in range(ell):
        Pm = P % ctx.primes[i]
        py[i] = np.array([int(v) * Pm % ctx.primes[i] for v in y[i]], dtype=np.uint64)
    assert np.array_equal(ctx.moddown(ell, py), y)


@pytest.mark.parametrize("ell", [2, 5])
def test_rescale_is_exact_rounding(ell, chain):
    ctx = _ctx(4, 5, 1, 2, chain=chain)
    rng = np.random.default_rng(100 + ell)
    x = _rand_ntt(ctx, rng, ell)
    out = ctx.rescale(ell, x)
    cx = ctx.ntt_inv_limbs(x, list(range(ell)))
    co = ctx.ntt_inv_limbs(out, list(range(ell - 1)))
    q = ctx.primes[:ell]
    for t in range(ctx.n):
        X = crt([int(cx[i][t]) for i in range(ell)], q)
        want = (X - centered(X, q[-1])) // q[-1]  # round(X / q_last)
        assert [int(co[i][t]) for i in range(ell - 1)] == [want % p for p in q[:-1]]


def _ternary(rng, n):
    return rng.integers(-1, 2, n, dtype=np.int64)


def _automorph_signed(s, g):
    n = s.size
    out = np.zeros(n, np.int64)
    for i in range(n):
        e = i * g % (2 * n)
        if e < n:
            out[e] += s[i]
        else:
            out[e - n] -= s[i]
    return out


def _poly_ntt(ctx, coeffs, prime_idx):
    res = np.stack([np.array([int(c) % ctx.primes[i] for c in coeffs], dtype=np.uint64) for i in prime_idx])
    return ctx.ntt_fwd_limbs(res, prime_idx)


@pytest.mark.parametrize("ell", [6, 5, 3])
def test_keyswitch_decrypt_invariant(ell, chain):
    """b + a s - d s' is small mod Q_ell: key generation and key switch agree with the algebra."""

    log_n, L, K, alpha = 10, 6, 2, 2
    ctx = _ctx(log_n, L, K, alpha, chain=chain)
    rng = np.random.default_rng(5 + ell)
    n = ctx.n
    s = _ternary(rng, n)
    g = 5 ** 3 % (2 * n)
    s_from = _automorph_signed(s, g)
    beta = ctx.beta(L)
    a = np.stack([_rand_ntt(ctx, rng, L + K, list(range(L + K))) for _ in range(beta)])
    e = np.rint(rng.normal(0, 3.2, (beta, n))).astype(np.int64)
    ksk = ctx.make_ksk(s_from, s, a, e)
    assert np.array_equal(ksk[1], a)
    d = _rand_ntt(ctx, rng, ell)
    b_out, a_out = ctx.keyswitch(ell, d, ksk)
    idx = list(range(ell))
    sn = _poly_ntt(ctx, s, idx)
    sfn = _poly_ntt(ctx, s_from, idx)
    err = np.zeros((ell, n), dtype=np.uint64)
    for i in idx:
        q = ctx.primes[i]
        err[i] = np.array(
            [(int(b_out[i][t]) + int(a_out[i][t]) * int(sn[i][t]) - int(d[i][t]) * int(sfn[i][t])) % q for t in range(n)],
            dtype=np.uint64,
        )
    ce = ctx.ntt_inv_limbs(err, idx)
    q = ctx.primes[:ell]
    Q = 1
    for p in q:
        Q *= p
    worst = max(abs(centered(crt([int(ce[i][t]) for i in idx], q), Q)) for t in range(n))
    assert worst < 2**20, worst


def test_keyswitch_key_is_gadget_of_secret(chain):
    """b_j + a_j s - e_j = P T_j s' with T_j = 1 on digit j, 0 on other Q primes and on P."""

    log_n, L, K, alpha = 5, 5, 2, 2
    ctx = _ctx(log_n, L, K, alpha, chain=chain)
    rng = np.random.default_rng(3)
    n = ctx.n
    s, sf = _ternary(rng, n), _ternary(rng, n)
    beta = ctx.beta(L)
    idx = list(range(L + K))
    a = np.stack([_rand_ntt(ctx, rng, L + K, idx) for _ in range(beta)])
    e = np.rint(rng.normal(0, 3.2, (beta, n))).astype(np.int64)
    ksk = ctx.make_ksk(sf, s, a, e)
    sn, sfn = _poly_ntt(ctx, s, idx), _poly_ntt(ctx, sf, idx)
    P = 1
    for p in ctx.primes[L:]:
        P *= p
    for j in range(beta):
        en = _poly_ntt(ctx, e[j], idx)
        for i in idx:
            q = ctx.primes[i]
            gadget = (P % q) if (i < L and i // alpha == j) else 0
            lhs = [(int(ksk[0][j][i][t]) + int(a[j][i][t]) * int(sn[i][t]) - int(en[i][t])) % q for t in range(n)]
            rhs = [gadget * int(sfn[i][t]) % q for t in range(n)]
            assert lhs == rhs


def test_bsgs_mac_matches_big_integer_sum(chain):
    ctx = _ctx(4, 3, 1, 3, chain=chain)
    rng = np.random.default_rng(9)
    limbs, nb, G = 3, 4, 2
    pt = np.stack([_rand_ntt(ctx, rng, limbs) for _ in range(G * nb)])
    baby = np.stack([np.stack([_rand_ntt(ctx, rng, limbs) for _ in range(2)]) for _ in range(nb)])
    res = ctx.bsgs_mac(limbs, nb, G, pt, baby)
    for c in range(2):
        for g in range(G):
            for l in range(limbs):
                q = ctx.primes[l]
                for j in range(ctx.n):
                    want = sum(int(pt[g * nb + b][l][j]) * int(baby[b][c][l][j]) for b in range(nb)) % q
                    assert int(res[c][g][l][j]) == want


@pytest.mark.parametrize("to", [2, 5])
def test_modraise_is_the_centered_lift(to, chain):
    # every output limb holds the centered representative of limb 0's coefficient (|x| < q_0 / 2)
    # reduced modulo its own prime; limb 0 is unchanged
    ctx = _ctx(4, 5, 1, 2, chain=chain)
    rng = np.random.default_rng(200 + to)
    x = _rand_ntt(ctx, rng, 1)
    out = ctx.modraise(to, x[0])
    assert np.array_equal(out[0], x[0])
    c0 = ctx.ntt_inv_limbs(x, [0])[0]
    co = ctx.ntt_inv_limbs(out, list(range(to)))
    q0 = ctx.primes[0]
    for t in range(ctx.n):
        v = centered(int(c0[t]), q0)
        assert [int(co[i][t]) for i in range(to)] == [v % ctx.primes[i] for i in range(to)]
