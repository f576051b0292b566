"""Pins of the oracle's ciphertext product: the tensor product, relinearisation and the grouped
scalar-weighted sum.

The tensor product is checked through the convolution theorem (the NTT-domain tensor of encrypted
polynomials must be the NTT of the schoolbook negacyclic products, computed here with Python
integers); relinearisation by its defining invariant, d0 + d1 s + d2 s^2 = out0 + out1 s + small
(mod Q), with the s^2 -> s key made from an independently computed s^2; the weighted sum against
Python big-integer sums.  Small rings (N = 2^4 .. 2^6), so a swapped operand, a dropped cross term
or a wrong key fails.
"""

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import centered, crt, negacyclic_mul


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


def _rand_coeffs(ctx, rng, limbs):
    return np.stack([rng.integers(0, ctx.primes[i], ctx.n, dtype=np.uint64) for i in range(limbs)])


def negacyclic_square_py(s):
    """s^2 in Z[X]/(X^N + 1) over the integers (schoolbook, Python ints)."""

    n = len(s)
    out = [0] * n
    for i, a in enumerate(s):
        if a == 0:
            continue
        for j, b in enumerate(s):
            if b == 0:
                continue
            k = i + j
            if k < n:
                out[k] += a * b
            else:
                out[k - n] -= a * b
    return out


def test_tensor_is_the_ntt_of_the_negacyclic_products(chain):
    ctx = _ctx(5, 3, 1, 3, chain=chain)
    rng = np.random.default_rng(7)
    limbs = 3
    idx = list(range(limbs))
    coef = [_rand_coeffs(ctx, rng, limbs) for _ in range(4)]  # a0, a1, b0, b1 (coefficient domain)
    ntt = [ctx.ntt_fwd_limbs(c, idx) for c in coef]
    d0, d1, d2 = ctx.tensor(limbs, *ntt)
    got = [ctx.ntt_inv_limbs(d, idx) for d in (d0, d1, d2)]
    for i in range(limbs):
        q = ctx.primes[i]
        a0, a1, b0, b1 = ([int(v) for v in c[i]] for c in coef)
        want0 = negacyclic_mul(a0, b0, q)
        want1 = [(u + v) % q for u, v in zip(negacyclic_mul(a0, b1, q), negacyclic_mul(a1, b0, q))]
        want2 = negacyclic_mul(a1, b1, q)
        assert [int(v) for v in got[0][i]] == want0
        assert [int(v) for v in got[1][i]] == want1
        assert [int(v) for v in got[2][i]] == want2


def test_tensor_is_not_symmetric_in_the_wrong_way(chain):
    # swapping the roles of (a0, a1) and (b0, b1) keeps d0, d1, d2; swapping a0 with a1 does not
    ctx = _ctx(4, 2, 1, 2, chain=chain)
    rng = np.random.default_rng(3)
    v = [_rand_coeffs(ctx, rng, 2) for _ in range(4)]
    base = ctx.tensor(2, *v)
    swapped = ctx.tensor(2, v[2], v[3], v[0], v[1])
    for x, y in zip(base, swapped):
        assert np.array_equal(x, y)
    crossed = ctx.tensor(2, v[1], v[0], v[2], v[3])
    assert not np.array_equal(base[0], crossed[0])


@pytest.mark.parametrize("ell", [4, 3, 1])
def test_relinearize_keeps_the_decryption(ell, chain):
    log_n, L, K, alpha = 4, 4, 2, 2
    ctx = _ctx(log_n, L, K, alpha, chain=chain)
    rng = np.random.default_rng(100 + ell)
    n = ctx.n
    s = rng.integers(-1, 2, n).astype(np.int64)
    s2 = np.asarray(negacyclic_square_py([int(v) for v in s]), dtype=np.int64)
    beta = ctx.beta(L)
    a = np.stack([_rand_coeffs(ctx, rng, L + K) for _ in range(beta)])
    e = rng.integers(-3, 4, (beta, n)).astype(np.int64)
    rlk = ctx.make_ksk(s2, s, a, e)
    idx = list(range(ell))
    d = [ctx.ntt_fwd_limbs(_rand_coeffs(ctx, rng, ell), idx) for _ in range(3)]
    o0, o1 = ctx.relinearize(ell, d[0], d[1], d[2], rlk)
    primes = [ctx.primes[i] for i in range(ell)]
    Q = 1
    for p in primes:
        Q *= p
    cd = [ctx.ntt_inv_limbs(x, idx) for x in d]
    co = [ctx.ntt_inv_limbs(x, idx) for x in (o0, o1)]
    sl = [int(v) for v in s]
    s2l = [int(v) for v in s2]

    def ints(row):
        return [int(v) for v in row]

    diffs = []  # per limb: (d0 + d1 s + d2 s^2) - (out0 + out1 s) mod q_i
    for i in range(ell):
        q = primes[i]
        lhs = [(x + y + z) % q for x, y, z in zip(ints(cd[0][i]), negacyclic_mul(ints(cd[1][i]), sl, q),
                                                  negacyclic_mul(ints(cd[2][i]), s2l, q))]
        rhs = [(x + y) % q for x, y in zip(ints(co[0][i]), negacyclic_mul(ints(co[1][i]), sl, q))]
        diffs.append([(u - v) % q for u, v in zip(lhs, rhs)])
    for t in range(n):
        noise = centered(crt([diffs[i][t] for i in range(ell)], primes), Q)
        assert abs(noise) < 2**20, noise


def test_secret_square_schoolbook_against_ntt(chain):
    # the negacyclic square of a ternary secret, computed through the oracle's NTT over one prime,
    # equals the schoolbook integer square (its coefficients are far below q / 2)
    ctx = _ctx(6, 1, 1, 1, chain=chain)
    rng = np.random.default_rng(11)
    s = rng.integers(-1, 2, ctx.n).astype(np.int64)
    q = ctx.primes[0]
    sn = ctx.ntt_fwd_limbs(np.asarray([[int(v) % q for v in s]], dtype=np.uint64), [0])
    sq = ctx.ntt_inv_limbs(np.asarray([[int(x) * int(x) % q for x in sn[0]]], dtype=np.uint64), [0])[0]
    got = [centered(int(v), q) for v in sq]
    assert got == negacyclic_square_py([int(v) for v in s])


def test_weighted_sum_matches_big_integer_sums(chain):
    ctx = _ctx(4, 3, 1, 3, chain=chain)
    rng = np.random.default_rng(5)
    limbs, n, G = 3, 5, 2
    x = np.stack([_rand_coeffs(ctx, rng, limbs) for _ in range(n)])
    w = np.stack([np.stack([[int(rng.integers(0, ctx.primes[l])) for l in range(limbs)] for _ in range(n)])
                  for _ in range(G)]).astype(np.uint64)
    out = ctx.weighted_sum(limbs, x, w)
    for g in range(G):
        for l in range(limbs):
            q = ctx.primes[l]
            for k in range(ctx.n):
                want = sum(int(w[g, j, l]) * int(x[j, l, k]) for j in range(n)) % q
                assert int(out[g, l, k]) == want
