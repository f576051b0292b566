"""Pins of the oracle's prime chain, root choice, NTT / INTT and automorphisms.

Each check comes from mathematics, not from the oracle's formulas: primality by an independent
Miller-Rabin base set, psi by its order, the NTT by the O(N^2) evaluation sum, the convolution
theorem against schoolbook negacyclic products, automorphisms by polynomial substitution.  Every
pin runs on 50-bit primes and on the reference's 59/60-bit widths (assets/feature_major.json:9-11).
"""

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import bitrev, is_prime_py, negacyclic_mul, small_primes


@pytest.mark.parametrize("log_n,bits", [(4, 30), (10, 50), (16, 50), (16, 59), (16, 60)])
def test_prime_chain_rule(log_n, bits):
    ps = O.gen_primes(log_n, bits, 6)
    assert ps == small_primes(log_n, bits, 6)
    step = 2 << log_n
    for p in ps:
        assert p % step == 1 and p < (1 << bits) and is_prime_py(p)
    # nothing skipped: every candidate between consecutive chain primes is composite
    for hi, lo in zip(ps, ps[1:]):
        for c in range(lo + step, hi, step):
            assert not is_prime_py(c)
    # exclusion list is honoured
    assert O.gen_primes(log_n, bits, 3, exclude=ps[:2]) == ps[2:5]


@pytest.mark.parametrize("bits", [50, 59, 60])
@pytest.mark.parametrize("log_n", [3, 10, 16])
def test_psi_is_primitive_2n_root(log_n, bits):
    for q in O.gen_primes(log_n, bits, 3):
        psi = O.find_psi(q, log_n)
        n = 1 << log_n
        assert pow(psi, n, q) == q - 1  # psi^N = -1 => order exactly 2N
        # smallest quadratic non-residue rule
        g = next(g for g in range(2, 1000) if pow(g, (q - 1) // 2, q) == q - 1)
        assert psi == pow(g, (q - 1) // (2 * n), q)


@pytest.mark.parametrize("bits", [50, 59, 60])
@pytest.mark.parametrize("log_n", [3, 5, 8, 10])
def test_ntt_equals_brute_force_evaluation(log_n, bits):
    n = 1 << log_n
    q = O.gen_primes(log_n, bits, 1)[0]
    psi = O.find_psi(q, log_n)
    fwd, inv = O.make_tables(q, psi, log_n)
    assert all(int(fwd[k]) == pow(psi, bitrev(k, log_n), q) for k in range(n))
    rng = np.random.default_rng(7)
    a = rng.integers(0, q, n, dtype=np.uint64)
    out = O.ntt_fwd(a, log_n, q, fwd)
    al = [int(v) for v in a]
    for k in range(n):
        e = 2 * bitrev(k, log_n) + 1
        w = pow(psi, e, q)
        assert int(out[k]) == sum(al[j] * pow(w, j, q) for j in range(n)) % q
    assert np.array_equal(O.ntt_inv(out, log_n, q, inv), a)


@pytest.mark.parametrize("bits", [50, 59, 60])
def test_ntt_edge_values(bits):
    log_n = 16
    n = 1 << log_n
    q = O.gen_primes(log_n, bits, 1)[0]
    fwd, inv = O.make_tables(q, O.find_psi(q, log_n), log_n)
    for a in (np.zeros(n, np.uint64), np.full(n, q - 1, np.uint64)):
        assert np.array_equal(O.ntt_inv(O.ntt_fwd(a, log_n, q, fwd), log_n, q, inv), a)
    # delta at 0 transforms to all ones
    d = np.zeros(n, np.uint64)
    d[0] = 1
    assert np.all(O.ntt_fwd(d, log_n, q, fwd) == 1)


@pytest.mark.parametrize("bits", [50, 59, 60])
@pytest.mark.parametrize("log_n", [4, 7])
def test_convolution_theorem(log_n, bits):
    n = 1 << log_n
    q = O.gen_primes(log_n, bits, 1)[0]
    fwd, inv = O.make_tables(q, O.find_psi(q, log_n), log_n)
    rng = np.random.default_rng(11)
    a = rng.integers(0, q, n, dtype=np.uint64)
    b = rng.integers(0, q, n, dtype=np.uint64)
    fa, fb = O.ntt_fwd(a, log_n, q, fwd), O.ntt_fwd(b, log_n, q, fwd)
    prod = np.array([int(x) * int(y) % q for x, y in zip(fa, fb)], dtype=np.uint64)
    c = O.ntt_inv(prod, log_n, q, inv)
    assert [int(v) for v in c] == negacyclic_mul([int(v) for v in a], [int(v) for v in b], q)


@pytest.mark.parametrize("bits", [50, 60])
@pytest.mark.parametrize("g", [5, 25, 5**7 % 256, 255])
def test_automorphism_coeff_and_ntt(g, bits):
    log_n = 7
    n = 1 << log_n
    q = O.gen_primes(log_n, bits, 1)[0]
    fwd, inv = O.make_tables(q, O.find_psi(q, log_n), log_n)
    rng = np.random.default_rng(g)
    a = rng.integers(0, q, n, dtype=np.uint64)
    # coefficient domain: a(X) -> a(X^g) by direct substitution
    want = [0] * n
    for i in range(n):
        e = i * g % (2 * n)
        if e < n:
            want[e] = (want[e] + int(a[i])) % q
        else:
            want[e - n] = (want[e - n] - int(a[i])) % q
    got = O.automorph_coeff(a, log_n, g, q)
    assert [int(v) for v in got] == want
    # NTT domain permutation == INTT -> substitute -> NTT
    fa = O.ntt_fwd(a, log_n, q, fwd)
    assert np.array_equal(O.automorph_ntt(fa, log_n, g), O.ntt_fwd(got, log_n, q, fwd))
