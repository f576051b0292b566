"""Pins of the oracle's CKKS encoder and BSGS diagonal packer.

Encoder: equal to the canonical-embedding formula computed by a different method (length-2N
NumPy FFT of the rotation-group scatter, holmes_amd.encoding) up to rounding ties; decode
round trip.  Packer: the diagonal method identity sum_g rot(sum_b row(g,b) * rot(x, b lanes),
g B lanes) = W x on slot vectors (rotations as np.roll), which is what the packing is for.
"""

import numpy as np
import pytest

from holmes_amd import encoding
from oracle import oracle as O


def test_encode_twiddles_are_the_rotation_group_roots():
    log_n = 6
    n, M = 1 << (log_n - 1), 1 << (log_n + 1)
    re, im = O.encode_twiddles(log_n)
    h = 1
    while h < n:
        lenq = 8 * h
        for j in range(h):
            idx = (lenq - pow(5, j, M) % lenq) * (M // lenq)
            w = np.exp(2j * np.pi * idx / M)
            assert abs(complex(re[h - 1 + j], im[h - 1 + j]) - w) < 1e-15
        h *= 2


@pytest.mark.parametrize("scale", [2.0**40, 1125899906826241.0])
def test_encode_matches_fft_canonical_embedding(scale):
    ps = O.gen_primes(16, 50, 3)
    ctx = O.OracleContext(16, 2, 1, 2, ps)
    rng = np.random.default_rng(3)
    z = rng.normal(scale=0.5, size=1 << 15)
    res, ok = ctx.encode_real(z, scale, [0, 1, 2], ntt=False)
    assert ok
    m = encoding.encode(z, scale, 16)
    q0 = ps[0]
    got = res[0].astype(object)
    got = np.where(got > q0 // 2, got - q0, got).astype(np.int64)
    diff = np.abs(got - m)
    # two FP evaluations of the same real coefficients: they may round differently only where the
    # value lies within the FP error (~2^-53 |m| log N) of a half-integer
    assert diff.max() <= 1 and np.count_nonzero(diff) <= max(8, diff.size // 100)
    # all limbs hold the same integer
    for l in (1, 2):
        q = ps[l]
        g = res[l].astype(object)
        assert np.array_equal(np.where(g > q // 2, g - q, g).astype(np.int64), got)
    back = encoding.decode(got.astype(np.float64), scale, 16)
    assert np.max(np.abs(back.real - z)) < 1e-9
    # NTT flag = encode then forward NTT of each limb
    res_ntt, _ = ctx.encode_real(z, scale, [0, 1, 2], ntt=True)
    assert np.array_equal(res_ntt, ctx.ntt_fwd_limbs(res, [0, 1, 2]))


def test_stage1_is_the_encoders_rounding_input():
    """encode_stage1 (the encode sidecar's stage-2 input, interleaved Re / Im) rounded half away
    from zero and reduced gives encode_real's coefficient-domain residues: coefficient k < n from
    Re w_k, k >= n from Im w_(k-n) (bench/cmp/kernels/holmes_encode.cu:108-111); and it is the
    canonical embedding's inverse, so it matches the independent NumPy encoder before rounding."""

    ps = O.gen_primes(16, 59, 2)
    ctx = O.OracleContext(16, 2, 0, 1, ps)
    rng = np.random.default_rng(8)
    z = rng.normal(size=1 << 15)
    scale = 2.0**45
    w = ctx.encode_stage1(z)
    x = w * scale
    r = np.trunc(x)
    d = x - r
    coef = r + (d >= 0.5) - (d <= -0.5)
    coef = np.array([int(c) for c in np.concatenate([coef[0::2], coef[1::2]])], dtype=object)
    res, ok = ctx.encode_real(z, scale, [0, 1], ntt=False)
    assert ok
    for l, q in enumerate(ps):
        assert np.array_equal(res[l].astype(object), coef % q)
    m = encoding.encode(z, scale, 16)  # the NumPy encoder, independently rounded
    assert np.max(np.abs(np.asarray(m, dtype=np.float64) - coef.astype(np.float64))) <= 1.0


def test_encode_reports_overflow():
    """The cap is |coefficient| < 2^61 (MAX_ENCODED_BITS, llama3fhe/operators/attention/prefill/
    softmax.py:559).  A constant slot vector c encodes exactly to the coefficient c * scale at
    position 0 and zeros elsewhere (every butterfly difference is 0), so the boundary is sharp."""
    primes = O.gen_primes(16, 50, 3)
    ctx = O.OracleContext(16, 2, 1, 2, primes)
    _, ok = ctx.encode_real(np.full(1 << 15, 2.0**21), 2.0**40, [0])
    assert not ok
    below = 2.0**21 - 2.0**-32  # the largest double below 2^21
    res, ok = ctx.encode_real(np.full(1 << 15, below), 2.0**40, [0, 1], ntt=False)
    assert ok
    dc = 2**61 - 2**8
    assert [int(v) for v in res[:, 0]] == [dc % q for q in primes[:2]]
    assert not np.any(res[:, 1:])


def _bsgs_slots(rows, x, D, lanes, B, G, giant_base=0):
    """sum_g rot(sum_b rows[g,b] * rot(x, b lanes), (giant_base + g) B lanes) with rot = left roll."""

    acc = np.zeros_like(x)
    for g in range(G):
        inner = np.zeros_like(x)
        for b in range(B):
            inner += rows[g * B + b] * np.roll(x, -b * lanes)
        acc += np.roll(inner, -(giant_base + g) * B * lanes)
    return acc


@pytest.mark.parametrize("D,lanes,B", [(64, 8, 16), (32, 4, 8)])
def test_diagonal_packing_realises_matvec(D, lanes, B):
    slots = D * lanes * 2  # features repeat (f mod D), as on a full ring
    rng = np.random.default_rng(D)
    W = rng.normal(size=(D, D))
    X = rng.normal(size=(D, lanes))  # feature-major: slot s holds X[s // lanes mod D, s % lanes]
    s = np.arange(slots)
    x = X[(s // lanes) % D, s % lanes]
    G = D // B
    rows = O.pack_diagonals(W, lanes, 0, B, 0, G, slots)
    y = _bsgs_slots(rows, x, D, lanes, B, G)
    want = (W @ X)[(s // lanes) % D, s % lanes]
    assert np.max(np.abs(y - want)) < 1e-9
    # chunked: two chunks of G/2 giants, second aligned by its giant base, give the same sum
    half = G // 2
    r0 = O.pack_diagonals(W, lanes, 0, B, 0, half, slots)
    r1 = O.pack_diagonals(W, lanes, 0, B, half, half, slots)
    y2 = _bsgs_slots(r0, x, D, lanes, B, half) + _bsgs_slots(r1, x, D, lanes, B, half, giant_base=half)
    assert np.max(np.abs(y2 - want)) < 1e-9
