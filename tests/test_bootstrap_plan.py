"""CPU pins of the bootstrap's host plan (no GPU).

* The butterfly layers factor the decoder: U0 w = L_1 ... L_logn (bit-reversed w), U0 the
  slot map of the host decoder (holmes_amd.encoding.decode, an FFT evaluation at the 5^j-th
  roots), and the inverse layers undo it; a wrong twiddle, block size or sign fails.
* Merged stages equal their layers applied one by one, and the BSGS rows (pre-rotated diagonals,
  then giant rotations) equal the merged stage, for both directions at several budgets.
* The rotation list of ``requirements`` holds every baby and giant rotation the stages use.
* The Chebyshev division identity, the canonical-scale recursion, and the EvalMod interpolant
  against sin(2 pi t) through the double angles.
* An end-to-end numeric run of the whole pipeline on slot values (no encryption): coefficients
  with a q_0 I overflow, CoeffToSlot, the real / imaginary split, EvalMod, SlotToCoeff, the
  integer 2^bits, with the program's own constants; it must return the input slots.
"""

import math

import numpy as np
import pytest

from holmes_amd import bootstrap as B
from holmes_amd import encoding


def _apply(diags, x):
    n = x.shape[-1]
    out = np.zeros_like(x)
    for d, v in diags.items():
        out += v * np.roll(x, -(d % n))
    return out


def _rot(x, r):
    return np.roll(x, -(int(r) % x.shape[-1]))


def _bsgs(st, x):
    n = x.shape[-1]
    rows = B.stage_rows(st, n)
    babies = [_rot(x, k1 * st.h_min) for k1 in range(st.n1)]
    out = np.zeros_like(x)
    for gi, k2 in enumerate(st.giants):
        inner = sum(rows[gi * st.n1 + k1] * babies[k1] for k1 in range(st.n1))
        out += _rot(inner, k2 * st.n1 * st.h_min)
    return out


def _slots_of(coeffs, log_n):
    return encoding.decode(coeffs, 1.0, log_n)


@pytest.mark.parametrize("log_n", [4, 6, 9])
def test_butterflies_factor_the_decoder(log_n):
    rng = np.random.default_rng(log_n)
    N = 1 << log_n
    n = N // 2
    c = rng.normal(size=N)
    w = c[:n] + 1j * c[n:]
    want = _slots_of(c, log_n)
    fwd = B.special_fft_layers(log_n - 1)
    y = B.bit_reverse_order(w)
    for t in range(log_n - 1, 0, -1):     # L_logn first, L_1 last
        y = _apply(fwd[t - 1], y)
    assert np.allclose(y, want, atol=1e-9 * n)
    inv = B.special_fft_layers(log_n - 1, inverse=True)
    z = want.copy()
    for t in range(1, log_n):             # L_1^-1 first
        z = _apply(inv[t - 1], z)
    assert np.allclose(z, B.bit_reverse_order(w), atol=1e-9)


def test_butterflies_reject_a_wrong_twiddle():
    # the pin above is sensitive: conjugating one layer's twiddles breaks the factorisation
    log_n = 6
    rng = np.random.default_rng(1)
    c = rng.normal(size=1 << log_n)
    n = (1 << log_n) // 2
    w = c[:n] + 1j * c[n:]
    fwd = B.special_fft_layers(log_n - 1)
    bad = {d: np.conj(v) for d, v in fwd[2].items()}
    y = B.bit_reverse_order(w)
    for t in range(log_n - 1, 0, -1):
        y = _apply(bad if t == 3 else fwd[t - 1], y)
    assert not np.allclose(y, _slots_of(c, log_n), atol=1e-6)


@pytest.mark.parametrize("budget", [1, 2, 3, 4])
@pytest.mark.parametrize("inverse", [True, False])
def test_merged_stages_and_bsgs_rows(budget, inverse):
    log_slots = 8
    n = 1 << log_slots
    rng = np.random.default_rng(budget + 10 * inverse)
    x = rng.normal(size=n) + 1j * rng.normal(size=n)
    layers = B.special_fft_layers(log_slots, inverse=inverse)
    stages = B.plan_stages(log_slots, budget, inverse, 0.75)
    seq = x.copy()
    got = x.copy()
    order = []
    for i, st in enumerate(stages):
        for t in st.layers:
            seq = _apply(layers[t - 1], seq)
            order.append(t)
        if i == 0:
            seq = seq * 0.75
        assert np.allclose(_apply({(k * st.h_min) % n: v for k, v in st.diags.items()}, got), seq, atol=1e-9)
        got = _bsgs(st, got)
        assert np.allclose(got, seq, atol=1e-9)
        _, _, kmax = B._bsgs_shape(st.layers, n)
        assert max(abs(k) for k in st.diags) <= kmax
    assert sorted(order) == list(range(1, log_slots + 1))
    assert order == (list(range(1, log_slots + 1)) if inverse else list(range(log_slots, 0, -1)))


def test_requirements_cover_every_stage_rotation():
    spec = B.BootstrapSpec(log_slots=9, level_budget=(3, 2), cheb_degree=32)
    req = B.requirements(spec, 10)
    n = 1 << 9
    rots = set(req.rotations)
    assert 4 * n - 1 in rots  # conjugation
    for st in B.plan_stages(9, 3, True, 1.0) + B.plan_stages(9, 2, False, 1.0):
        for k1 in range(1, st.n1):
            assert (k1 * st.h_min) % n in rots
        for k2 in st.giants:
            if k2:
                assert (k2 * st.n1 * st.h_min) % n in rots
    assert req.depth == 3 + 2 + B.evalmod_levels(spec, 40, [2] * 41)


def test_spec_validation_and_sparse_rotations():
    for bad in (B.BootstrapSpec(log_slots=0), B.BootstrapSpec(log_slots=16), B.BootstrapSpec(mode="slots_first"),
                B.BootstrapSpec(log_slots=2, level_budget=(3, 2))):
        with pytest.raises(ValueError):
            B.requirements(bad, 16)
    sparse = B.BootstrapSpec(log_slots=12, level_budget=(2, 2))
    assert sparse.trace_rotations(16) == (4096, 8192, 16384)
    rots = set(B.requirements(sparse, 16).rotations)
    assert {4096, 8192, 16384, (1 << 17) - 1} <= rots and all(r < 4096 for r in rots - {4096, 8192, 16384, (1 << 17) - 1})
    assert B.BootstrapSpec().trace_rotations(16) == ()


def test_chebyshev_division_identity():
    rng = np.random.default_rng(3)
    C = np.polynomial.chebyshev
    for M, ln in ((8, 13), (16, 32), (32, 49)):
        c = rng.normal(size=ln)
        q, r = B.chebyshev_divide(c, M)
        u = np.linspace(-1, 1, 101)
        TM = C.chebval(u, np.eye(M + 1)[M])
        assert np.allclose(C.chebval(u, c), C.chebval(u, q) * TM + C.chebval(u, r), atol=1e-12)
        assert len(r) <= M


def test_canonical_scales_close_under_products():
    primes = [2**50 - 2**26 * k + 1 for k in range(1, 12)]
    sc = B.canonical_scales(primes, 10, 2.0**50)
    for l in range(2, 11):
        assert sc[l - 1] == pytest.approx(sc[l] * sc[l] / primes[l - 1], rel=1e-15)
    assert abs(math.log2(sc[1]) - 50) < 0.01


def test_evalmod_interpolant_gives_sine():
    spec = B.BootstrapSpec()
    c = B.evalmod_coefficients(spec)
    Kp = spec.mod_bound + 1
    t = np.concatenate([np.linspace(-Kp + 0.5, Kp - 0.5, 4001), np.arange(-spec.mod_bound, spec.mod_bound + 1) + 1e-4])
    y = np.polynomial.chebyshev.chebval(t / Kp, c)
    for _ in range(spec.double_angle):
        y = 2 * y * y - 1
    assert np.max(np.abs(y - np.sin(2 * np.pi * t))) < 2.0**-30


def test_evalmod_levels_match_schedule():
    spec = B.BootstrapSpec()
    # baby basis T_1..T_8 (3), giants T_16 (4), T_32 (5), the top product (6), 3 double angles
    assert B.evalmod_levels(spec, 21, [2] * 30) == 9


def _simulate(prog, v, q0, I, S_in, log_n, bits):
    """The bootstrap on slot values: what the GPU path computes, less the encryption noise.  A
    sparse program (v of 2^log_slots < N / 2 slots) traces the raised slot vector onto its period
    and then works on one period, as the GPU's tiled diagonals and rotations modulo n do."""

    S = prog.nominal_scale
    n = len(v)
    m = encoding.encode_real_coeffs(v, S_in * 2.0**-bits, log_n, n)  # message at one limb
    M = m + float(q0) * I                                             # after ModRaise
    z = encoding.decode(M, S, log_n)
    for r in prog.spec.trace_rotations(log_n):
        z = z + _rot(z, r)
    z = z[:n]
    for st in prog.cts:
        z = _bsgs(st, z)
    z = z * prog.cts_rho ** len(prog.cts)
    R, J = 2 * z.real, 2 * z.imag                                     # x + conj(x), -i (x - conj(x))
    ys = []
    for u in (R, J):
        assert np.max(np.abs(u)) <= 1.0
        y = np.polynomial.chebyshev.chebval(u, prog.cheb)
        for _ in range(prog.spec.double_angle):
            y = 2 * y * y - 1
        ys.append(y)
    w = ys[0] + 1j * ys[1]
    for st in prog.stc:
        w = _bsgs(st, w)
    w = w * prog.stc_rho ** len(prog.stc) * float(1 << bits)
    return w * prog.evalmod_out_scale / S_in                          # decryption / S_in


@pytest.mark.parametrize("seed", [0, 1])
def test_numeric_pipeline_returns_the_input(seed):
    log_n = 10
    spec = B.BootstrapSpec(log_slots=log_n - 1, level_budget=(3, 3))
    rng = np.random.default_rng(seed)
    primes = [2**50 - 2**27 * k + 1 for k in range(1, 31)]
    prog = B.plan_program(spec, primes, 2.0**50, 30, log_n)
    n = 1 << (log_n - 1)
    v = (rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)) / math.sqrt(2)
    I = rng.integers(-spec.mod_bound + 1, spec.mod_bound, 1 << log_n).astype(np.float64)
    S_in = 2.0**50
    bits = int(round(math.log2(S_in / primes[0]))) + spec.message_ratio_bits
    got = _simulate(prog, v, primes[0], I, S_in, log_n, bits)
    err = np.max(np.abs(got - v))
    assert err < 2.0**-20, err


def test_numeric_pipeline_catches_a_wrong_constant():
    log_n = 8
    spec = B.BootstrapSpec(log_slots=log_n - 1, level_budget=(2, 2))
    primes = [2**50 - 2**27 * k + 1 for k in range(1, 31)]
    prog = B.plan_program(spec, primes, 2.0**50, 30, log_n)
    rng = np.random.default_rng(5)
    n = 1 << (log_n - 1)
    v = rng.uniform(-1, 1, n) + 0j
    I = rng.integers(-5, 6, 1 << log_n).astype(np.float64)
    good = _simulate(prog, v, primes[0], I, 2.0**50, log_n, 12)
    assert np.max(np.abs(good - v)) < 2.0**-20
    prog.stc[0].diags = {k: d * (1 + 2.0**-10) for k, d in prog.stc[0].diags.items()}
    bad = _simulate(prog, v, primes[0], I, 2.0**50, log_n, 12)
    assert np.max(np.abs(bad - v)) > 2.0**-12


@pytest.mark.parametrize("log_slots,budget", [(6, (2, 2)), (3, (2, 3)), (1, (1, 1))])
def test_numeric_sparse_pipeline_returns_the_input(log_slots, budget):
    """Sparse slots: the message is periodic with period n = 2^log_slots; q_0 I is a full-ring
    polynomial (only the trace makes it sparse), and the pipeline must return the n slots."""

    log_n = 10
    spec = B.BootstrapSpec(log_slots=log_slots, level_budget=budget)
    primes = [2**50 - 2**27 * k + 1 for k in range(1, 31)]
    prog = B.plan_program(spec, primes, 2.0**50, 30, log_n)
    rng = np.random.default_rng(log_slots)
    n = 1 << log_slots
    v = (rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)) / math.sqrt(2)
    I = rng.integers(-spec.mod_bound + 1, spec.mod_bound, 1 << log_n).astype(np.float64)
    bits = int(round(math.log2(2.0**50 / primes[0]))) + spec.message_ratio_bits + spec.sparse_extra_bits(log_n)
    got = _simulate(prog, v, primes[0], I, 2.0**50, log_n, bits)
    assert np.max(np.abs(got - v)) < 2.0**-20
    # without the extra scale-down bits the sine's cubic error grows with R = N / 2n (the 2n
    # coefficients of a sparse message are sqrt(R) times those of a full one of the same slot size)
    R = 1 << (log_n - 1 - log_slots)
    plain = _simulate(prog, v, primes[0], I, 2.0**50, log_n, bits - spec.sparse_extra_bits(log_n))
    if R >= 64:
        assert np.max(np.abs(plain - v)) > 2.0**-20
    # without the trace's gain in the constant the result is off by R = N / 2n
    prog.cts_rho *= (1 << (log_n - 1 - log_slots)) ** (1.0 / len(prog.cts))
    try:
        bad = _simulate(prog, v, primes[0], I, 2.0**50, log_n, bits)
    except AssertionError:
        return  # the EvalMod input left [-1, 1]: caught
    assert np.max(np.abs(bad - v)) > 2.0**-8


def test_raise_target_is_the_fewest_limbs_that_leave_the_output():
    """raise_for_output: the program raised to the returned limb count leaves the requested limbs
    (plus one for the two-pass correction), one limb fewer does not, and the lower-raised program
    still returns its input on the numeric pipeline (its scales come from the shorter chain)."""

    log_n = 10
    spec = B.BootstrapSpec(log_slots=log_n - 1, level_budget=(3, 3))
    primes = [2**50 - 2**27 * k + 1 for k in range(1, 31)]
    top = B.plan_program(spec, primes, 2.0**50, 30, log_n).output_limbs
    for need in (3, 8, top - 1):
        r = B.raise_for_output(spec, primes, need, log_n=log_n)
        assert B.plan_program(spec, primes, 2.0**50, r, log_n).output_limbs >= need + 1
        assert B.plan_program(spec, primes, 2.0**50, r - 1, log_n).output_limbs < need + 1
        assert B.raise_for_output(spec, primes, need, two_pass=False, log_n=log_n) == r - 1
    assert B.raise_for_output(spec, primes, top + 5, log_n=log_n) == 30
    r = B.raise_for_output(spec, primes, 4, log_n=log_n)
    prog = B.plan_program(spec, primes, 2.0**50, r, log_n)
    rng = np.random.default_rng(9)
    n = 1 << (log_n - 1)
    v = (rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)) / math.sqrt(2)
    I = rng.integers(-spec.mod_bound + 1, spec.mod_bound, 1 << log_n).astype(np.float64)
    bits = int(round(math.log2(2.0**50 / primes[0]))) + spec.message_ratio_bits
    assert np.max(np.abs(_simulate(prog, v, primes[0], I, 2.0**50, log_n, bits) - v)) < 2.0**-20
    for bad in (-1, 1):
        with pytest.raises(ValueError, match="raise_limbs"):
            B.BootstrapSpec(raise_limbs=bad).validate(16)
