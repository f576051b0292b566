"""The coefficient dictionaries follow the reference's convention: its evaluator
(llama3fhe/approx/chebyshev.py:136-163) computes c_0 / 2 + sum_(j>=1) c_j T_j by the three-term
recurrence.  That evaluator, restated here, must reproduce the fitted function from this build's
dictionary, and the numpy-convention series this build evaluates must agree with it."""

import numpy as np

from holmes_amd.norm import rmsnorm_coefficients, rmsnorm_numpy
from holmes_amd.polynomial import entry_coefficients, series_from_entry


def _reference_eval(x, coeffs, a, b):
    y = (2.0 * np.asarray(x) - (a + b)) / (b - a)
    t_prev, t_cur = np.ones_like(y), y
    acc = np.full_like(y, coeffs[0] / 2.0) + coeffs[1] * t_cur
    for c in coeffs[2:]:
        t_prev, t_cur = t_cur, 2.0 * y * t_cur - t_prev
        acc += c * t_cur
    return acc


def test_rmsnorm_entry_matches_reference_evaluator():
    e = rmsnorm_coefficients(15, (0.5, 2.0), 1e-5)
    m = np.linspace(0.5, 2.0, 101)
    ref = _reference_eval(m, e["coefficients"], 0.5, 2.0)
    assert np.max(np.abs(ref - 1.0 / np.sqrt(m + 1e-5))) < 1e-4
    ours = np.polynomial.chebyshev.chebval((2 * m - 2.5) / 1.5, series_from_entry(e))
    assert np.allclose(ours, ref, atol=1e-13)
    assert np.allclose(entry_coefficients(series_from_entry(e)), e["coefficients"])


def test_rmsnorm_numpy_uses_the_entry_convention():
    rng = np.random.default_rng(0)
    x = rng.normal(size=(3, 64))
    e = rmsnorm_coefficients(15, (0.5, 2.0), 1e-5)
    want = x * _reference_eval(np.mean(x * x, axis=1, keepdims=True), e["coefficients"], 0.5, 2.0)
    assert np.allclose(rmsnorm_numpy(x, None, e), want, atol=1e-12)
