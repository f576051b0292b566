"""Feature-major RMSNorm on ciphertexts (llama3fhe/operators/norm/rmsnorm.py:203-250,572-960).

y[t, d] = gamma[d] * x[t, d] / sqrt(mean_d x[t, d]^2 + eps), with the inverse square root a
Chebyshev series fitted on an interval of the mean square (``coeffs = {"coefficients": c,
"fit_interval": (lo, hi)}``, the reference's coefficient dictionary).  In the feature-major layout
(slot d * tokens_per_cipher + t) the sum over the features of a token is the rotate-and-add tree
over strides tokens_per_cipher * 2^k (``_fold_feature_orbit``, ascending), which leaves the sum in
every feature slot of that token, so the polynomial's output multiplies x slot-wise with no
broadcast.  The reference packs the 128 mean squares into one slim ciphertext to evaluate the
polynomial once; here the polynomial runs on all input ciphertexts as one batch (each product a
batched key switch), which needs no masks or broadcast rotations.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass, field

import numpy as np

from . import fhe
from .context import Cipher, CKKSContext
from .layouts import FeatureMajorPrefillLayout
from .polynomial import chebyshev_coefficients, entry_coefficients, eval_chebyshev, series_from_entry

__all__ = ["FeatureMajorRMSNormResult", "rmsnorm_coefficients", "rmsnorm_fhe", "rmsnorm_numpy", "rmsnorm_rotations"]


@dataclass
class FeatureMajorRMSNormResult:
    outputs: tuple
    stage_seconds: dict = field(default_factory=dict)
    level_schedule: dict = field(default_factory=dict)


def rmsnorm_rotations(layout: FeatureMajorPrefillLayout) -> tuple:
    """The fold strides tokens_per_cipher * 2^k, k < log2(hidden_dim) (rmsnorm.py:132-144)."""

    t = layout.tokens_per_cipher
    return tuple(t << k for k in range(int(math.log2(layout.hidden_dim))))


def rmsnorm_coefficients(degree: int = 15, interval=(0.5, 2.0), eps: float = 1e-5) -> dict:
    """Chebyshev interpolant of 1 / sqrt(m + eps) on ``interval`` of the mean square m, as the
    reference's coefficient dictionary (its evaluator halves the constant term)."""

    series = chebyshev_coefficients(lambda m: 1.0 / np.sqrt(m + eps), degree, interval)
    return {"coefficients": entry_coefficients(series), "fit_interval": tuple(float(v) for v in interval),
            "eps": float(eps)}


def rmsnorm_numpy(x: np.ndarray, weight: np.ndarray | None, coeffs: dict) -> np.ndarray:
    """The same computation in float64 with the same polynomial (the decrypted-output oracle); a
    ``{"function": f}`` dictionary evaluates f(mean square) instead (exact mode)."""

    x = np.asarray(x, dtype=np.float64)
    m = np.mean(x * x, axis=1, keepdims=True)
    if "function" in coeffs:   # exact mode: the function the series approximates
        r = coeffs["function"](m)
    else:
        lo, hi = coeffs["fit_interval"]
        r = np.polynomial.chebyshev.chebval((2.0 * m - (lo + hi)) / (hi - lo), series_from_entry(coeffs))
    y = x * r
    return y if weight is None else y * np.asarray(weight, dtype=np.float64)[None, :]


def _fold(batch: Cipher, layout: FeatureMajorPrefillLayout, ctx: CKKSContext) -> Cipher:
    """Rotate-and-add over the feature orbit of every ciphertext of the batch: each step one
    batched rotation fused with the addition (the accumulator is the step's input)."""

    limbs = int(batch.state.cur_limbs)
    c0, c1 = batch.cv[0][:, :limbs], batch.cv[1][:, :limbs]
    for stride in rmsnorm_rotations(layout):
        g = ctx.galois_element(stride)
        n0, n1 = ctx.rotate_raw(c0, c1, limbs, g, ctx.key_for_galois(g), acc=(c0, c1))
        c0, c1 = n0, n1
    return batch.cipher_like([c0, c1])


def rmsnorm_fhe(input_ciphers, weight: np.ndarray | None = None, *, coeffs: dict,
                layout: FeatureMajorPrefillLayout, crypto_context) -> FeatureMajorRMSNormResult:
    """RMSNorm of feature-major ciphertexts (one level for the square, ``chebyshev_depth`` for the
    inverse square root, one for the product, one more with ``weight``).  Inputs share one level
    and scale; the outputs come back at one common level."""

    ctx = getattr(crypto_context, "context", crypto_context)
    cts = tuple(input_ciphers)
    if not cts:
        raise ValueError("RMSNorm needs at least one ciphertext")
    if int(layout.slots) != int(ctx.max_slots):
        raise ValueError("feature-major RMSNorm requires layout.slots == context.max_slots")
    times: dict = {}
    sched: dict = {}
    t0 = time.perf_counter()
    x = fhe.pack_cipher_batch(cts)
    sq = fhe.homo_mul_relin_rescale(x, x, ctx)
    times["square"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    s = _fold(sq, layout, ctx)
    times["fold"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    lo, hi = (float(v) for v in coeffs["fit_interval"])
    D = float(layout.hidden_dim)
    r = eval_chebyshev(s, series_from_entry(coeffs), ctx, interval=(D * lo, D * hi))
    times["rsqrt_polynomial"] = time.perf_counter() - t0
    sched["rsqrt_output_limbs"] = int(r.state.cur_limbs)
    t0 = time.perf_counter()
    xr = fhe.align_to(x, x.state.replace(cur_limbs=int(r.state.cur_limbs)), ctx)
    y = fhe.homo_mul_relin_rescale(xr, r, ctx)
    if weight is not None:
        w = np.asarray(weight, dtype=np.float64).reshape(-1)
        if w.shape != (int(layout.hidden_dim),):
            raise ValueError(f"RMSNorm gamma must have width {layout.hidden_dim}")
        row = layout.pack(np.tile(w[None, :], (int(layout.seq_len), 1)))[0]
        limbs = int(y.state.cur_limbs)
        pt = fhe.encode_plaintext(row, y.state.replace(scaling_factor=float(ctx.rescale_divisor_at(limbs))),
                                  ctx.max_slots, ctx)
        y = fhe.rescale(fhe.homo_mul_pt(y, pt, ctx), ctx)
    times["scale"] = time.perf_counter() - t0
    sched["output_limbs"] = int(y.state.cur_limbs)
    outs = tuple(fhe.cipher_batch_item(y, i) for i in range(y.batch_size))
    return FeatureMajorRMSNormResult(outputs=outs, stage_seconds=times, level_schedule=sched)
