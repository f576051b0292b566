"""CKKS canonical-embedding encode / decode on the client (NumPy, float64).

Slot j of a degree-N message polynomial m is m(zeta_j) / scale with zeta_j = exp(2 pi i g_j / 2N),
g_j = 5^j mod 2N (the rotation group), j < N/2.  Rotation by r slots is then the automorphism
X -> X^(5^r), matching rotate(v, r)[s] = v[(s + r) mod slots] of
llama3fhe/layouts/shifted_lane.py:24-37, and conjugation is X -> X^(2N - 1)
(llama3fhe/operators/linear/complex.py:63-67).

Encoding solves m(zeta_j) = scale * z_j, m(conj zeta_j) = conj(scale * z_j) for real m:
    m_k = (2 / N) Re(sum_j scale z_j zeta_j^-k) = (2 scale / N) Re(FFT_2N(w))[k],  w[g_j] = z_j,
then rounds to the nearest integer (EasyFHE rounds with llround; bench/cmp/kernels/holmes_encode.cu:
108-111).  Sparse packing with n < N/2 slots places the vector at every (N/2n)-th slot of the full
embedding (the standard replicated layout), so decoding n slots reads slots 0..n-1.
"""

from __future__ import annotations

import numpy as np

MAX_ENCODED_BITS = 61  # |value * scale| must stay below 2^61 (llama3fhe softmax.py:559 cap)

_ROT_CACHE: dict[int, np.ndarray] = {}


def rotation_group(log_n: int) -> np.ndarray:
    """g_j = 5^j mod 2N for j < N/2."""

    g = _ROT_CACHE.get(log_n)
    if g is None:
        n = 1 << log_n
        two_n = 2 * n
        g = np.empty(n // 2, dtype=np.int64)
        v = 1
        for j in range(n // 2):
            g[j] = v
            v = v * 5 % two_n
        _ROT_CACHE[log_n] = g
    return g


def _full_slots(values: np.ndarray, slots: int, n: int) -> np.ndarray:
    half = n // 2
    z = np.zeros(half, dtype=np.complex128)
    v = np.asarray(values).reshape(-1).astype(np.complex128)
    if v.size > slots:
        raise ValueError(f"{v.size} values do not fit {slots} slots")
    vec = np.zeros(slots, dtype=np.complex128)
    vec[: v.size] = v
    if slots == half:
        return vec
    if half % slots:
        raise ValueError("slots must divide N/2")
    # sparse packing: the n-slot vector repeats N/(2n) times across the full embedding
    return np.tile(vec, half // slots)


def encode_real_coeffs(values, scale: float, log_n: int, slots: int | None = None) -> np.ndarray:
    """Real coefficients m_k * 1 (float64, not yet rounded) of the encoding of ``values``."""

    n = 1 << log_n
    slots = n // 2 if slots is None else int(slots)
    z = _full_slots(values, slots, n)
    w = np.zeros(2 * n, dtype=np.complex128)
    w[rotation_group(log_n)] = z
    m = np.fft.fft(w)[:n].real * (2.0 / n)
    return m * float(scale)


def encode(values, scale: float, log_n: int, slots: int | None = None) -> np.ndarray:
    """Rounded integer coefficients (int64) of the encoding; raises past the 2^61 cap."""

    m = np.rint(encode_real_coeffs(values, scale, log_n, slots))
    if m.size and float(np.max(np.abs(m))) >= float(2**MAX_ENCODED_BITS):
        raise ValueError("encoded value exceeds 2^61; lower the scale or the input range")
    return m.astype(np.int64)


def decode(coeffs, scale: float, log_n: int, slots: int | None = None) -> np.ndarray:
    """Complex slots of a real coefficient vector (float64 or int) divided by ``scale``."""

    n = 1 << log_n
    slots = n // 2 if slots is None else int(slots)
    m = np.zeros(2 * n, dtype=np.float64)
    m[:n] = np.asarray(coeffs, dtype=np.float64)
    ev = np.fft.ifft(m) * (2 * n)
    z = ev[rotation_group(log_n)] / float(scale)
    return z[:slots]


__all__ = ["encode", "encode_real_coeffs", "decode", "rotation_group", "MAX_ENCODED_BITS"]
