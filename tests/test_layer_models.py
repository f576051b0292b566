"""Pins of the float64 layer models the encrypted layers are checked against
(holmes_amd.prefill.prefill_layer_numpy, holmes_amd.decode.decode_layer_numpy,
holmes_amd.mlp.mlp_block_numpy), without the reference's code:

* closed form: with the functions themselves in place of every series (exact mode), each model is
  a textbook Llama-3-8B layer -- RMSNorm, RoPE at theta = 500000 (rotate-half, with the reference's
  float32 angle rounding, llama3fhe/approx/attention.py:23-38), causal grouped-query softmax
  attention, SwiGLU -- written here from the architecture, to 1e-12;
* the known answers of the reference's layer-math tests, restated for these models:
  the causal prefill's last query row equals the one-query decode computation over the same keys
  (tests/test_poly_alg2_layer.py:23-53); with an identity RMSNorm the layer equals the manual
  layer built from its own series (tests/test_poly_layer.py:23-85); the MLP block equals a direct
  SwiGLU, and folding the RMSNorm gamma into the gate / up weights -- what the encrypted block
  does -- changes nothing (tests/test_mlp.py:51-112).
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from holmes_amd import decode as Dm
from holmes_amd import prefill as P
from holmes_amd.mlp import MLPBlockSpec, mlp_block_numpy, silu_coefficients

THETA = 500000.0


def _rope(x: np.ndarray, heads: int, positions: np.ndarray) -> np.ndarray:
    """Rotate-half RoPE, head dim 128: x cos + rotate_half(x) sin with float32 angles."""

    n = x.shape[0]
    inv = (1.0 / (np.float32(THETA) ** (np.arange(0, 128, 2, dtype=np.float32) / np.float32(128)))).astype(np.float32)
    ang = (positions.astype(np.float32)[:, None] * inv[None, :]).astype(np.float32)
    ang = np.concatenate([ang, ang], axis=1)
    cos, sin = np.cos(ang).astype(np.float64), np.sin(ang).astype(np.float64)
    h = x.reshape(n, heads, 128)
    rot = np.concatenate([-h[..., 64:], h[..., :64]], axis=-1)
    return (h * cos[:, None, :] + rot * sin[:, None, :]).reshape(n, -1)


def _rms(v: np.ndarray, gamma: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    return v / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + eps) * gamma


def _silu(v):
    return v / (1.0 + np.exp(-v))


def _attention(q, k, v, q_pos, k_pos):
    """Causal GQA softmax attention: query head h reads KV head h // 4; key j visible to query i
    when k_pos[j] <= q_pos[i]."""

    nq = q.shape[0]
    out = np.zeros((nq, 32 * 128))
    for h in range(32):
        g = h // 4
        qh = q[:, 128 * h:128 * (h + 1)]
        kh = k[:, 128 * g:128 * (g + 1)]
        vh = v[:, 128 * g:128 * (g + 1)]
        s = qh @ kh.T / math.sqrt(128.0)
        s = np.where(k_pos[None, :] <= q_pos[:, None], s, -np.inf)
        s = s - s.max(axis=1, keepdims=True)
        e = np.exp(s)
        out[:, 128 * h:128 * (h + 1)] = (e / e.sum(axis=1, keepdims=True)) @ vh
    return out


def _textbook_prefill(x, w):
    n = x.shape[0]
    pos = np.arange(n)
    xn = _rms(x, w.input_layernorm)
    q = _rope(xn @ w.q_proj.T, 32, pos)
    k = _rope(xn @ w.k_proj.T, 8, pos)
    v = xn @ w.v_proj.T
    h = x + _attention(q, k, v, pos, pos) @ w.o_proj.T
    y = _rms(h, w.post_attention_layernorm)
    return h + (_silu(y @ w.gate_proj.T) * (y @ w.up_proj.T)) @ w.down_proj.T


@pytest.fixture(scope="module")
def prefill_case():
    spec = P.PrefillSpec()
    rng = np.random.default_rng(20261206)
    w = P.random_weights(spec, rng)
    x = rng.normal(size=(128, spec.hidden_dim))
    return spec, w, x


def test_prefill_model_is_a_textbook_layer_in_exact_mode(prefill_case):
    spec, w, x = prefill_case
    got = P.prefill_layer_numpy(x, w, spec, exact=True)
    want = _textbook_prefill(x, w)
    assert np.max(np.abs(got["output"] - want)) < 1e-12 * np.max(np.abs(want))
    # the series model differs from it only by the approximations (its softmax error, measured)
    approx = P.prefill_layer_numpy(x, w, spec)
    assert 0 < np.max(np.abs(approx["output"] - want)) < 0.05


def test_decode_model_is_a_textbook_step_in_exact_mode():
    spec = Dm.DecodeSpec()
    rng = np.random.default_rng(20261205)
    w = Dm.random_weights(spec, rng)
    hist = 40
    x = rng.normal(size=spec.hidden_dim)
    ck = rng.normal(size=(hist, 1024))
    cv = rng.normal(size=(hist, 1024))
    got = Dm.decode_layer_numpy(x, ck, cv, w, spec, position=hist, polys=Dm.DecodePolynomials.exact(spec))
    xn = _rms(x[None, :], w.input_layernorm)
    q = _rope(xn @ w.q_proj.T, 32, np.array([hist]))
    k = np.vstack([ck, _rope(xn @ w.k_proj.T, 8, np.array([hist]))])
    v = np.vstack([cv, xn @ w.v_proj.T])
    h = x[None, :] + _attention(q, k, v, np.array([hist]), np.arange(hist + 1)) @ w.o_proj.T
    y = _rms(h, w.post_attention_layernorm)
    want = (h + (_silu(y @ w.gate_proj.T) * (y @ w.up_proj.T)) @ w.down_proj.T)[0]
    assert np.max(np.abs(got["output"] - want)) < 1e-12 * np.max(np.abs(want))


def test_causal_last_row_equals_the_one_query_decode(prefill_case):
    """The prefill's last query (token 127) against keys 0..127 is the decode step of token 127
    over a cache of tokens 0..126 (their RoPE'd keys and values): same attention output, same
    RoPE positions, same GQA mapping -- restated from tests/test_poly_alg2_layer.py:23-53."""

    spec, w, x = prefill_case
    dspec = Dm.DecodeSpec()
    pre = P.prefill_layer_numpy(x, w, spec, exact=True)
    dec = Dm.decode_layer_numpy(x[127], pre["k"][:127], pre["v"][:127], w, dspec, position=127,
                                polys=Dm.DecodePolynomials.exact(dspec))
    assert np.max(np.abs(dec["attn"] - pre["attn"][127])) < 1e-12 * np.max(np.abs(pre["attn"][127]))
    assert np.allclose(dec["q"], pre["q"][127], rtol=0, atol=1e-12)
    assert np.allclose(dec["k"], pre["k"][127], rtol=0, atol=1e-12)


def test_identity_rmsnorm_layer_equals_manual_layer(prefill_case):
    """RMSNorm replaced by the identity (the reference's constant-series test), the layer's own
    series elsewhere: equal to the manual layer built from those series
    (tests/test_poly_layer.py:23-85)."""

    spec, w, x = prefill_case
    x = 0.1 * x
    got = P.prefill_layer_numpy(x, w, spec, functions={"rms": lambda m: np.ones_like(m)})
    polys = P.PrefillPolynomials.fit(spec)

    def cheb(v, c, iv):
        return np.polynomial.chebyshev.chebval((2 * v - iv[0] - iv[1]) / (iv[1] - iv[0]), c)

    n = x.shape[0]
    xn = x * w.input_layernorm
    pos = np.arange(n)
    q = _rope(xn @ w.q_proj.T, 32, pos)
    k = _rope(xn @ w.k_proj.T, 8, pos)
    v = xn @ w.v_proj.T
    attn = np.zeros((n, 4096))
    for h in range(32):
        g = h // 4
        for i in range(n):
            s = q[i, 128 * h:128 * h + 128] @ k[:i + 1, 128 * g:128 * g + 128].T
            u = (s - s.mean()) / (2 * math.sqrt(128))
            y = cheb(u, polys.exp, spec.exp_interval)
            lam = cheb(np.sum(y * y) / (i + 1), polys.rsqrt, spec.rsqrt_interval) / math.sqrt(i + 1)
            attn[i, 128 * h:128 * h + 128] = ((y * lam) ** 2) @ v[:i + 1, 128 * g:128 * g + 128]
    h1 = x + attn @ w.o_proj.T
    yy = h1 * w.post_attention_layernorm
    gate = yy @ w.gate_proj.T
    act = cheb(gate, silu_coefficients(spec.silu_degree, spec.silu_interval), spec.silu_interval) * (yy @ w.up_proj.T)
    want = h1 + act @ w.down_proj.T
    assert np.max(np.abs(got["output"] - want)) < 1e-10 * np.max(np.abs(want))


def test_mlp_block_is_swiglu_and_gamma_folds_into_the_weights():
    """mlp_block_numpy equals a direct SwiGLU in exact mode (tests/test_mlp.py:51-80), and the
    gamma folded into the gate / up columns -- the encrypted block's weight fusion -- gives the
    same block with its series (tests/test_mlp.py:82-112)."""

    rng = np.random.default_rng(26081431)
    D, I = 64, 96
    spec = MLPBlockSpec(hidden_dim=D, intermediate_width=I)
    x = rng.normal(size=(8, D))
    gate, up = rng.normal(scale=0.1, size=(I, D)), rng.normal(scale=0.1, size=(I, D))
    down = rng.normal(scale=0.1, size=(D, I))
    gamma = rng.uniform(0.75, 1.25, size=D)
    y = _rms(x, gamma)
    want = (_silu(y @ gate.T) * (y @ up.T)) @ down.T
    got = mlp_block_numpy(x, gate, up, down, gamma, spec, exact=True)
    assert np.max(np.abs(got - want)) < 1e-13
    plain = mlp_block_numpy(x, gate, up, down, gamma, spec)
    fused = mlp_block_numpy(x, gate * gamma[None, :], up * gamma[None, :], down, None, spec)
    assert np.max(np.abs(plain - fused)) < 1e-13
    assert np.max(np.abs(plain - want)) < 1e-3   # the SiLU / RMSNorm series' own error
