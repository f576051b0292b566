"""CPU checks of the prefill layer: the float64 model against a loop-level restatement of the
reference's prefill semantics, the weight blocks and slot constants, and the encrypted attention
dataflow (``PrefillAttention``) on the slot simulator with the production prime chain's level and
scale bookkeeping: layouts, lane rotations, packing, masks and levels must reproduce the float64
attention output to round-off."""

import math

import numpy as np
import pytest

from holmes_amd import prefill as P
from holmes_amd.decode import random_weights
from holmes_amd.layouts import FeatureMajorPrefillLayout
from holmes_amd.norm import rmsnorm_coefficients, rmsnorm_numpy

from .slot_sim import SimCt, SlotOps, make_programs

SEED = 20261206


@pytest.fixture(scope="module")
def env():
    spec = P.PrefillSpec()
    rng = np.random.default_rng(SEED)
    w = random_weights(spec, rng)
    x = rng.normal(size=(128, 4096))
    rms = rmsnorm_coefficients(spec.rms_degree, spec.rms_interval, spec.eps)
    xn = rmsnorm_numpy(x, w.input_layernorm, rms)
    return spec, w, x, xn


def test_model_matches_a_loop_restatement(env):
    """Scores, causal Alg2 and PV of attention_numpy against explicit per-head loops with the
    same polynomials; RoPE as the rotate-half rotation written out."""
    spec, w, x, xn = env
    att = P.attention_numpy(xn, w, spec)
    polys = P.PrefillPolynomials.fit(spec)
    q = xn @ w.q_proj.T
    k = xn @ w.k_proj.T
    v = xn @ w.v_proj.T
    inv = 1.0 / (np.float32(spec.rope_theta) ** (np.arange(0, 128, 2, dtype=np.float32) / np.float32(128)))

    def rope(vec, pos):
        ang = (np.float32(pos) * inv.astype(np.float32)).astype(np.float32)
        c, s = np.cos(ang).astype(np.float64), np.sin(ang).astype(np.float64)
        a, b = vec[:64], vec[64:]
        return np.concatenate([a * c - b * s, b * c + a * s])

    for h in (0, 5, 31):
        g = h // 4
        for qi in (0, 7, 64, 127):
            qv = rope(q[qi, 128 * h:128 * h + 128], qi)
            keys = [rope(k[ki, 128 * g:128 * g + 128], ki) for ki in range(qi + 1)]
            s = np.array([qv @ kv for kv in keys])
            assert np.allclose(s, att["scores"][h, qi, :qi + 1], rtol=1e-9, atol=1e-9)
            u = (s - s.mean()) / (2.0 * math.sqrt(128))
            a, b = spec.exp_interval
            y = np.polynomial.chebyshev.chebval((2 * u - (a + b)) / (b - a), polys.exp)
            r = np.sum(y * y) / (qi + 1)
            a2, b2 = spec.rsqrt_interval
            lam = np.polynomial.chebyshev.chebval((2 * r - (a2 + b2)) / (b2 - a2), polys.rsqrt) / math.sqrt(qi + 1)
            p = (y * lam) ** 2
            o = sum(p[ki] * v[ki, 128 * g:128 * g + 128] for ki in range(qi + 1))
            assert np.allclose(o, att["attn"][qi, 128 * h:128 * h + 128], rtol=1e-9, atol=1e-12)
    # the Alg2 probabilities approximate the exact softmax on these inputs, and stay in range
    assert att["in_range"]["exp"] and att["in_range"]["rsqrt"], att["in_range"]
    assert att["softmax_vs_exact"] < 5e-3, att["softmax_vs_exact"]


def test_weight_blocks_carry_the_folded_heads(env):
    spec, w, x, xn = env
    lay = FeatureMajorPrefillLayout()
    a = xn @ P.qk_matrix(w).T
    q = xn @ w.q_proj.T
    k = xn @ w.k_proj.T
    assert np.allclose(a[:, 64 * 7 + 3], q[:, 128 * 7 + 3] + 1j * q[:, 128 * 7 + 67])
    g = 9 // 4
    assert np.allclose(a[:, 2048 + 64 * 9 + 5], k[:, 128 * g + 5] - 1j * k[:, 128 * g + 69])
    o = np.random.default_rng(1).normal(size=(128, 4096))
    oz = (o.reshape(128, 32, 128)[:, :, :64] + 1j * o.reshape(128, 32, 128)[:, :, 64:]).reshape(128, 2048)
    oz = np.hstack([oz, np.zeros_like(oz)])
    d = oz @ P.wo_matrix(w).T
    assert np.allclose(2 * d.real, o @ w.o_proj.T)
    assert len(lay.pack(a.real)) == 16


def test_slot_constants():
    lo, hi = P.lane_masks(3)
    d, t = np.arange(32768) // 8, np.arange(32768) % 8
    assert np.all((lo + hi) == (d < 2048)) and np.all(lo[(d < 2048) & (t < 5)] == 1)
    ulo, uhi = P.lane_masks(3, upper=True)
    assert np.all((ulo + uhi) == (d >= 2048)) and np.all(uhi[(d >= 2048) & (t >= 5)] == 1)
    valid = P.validity_rows()
    # query ciphertext c keeps keys j < 4 (c + 1) at channel position j of the lower half and
    # the others at j - 4 (c + 1) of the upper; key j = 8 c' + rho reaches lane t as token
    # 8 c' + (t + rho) % 8
    s = 8 * (64 * 3 + 5) + 2                  # head 3, position 5, lane 2
    assert valid[1, s] == 1                   # c = 1: j = 5 (c' = 0) -> key 7 <= query 10
    assert valid[1, 16384 + s] == 0           # j = 13 (c' = 1, rho = 5) -> key 15 > query 10
    assert valid[1, 16384 + s + 4] == 1       # lane 6: key 8 + 3 = 11 <= query 14
    assert valid[2, 16384 + s] == 0           # c = 2: j = 17 (c' = 2, rho = 1) -> key 19 > query 18
    assert valid[2, 8 * (64 * 3 + 11) + 2] == 1   # j = 11 (c' = 1) in the lower half
    assert valid[2, 8 * (64 * 3 + 12) + 2] == 0   # position 12 of the lower half is unused at c = 2
    assert valid[0, 8 * 4] == 0 and valid[0, 16384 + 8 * 4] == 0   # position 4 is unused at c = 0
    assert valid.sum() == 32 * sum(8 * c + t + 1 for c in range(16) for t in range(8))
    assert P.key_slot(15, 70) == 16384 + 48 and P.key_slot(1, 10) == 16384 + 16 and P.key_slot(1, 7) == 56
    rots = P.attention_rotations()
    assert 16384 in rots and all(0 < r < 32768 for r in rots)


def test_attention_dataflow_on_the_slot_simulator(env):
    spec, w, x, xn = env
    cs = P.prefill_context_spec()
    q_primes, _ = cs.prime_chain()
    scale = 2.0**50
    ops = SlotOps(q_primes, *make_programs(q_primes, len(q_primes), scale))
    attn = P.PrefillAttention(ops, spec)
    A, V = P.attention_input_numpy(xn, spec, w)
    a_ct, v_ct = SimCt(A, 29, scale), SimCt(V, 29, scale)
    out, mid = attn.forward(a_ct, v_ct)
    model = P.attention_numpy(xn, w, spec)
    oz = model["attn"].reshape(128, 32, 128)
    oz = (oz[:, :, :64] + 1j * oz[:, :, 64:]).reshape(128, 2048)
    oz = np.hstack([oz, np.zeros_like(oz)])
    lay = FeatureMajorPrefillLayout()
    want = np.asarray(lay.pack(oz.real)) + 1j * np.asarray(lay.pack(oz.imag))
    got = out.values.copy()
    got[:, 16384:] = 0  # the upper half carries nothing for W_O (its columns are zero)
    err = np.max(np.abs(got[:, :16384] - want[:, :16384]))
    mag = np.max(np.abs(want))
    print(f"attention sim: max error {err:.3e} of magnitude {mag:.3f}; output at {ops.limbs(out)} limbs; "
          f"probabilities at {ops.limbs(mid['probs'])}; log {ops.log[:3]}")
    assert err < 1e-9 * mag
    assert ops.limbs(out) >= 3  # W_O (one level) leaves the residual two limbs for its refresh


def test_steady_state_attention_on_the_slot_simulator(env):
    """The steady-state layer's attention with the layer's own refresh programs (each raised only as
    far as its consumer needs): A and V at the level the refreshed layer input leaves after RMSNorm1
    and the projections, the exp and inverse-square-root inputs refreshed; the output must still
    leave levels for W_O and the residual."""
    spec, w, x, xn = env
    cs = P.prefill_context_spec()
    q_primes, _ = cs.prime_chain()
    scale = 2.0**50
    ops = SlotOps(q_primes, *make_programs(q_primes, len(q_primes), scale))
    from holmes_amd import bootstrap as B

    raises = P.refresh_raise_limbs(q_primes)
    progs = {k: B.plan_program(P.prefill_bootstrap_spec(r), q_primes, scale, r) for k, r in raises.items()}
    assert all(progs[k].output_limbs - 1 >= v for k, v in P.REFRESH_LIMBS.items()), raises
    start = progs["input"].output_limbs - 1 - 9                # refreshed input -> RMSNorm1 (8) -> projections (1)
    attn = P.PrefillAttention(ops, spec, refresh_series_inputs=True, series_programs=progs)
    A, V = P.attention_input_numpy(xn, spec, w)
    out, mid = attn.forward(SimCt(A, start, scale), SimCt(V, start, scale))
    model = P.attention_numpy(xn, w, spec)
    oz = model["attn"].reshape(128, 32, 128)
    oz = np.hstack([(oz[:, :, :64] + 1j * oz[:, :, 64:]).reshape(128, 2048), np.zeros((128, 2048))])
    lay = FeatureMajorPrefillLayout()
    want = np.asarray(lay.pack(oz.real)) + 1j * np.asarray(lay.pack(oz.imag))
    err = np.max(np.abs(out.values[:, :16384] - want[:, :16384]))
    print(f"steady attention sim: A at {start} limbs, output at {ops.limbs(out)} limbs, {ops.refreshes} refreshed "
          f"items, error {err:.2e}")
    assert err < 1e-9 * np.max(np.abs(want))
    assert ops.limbs(out) >= 3 and ops.refreshes == 17
