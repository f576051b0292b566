"""Shifted-lane (SL) packing of the decode linears, after llama3fhe/layouts/shifted_lane.py:1-241
and its tests (tests/test_shifted_lane.py): lane l of channel c holds x[(c + shift l) mod D],
shift = D / lanes; a D x D block costs `shift` diagonals.  The known answers of the reference's
plan test, the BSGS composition of this build's diagonal packer (the C oracle's
or_pack_diagonals, the same formula as the HIP packer) against W @ x, and the lane-0 expansion
by rotate-and-add doubling against the SL packing."""

import numpy as np
import pytest

from holmes_amd.linear import LinearOperatorConfig, linear_rotations
from oracle import oracle as O


def _pack(x, D, slots):
    lanes = slots // D
    shift = D // lanes
    s = np.arange(slots)
    return x[((s // lanes) + shift * (s % lanes)) % D]


def _roll(v, r):
    return np.roll(v, -int(r))  # rot(v, r)[s] = v[s + r]


def test_shifted_lane_plan_known_answers():
    """The reference's plan test (tests/test_shifted_lane.py:83-97)."""

    config = LinearOperatorConfig(baby_steps=64, baby_anchor_step=64, max_plaintext_rows=64, lane_shift=512)
    plan = config.plan(dimension=4096, token_lanes=8)
    assert plan.diagonals == 512
    assert plan.giant_steps == 8
    assert plan.plaintext_chunks == 8
    assert plan.fold_offsets == (1, 2, 4)
    assert plan.lane_expand_offsets == tuple(4095 * l for l in range(1, 8))
    keys = set(linear_rotations(dimension=4096, token_lanes=8, operator_config=config))
    assert {1, 2, 4, 4095, 4095 * 7} <= keys
    with pytest.raises(ValueError):
        LinearOperatorConfig(lane_shift=256).plan(dimension=4096, token_lanes=8)


@pytest.mark.parametrize("baby_steps", (1, 2, 4, 8))
def test_packed_diagonals_compose_to_the_matvec(baby_steps):
    """sum_g rot(sum_b row(g, b) * rot(x, b lanes), g B lanes), lanes folded, equals W @ x for
    every baby size (tests/test_shifted_lane.py:48-55), from the packer's own rows."""

    D, slots = 64, 512
    lanes, shift = slots // D, D // (slots // D)
    rng = np.random.default_rng(2)
    W = rng.standard_normal((D, D))
    x = rng.standard_normal(D)
    carrier = _pack(x, D, slots)
    giants = shift // baby_steps
    rows = O.pack_diagonals(W, lanes, shift, baby_steps, 0, giants, slots)
    out = np.zeros(slots)
    for g in range(giants):
        acc = sum(rows[g * baby_steps + b] * _roll(carrier, b * lanes) for b in range(baby_steps))
        out += _roll(acc, g * baby_steps * lanes)
    folded = out.copy()
    for f in (1, 2, 4):
        folded = folded + _roll(folded, f)
    assert np.allclose(folded[::lanes], W @ x, atol=1e-12)
    # each lane holds the partial product over its input block
    part = out.reshape(D, lanes)
    for l in range(lanes):
        cols = (np.arange(D)[:, None] + np.arange(shift)[None, :] + shift * l) % D
        assert np.allclose(part[:, l], np.einsum("cj,cj->c", W[np.arange(D)[:, None], cols], x[cols]))


def test_lane0_doubling_expansion_equals_the_packing():
    """Three rotate-and-adds by (D - 1) 2^k build the SL carrier from lane 0 (the expansion of
    llama3fhe/layouts/shifted_lane.py:133-160 in log2(lanes) steps)."""

    D, slots = 64, 512
    rng = np.random.default_rng(1)
    x = rng.standard_normal(D)
    v = np.zeros(slots)
    v[::8] = x
    for k in range(3):
        v = v + _roll(v, (D - 1) << k)
    assert np.allclose(v, _pack(x, D, slots))
