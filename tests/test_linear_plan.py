"""BSGS schedule known answers (the reference's own plan tests, tests/test_linear.py:21-164,
restated against holmes_amd.linear)."""

import pytest

from holmes_amd.linear import LinearOperatorConfig, bsgs_rotations, linear_rotations


def test_production_plan_shape():
    plan = LinearOperatorConfig(baby_steps=32, max_plaintext_rows=512,
                                hoist_strategy="ext_double_hoist").plan(dimension=4096, token_lanes=8)
    assert plan.giant_steps == 128
    assert plan.chunk_giants == 16
    assert plan.chunk_sizes == (16,) * 8
    assert plan.plaintext_chunks == 8
    assert plan.giant_offset == 256
    assert plan.baby_offsets == tuple(8 * i for i in range(32))


def test_large_baby_schedule_caps_fast_rotation_keys_at_32():
    cfg = LinearOperatorConfig(baby_steps=32, baby_anchor_step=32, max_plaintext_rows=512)
    plan = cfg.plan(dimension=4096, token_lanes=8)
    rot = set(linear_rotations(dimension=4096, token_lanes=8, operator_config=cfg))
    assert tuple(b.width for b in plan.baby_blocks) == (32,)
    assert plan.baby_rotation_count == 31
    assert plan.baby_key_offsets == tuple(8 * i for i in range(1, 32))
    assert set(plan.baby_key_offsets) <= rot and 256 not in plan.baby_key_offsets
    large = LinearOperatorConfig(baby_steps=128, baby_anchor_step=32, max_plaintext_rows=512).plan(
        dimension=4096, token_lanes=8)
    assert tuple(b.width for b in large.baby_blocks) == (32,) * 4
    assert large.baby_rotation_count == 127
    assert large.baby_key_offsets == tuple(8 * i for i in range(1, 33))


def test_baby_step_64_single_block():
    cfg = LinearOperatorConfig(baby_steps=64, baby_anchor_step=64, max_plaintext_rows=512)
    plan = cfg.plan(dimension=4096, token_lanes=8)
    assert plan.anchor_enabled is False
    assert len(linear_rotations(dimension=4096, token_lanes=8, operator_config=cfg)) == 71


@pytest.mark.parametrize(("strategy", "baby", "anchor", "keys"), [
    ("normal", 32, 32, 39), ("ext_normal", 32, 32, 39), ("ext_double_hoist", 32, 32, 53),
    ("normal", 64, 64, 71), ("ext_normal", 64, 64, 71), ("ext_double_hoist", 64, 64, 77),
    ("normal", 128, 64, 72), ("ext_normal", 128, 64, 72), ("ext_double_hoist", 128, 64, 74),
])
def test_rotation_key_counts(strategy, baby, anchor, keys):
    cfg = LinearOperatorConfig(baby_steps=baby, baby_anchor_step=anchor, max_plaintext_rows=512,
                               hoist_strategy=strategy)
    rot = linear_rotations(dimension=4096, token_lanes=8, operator_config=cfg)
    assert len(rot) == keys and len(set(rot)) == len(rot)


def test_conjugation_key_and_c3_schedule():
    rot = linear_rotations(dimension=4096, token_lanes=8, slots=32768, include_conjugation=True,
                           operator_config=LinearOperatorConfig(baby_steps=32))
    assert 4 * 32768 - 1 in rot
    # BASELINE C3: q_proj, baby 16, 512 plaintext rows: 256 giants in 8 chunks of 32
    plan = LinearOperatorConfig(baby_steps=16, baby_anchor_step=-1, max_plaintext_rows=512).plan(
        dimension=4096, token_lanes=8)
    assert plan.giant_steps == 256 and plan.chunk_sizes == (32,) * 8 and plan.giant_offset == 128
    keys = bsgs_rotations(plan)
    assert len(keys) == 15 + 1 + 7  # babies, giant offset, chunk bases


def test_invalid_schedules_raise():
    with pytest.raises(ValueError):
        LinearOperatorConfig(baby_steps=0)
    with pytest.raises(ValueError):
        LinearOperatorConfig(baby_anchor_step=1)
    with pytest.raises(ValueError):
        LinearOperatorConfig(baby_steps=24).plan(dimension=4096, token_lanes=8)
