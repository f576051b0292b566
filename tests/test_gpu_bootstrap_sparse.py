"""GPU checks of the sparse-slot and deep bootstrap programs through the operator surface Holmes
refreshes with (holmes_amd.refresh, after llama3fhe/operators/nonlinear/bootstrap.py:47-160,
380-470): N = 2^16, 24 x 50-bit Q primes, dnum 3, scale 2^50, sparse ternary secret (h = 192).

* sparse programs (4096 and 16 slots): a ciphertext of n slots at 3 limbs comes back at the
  program's output level with its slots restored (measured: 2^-14.3 / 2^-19.5 in one pass,
  2^-22.8 / 2^-23.3 with the two-pass correction, which converges only because the output is
  projected back onto the subring);
* the periodic view: a full-slot ciphertext whose message repeats every 4096 slots refreshes
  through the 4096-slot program and decrypts to the same full-slot vector;
* the deep program (budget (2, 2)) leaves two more limbs than the main (3, 3) one and restores
  the slots as well;
* requests without a matching program are refused.
Decryption is the check, as for the full-slot program (the kernels' parity is tested elsewhere)."""

import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def env():
    from holmes_amd import bootstrap as B
    from holmes_amd import fhe
    from holmes_amd.refresh import BootstrapConfig, BootstrapOperator

    spec = fhe.CKKSContextSpec(depth=23, dnum=3, dcrt_bits=50, first_mod=50, scale_bits=50,
                               secret_key_dist="SPARSE_TERNARY", hamming_weight=192, seed=20261231)
    client, ctx = fhe.generate_client_context(spec, device="cuda")
    cfg = BootstrapConfig(level_budget=(3, 3), deep_level_budget=(2, 2), deep_output_levels=0,
                          sparse_log_slots=(12, 4))
    client.generate_rotation_keys(B.requirements(cfg.all_specs(), ctx.logN).rotations)
    op = BootstrapOperator.prepare(ctx, cfg)
    print(f"programs: main {op.program.output_limbs}, deep {op.deep_program.output_limbs}, sparse "
          f"{ {k: p.output_limbs for k, p in op.sparse_programs.items()} } limbs", flush=True)
    return B, fhe, client, ctx, op


def _slots(rng, n):
    return (rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)) / math.sqrt(2)


@pytest.mark.parametrize("n,tol1,tol2", [(4096, 2.0**-12, 2.0**-20), (16, 2.0**-16, 2.0**-20)])
def test_sparse_program_restores_the_slots(env, n, tol1, tol2):
    B, fhe, client, ctx, op = env
    prog = op.sparse_programs[n]
    rng = np.random.default_rng(n)
    v = _slots(rng, n)
    ct = client.encrypt(v, cur_limbs=3, slots=n)
    one = B.bootstrap_with_correction(ct, ctx, prog, iterations=1)
    two = B.bootstrap_with_correction(ct, ctx, prog, iterations=2, precision_bits=12)
    assert one.slots == n and one.state.cur_limbs == prog.output_limbs
    assert two.state.scaling_factor == ct.state.scaling_factor
    e1 = float(np.max(np.abs(client.decrypt(one) - v)))
    e2 = float(np.max(np.abs(client.decrypt(two) - v)))
    print(f"sparse {n} slots: one pass 2^{math.log2(e1):.1f}, two passes 2^{math.log2(e2):.1f}", flush=True)
    assert e1 < tol1 and e2 < tol2


def test_periodic_full_slot_message_through_the_sparse_program(env):
    B, fhe, client, ctx, op = env
    rng = np.random.default_rng(7)
    period = _slots(rng, 4096)
    full = np.tile(period, ctx.max_slots // 4096)
    ct = client.encrypt(full, cur_limbs=3)
    out = op.refresh(ct, periodic_slots=4096)
    assert out.slots == ctx.max_slots and op.sparse_calls == 1
    err = float(np.max(np.abs(client.decrypt(out) - full)))
    print(f"periodic view: 2^{math.log2(err):.1f}", flush=True)
    assert err < 2.0**-20


def test_deep_program_leaves_two_more_limbs(env):
    B, fhe, client, ctx, op = env
    assert op.deep_program.output_limbs == op.program.output_limbs + 2
    rng = np.random.default_rng(8)
    v = _slots(rng, ctx.max_slots)
    ct = client.encrypt(v, cur_limbs=3)
    out = op.refresh(ct, use_deep_program=True)
    assert out.state.cur_limbs == op.deep_program.output_limbs - 1  # two passes: one level for 2^-p
    err = float(np.max(np.abs(client.decrypt(out) - v)))
    print(f"deep program, two passes: 2^{math.log2(err):.1f}", flush=True)
    assert err < 2.0**-20


def test_requests_without_a_program_are_refused(env):
    B, fhe, client, ctx, op = env
    ct = client.encrypt(np.zeros(ctx.max_slots), cur_limbs=3)
    with pytest.raises(ValueError, match="sparse program"):
        op.refresh(ct, periodic_slots=256)
    with pytest.raises(ValueError):
        op.refresh(ct, periodic_slots=4096, use_deep_program=True)
    with pytest.raises(ValueError, match="4096 slots"):
        B.bootstrap(ct, ctx, op.sparse_programs[4096])
