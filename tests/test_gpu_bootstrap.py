"""GPU checks of the bootstrap (N = 2^16, full slots, 24 x 50-bit Q primes, 8 special primes,
dnum 3, scale 2^50, sparse ternary secret of Hamming weight 192):

* ModRaise of an encryption decrypts, over the raised modulus, to m + q_0 I with the small
  overflow polynomial I the EvalMod bound assumes (|I| <= mod_bound);
* one linear-transform stage (baby rotations, the plaintext MAC, giant rotations, rescale)
  decrypts to the stage applied to the slot values on the host, and keeps the scale;
* EvalMod (the Chebyshev series by Paterson-Stockmeyer with exact scales, then the double
  angles) decrypts to the same polynomial evaluated on the host, ending on the canonical scale;
* the whole bootstrap: a ciphertext at 3 or 2 limbs comes back at the program's output level with
  its scaling factor and its slots within 2^-12 (measured: 2^-13.4 max, 2^-15 rms for random
  slots; the limit is EvalMod's rescale noise at scale 2^50, about 2^-29 after the double angles,
  against a message of 2^-8 q_0), a constant vector (one large coefficient: the sine's worst case)
  likewise, the two-pass correction of the reference within 2^-20, and this build's third pass
  below 2^-26.
The oracle is not used here: the bootstrap is built from kernels whose bit-exact parity the other
GPU tests check, so these tests check its mathematics through decryption.
"""

import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = 2.0**-12


@pytest.fixture(scope="module")
def env():
    from holmes_amd import bootstrap as B
    from holmes_amd import fhe

    spec = fhe.CKKSContextSpec(depth=23, dnum=3, dcrt_bits=50, first_mod=50, scale_bits=50,
                               secret_key_dist="SPARSE_TERNARY", hamming_weight=192, seed=20261230)
    client, ctx = fhe.generate_client_context(spec, device="cuda")
    bspec = B.BootstrapSpec(log_slots=ctx.logN - 1, level_budget=(3, 3))
    client.generate_rotation_keys(B.requirements(bspec, ctx.logN).rotations)
    prog = B.generate(ctx, bspec)
    return B, fhe, client, ctx, prog


def _slots(rng, n, scale=1.0):
    return scale * (rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)) / math.sqrt(2)


def test_program_levels(env):
    B, fhe, client, ctx, prog = env
    assert prog.raise_to_limbs == ctx.L == 24
    assert prog.evalmod_limbs == 21
    assert prog.output_limbs == 24 - 3 - 9 - 3


def test_modraise_decrypts_to_message_plus_q0_multiple(env):
    B, fhe, client, ctx, prog = env
    rng = np.random.default_rng(1)
    v = _slots(rng, ctx.max_slots)
    ct = client.encrypt(v, cur_limbs=1, scaling_factor=2.0**38)
    m = np.array([int(c) for c in client.decrypt_coeffs(ct)[0]], dtype=object)
    raised = [ctx.modraise(c[:, :1].contiguous(), 24) for c in ct.cv]
    big = ct.cipher_like(raised, state=ct.state.replace(cur_limbs=24))
    M = client.decrypt_coeffs(big)[0]  # centered over q_0 q_1 (the CRT of two limbs)
    q0 = int(ctx.q_primes[0])
    I = np.array([(int(a) - int(b)) // q0 for a, b in zip(M, m)], dtype=object)
    assert all((int(a) - int(b)) % q0 == 0 for a, b in zip(M, m))
    bound = int(np.max(np.abs(I.astype(np.int64))))
    assert bound <= prog.spec.mod_bound, bound
    assert bound >= 4  # a sparse secret of weight 192 still spreads I well past +-1


def _host_stage(B, st, x):
    n = x.shape[-1]
    rows = B.stage_rows(st, n)
    babies = [np.roll(x, -(k1 * st.h_min)) for k1 in range(st.n1)]
    out = np.zeros_like(x)
    for gi, k2 in enumerate(st.giants):
        inner = sum(rows[gi * st.n1 + k1] * babies[k1] for k1 in range(st.n1))
        out += np.roll(inner, -((k2 * st.n1 * st.h_min) % n))
    return out


@pytest.mark.parametrize("which", ["cts1", "stc0"])
def test_linear_stage_matches_host(env, which):
    B, fhe, client, ctx, prog = env
    st = prog.cts[1] if which == "cts1" else prog.stc[0]
    rng = np.random.default_rng(2)
    v = _slots(rng, ctx.max_slots, 0.5)
    ct = client.encrypt(v, cur_limbs=22)
    q = float(ctx.rescale_divisor_at(22))
    out = fhe.rescale(B.apply_stage(ct, st, ctx, q), ctx)
    assert out.state.cur_limbs == 21
    assert out.state.scaling_factor == pytest.approx(ct.state.scaling_factor, rel=1e-15)
    want = _host_stage(B, st, v)
    got = client.decrypt(out)
    assert np.max(np.abs(got - want)) < 2.0**-25 * max(1.0, float(np.max(np.abs(want))))


def test_deferred_stages_match_host(env):
    # three CoeffToSlot stages at one level with the constant shares, then three rescales
    B, fhe, client, ctx, prog = env
    rng = np.random.default_rng(5)
    v = _slots(rng, ctx.max_slots, 0.5)
    ct = client.encrypt(v, cur_limbs=20)
    out = B.apply_stages(ct, prog.cts, 0.75, ctx, keep=False)
    assert out.state.cur_limbs == 20 and out.state.scale_degree == 4
    for _ in range(3):
        out = fhe.rescale(out, ctx)
    assert out.state.cur_limbs == 17
    assert out.state.scaling_factor == pytest.approx(ct.state.scaling_factor * 0.75**3, rel=1e-14)
    want = v
    for st in prog.cts:
        want = _host_stage(B, st, want)
    got = client.decrypt(out) * 0.75**3
    assert np.max(np.abs(got - want * 0.75**3)) < 2.0**-30


def test_evalmod_matches_host_polynomial(env):
    B, fhe, client, ctx, prog = env
    rng = np.random.default_rng(3)
    u = rng.uniform(-1, 1, (2, ctx.max_slots))
    l0 = prog.evalmod_limbs
    S = prog.nominal_scale
    both = fhe.pack_cipher_batch([client.encrypt(u[0], cur_limbs=l0, scaling_factor=S),
                                  client.encrypt(u[1], cur_limbs=l0, scaling_factor=S)])
    ev = B._PSEval(ctx, both, l0, S, prog.spec.cheb_degree, ctx.q_primes)
    y = ev.evaluate(prog.cheb)
    for _ in range(prog.spec.double_angle):
        y = ev.double_minus(y, y)
    assert y.state.cur_limbs == prog.output_limbs + 3
    assert y.state.scaling_factor == prog.evalmod_out_scale
    want = np.polynomial.chebyshev.chebval(u, prog.cheb)
    for _ in range(prog.spec.double_angle):
        want = 2 * want * want - 1
    got = client.decrypt(y).real
    # the evaluation's own noise at scale 2^50 (fresh encryption noise through the T_k chain and three
    # double angles) sits near 2^-24.3 at the maximum over 65536 slots; 2^-23 leaves it a margin
    assert np.max(np.abs(got - want)) < 2.0**-23


@pytest.mark.parametrize("limbs", [3, 2])
def test_bootstrap_restores_levels_and_slots(env, limbs):
    B, fhe, client, ctx, prog = env
    rng = np.random.default_rng(10 + limbs)
    v = _slots(rng, ctx.max_slots)
    ct = client.encrypt(v, cur_limbs=limbs)
    out = B.bootstrap(ct, ctx, prog)
    assert out.state.cur_limbs == prog.output_limbs
    assert out.state.scaling_factor == ct.state.scaling_factor and out.state.scale_degree == 1
    got = client.decrypt(out)
    err = float(np.max(np.abs(got - v)))
    print(f"bootstrap from {limbs} limbs: max error 2^{math.log2(err):.1f}")
    assert err < TOL, err
    # the refreshed ciphertext computes on: a product with a fresh one at its level
    w = _slots(rng, ctx.max_slots)
    cw = client.encrypt(w, cur_limbs=out.state.cur_limbs, scaling_factor=out.state.scaling_factor)
    prod = fhe.rescale(fhe.homo_mul_relin(out, cw, ctx), ctx)
    assert np.max(np.abs(client.decrypt(prod) - v * w)) < 2 * TOL


def test_bootstrap_of_a_constant(env):
    B, fhe, client, ctx, prog = env
    v = np.full(ctx.max_slots, 0.9)
    out = B.bootstrap(client.encrypt(v, cur_limbs=2), ctx, prog)
    err = float(np.max(np.abs(client.decrypt(out) - v)))
    print(f"bootstrap of a constant: max error 2^{math.log2(err):.1f}")
    assert err < TOL, err


def test_two_pass_correction(env):
    B, fhe, client, ctx, prog = env
    rng = np.random.default_rng(21)
    v = _slots(rng, ctx.max_slots)
    ct = client.encrypt(v, cur_limbs=3)
    one = B.bootstrap_with_correction(ct, ctx, prog, iterations=1)
    two = B.bootstrap_with_correction(ct, ctx, prog, iterations=2, precision_bits=12)
    assert one.state.cur_limbs == prog.output_limbs
    assert two.state.cur_limbs == prog.output_limbs - 1
    assert two.state.scaling_factor == ct.state.scaling_factor
    e1 = float(np.max(np.abs(client.decrypt(one) - v)))
    e2 = float(np.max(np.abs(client.decrypt(two) - v)))
    print(f"one pass 2^{math.log2(e1):.1f}, two passes 2^{math.log2(e2):.1f}")
    assert e2 < 2.0**-20 and e2 < e1 / 64


def test_three_pass_correction(env):
    """The third correction pass (this build's extension) leaves the two-pass output level and the
    input's scale, and cuts the error below the two-pass error."""
    B, fhe, client, ctx, prog = env
    rng = np.random.default_rng(22)
    v = _slots(rng, ctx.max_slots)
    ct = client.encrypt(v, cur_limbs=3)
    two = B.bootstrap_with_correction(ct, ctx, prog, iterations=2, precision_bits=12)
    three = B.bootstrap_with_correction(ct, ctx, prog, iterations=3, precision_bits=12)
    assert three.state.cur_limbs == two.state.cur_limbs == prog.output_limbs - 1
    assert three.state.scaling_factor == ct.state.scaling_factor
    e2 = float(np.max(np.abs(client.decrypt(two) - v)))
    e3 = float(np.max(np.abs(client.decrypt(three) - v)))
    print(f"two passes 2^{math.log2(e2):.1f}, three passes 2^{math.log2(e3):.1f}")
    assert e3 < 2.0**-26 and e3 < e2 / 4


@pytest.mark.parametrize("iterations", [2, 1])
def test_refresh_graph_replays_equal_eager(env, iterations):
    """A refresh captured as one HIP graph: every replay, with eager refreshes and other kernels
    between the replays, gives the eager result bit for bit, for two different inputs in turn."""
    B, fhe, client, ctx, prog = env
    rng = np.random.default_rng(40 + iterations)
    cts = [client.encrypt(_slots(rng, ctx.max_slots), cur_limbs=3) for _ in range(2)]
    graph = B.RefreshGraph(ctx, prog, cts[0], iterations=iterations)
    for rep in range(3):
        for ct in cts:
            got = graph(ct)
            want = B.bootstrap_with_correction(ct, ctx, prog, iterations=iterations)
            fhe.homo_add(want, want, ctx)  # other eager work between replays
            torch.cuda.synchronize()
            assert got.state.cur_limbs == want.state.cur_limbs
            for a, b in zip(got.cv, want.cv):
                assert torch.equal(a[:, :want.state.cur_limbs], b[:, :want.state.cur_limbs]), rep
    with pytest.raises(ValueError):
        graph(client.encrypt(_slots(rng, ctx.max_slots), cur_limbs=4))


def test_batched_bootstrap_equals_single_ones(env):
    # every kernel of the pipeline works per item, so a batch refreshes bit-identically
    B, fhe, client, ctx, prog = env
    rng = np.random.default_rng(6)
    cts = [client.encrypt(_slots(rng, ctx.max_slots), cur_limbs=3) for _ in range(3)]
    batch = B.bootstrap(fhe.pack_cipher_batch(cts), ctx, prog)
    assert batch.batch_size == 3 and batch.state.cur_limbs == prog.output_limbs
    for i, ct in enumerate(cts):
        one = B.bootstrap(ct, ctx, prog)
        for a, b in zip(batch.cv, one.cv):
            assert torch.equal(a[i:i + 1, :one.state.cur_limbs], b[:, :one.state.cur_limbs]), f"item {i}"
    two = B.bootstrap_with_correction(fhe.pack_cipher_batch(cts), ctx, prog, iterations=2)
    for i, ct in enumerate(cts):
        assert np.max(np.abs(client.decrypt(fhe.cipher_batch_item(two, i)) - client.decrypt(ct))) < 2.0**-20


def test_bootstrap_checks_its_input(env):
    B, fhe, client, ctx, prog = env
    rng = np.random.default_rng(4)
    one = client.encrypt(_slots(rng, ctx.max_slots), cur_limbs=1)
    with pytest.raises(ValueError):
        B.bootstrap(one, ctx, prog)
    three = one.cipher_like([one.cv[0], one.cv[1], one.cv[0]])
    with pytest.raises(ValueError):
        B.bootstrap(three, ctx, prog)
