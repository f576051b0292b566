"""End-to-end CKKS semantics on the GPU: encrypt -> op -> decrypt against NumPy float64.

Pins the slot conventions of llama3fhe: rotate(v, r)[s] = v[(s + r) mod slots]
(llama3fhe/layouts/shifted_lane.py:24-37), conjugation through galois element 2N - 1
(operators/linear/complex.py:63-67), multiplication by i through homo_mul_i, and rescale
dividing the scale by q_last.  Tolerance: 2^-16 relative to the slot scale (the bar of the
decrypted-output parity).
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

TOL = 2.0**-16


@pytest.fixture(scope="module")
def env():
    from holmes_amd import fhe

    spec = fhe.CKKSContextSpec(depth=23, dnum=3, seed=7, rotations=(1, 5, -3, 64, (1 << 17) - 1))
    client, ctx = fhe.generate_client_context(spec)
    return fhe, client, ctx


def test_encrypt_decrypt_roundtrip(env):
    fhe, client, ctx = env
    rng = np.random.default_rng(1)
    v = rng.normal(size=ctx.max_slots)
    ct = client.encrypt(v, cur_limbs=20)
    out = client.decrypt(ct)
    assert np.max(np.abs(out.real - v)) < TOL


@pytest.mark.parametrize("r", [1, 5, -3, 64])
def test_rotation_semantics(env, r):
    fhe, client, ctx = env
    rng = np.random.default_rng(r + 100)
    v = rng.normal(size=ctx.max_slots) + 1j * rng.normal(size=ctx.max_slots)
    ct = client.encrypt(v, cur_limbs=24)
    rot = fhe.homo_rotate(ct, r, ctx)
    out = client.decrypt(rot)
    assert np.max(np.abs(out - np.roll(v, -r))) < TOL


def test_conjugation(env):
    fhe, client, ctx = env
    rng = np.random.default_rng(2)
    v = rng.normal(size=ctx.max_slots) + 1j * rng.normal(size=ctx.max_slots)
    ct = client.encrypt(v, cur_limbs=12)
    out = client.decrypt(fhe.homo_rotate(ct, ctx.M - 1, ctx))
    assert np.max(np.abs(out - np.conj(v))) < TOL


def test_mul_i_add_sub(env):
    fhe, client, ctx = env
    rng = np.random.default_rng(3)
    a = rng.normal(size=ctx.max_slots)
    b = rng.normal(size=ctx.max_slots)
    ca, cb = client.encrypt(a, cur_limbs=10), client.encrypt(b, cur_limbs=10)
    out = client.decrypt(fhe.homo_add(fhe.homo_mul_i(ca, ctx), cb, ctx))
    assert np.max(np.abs(out - (1j * a + b))) < TOL
    out = client.decrypt(fhe.homo_sub(fhe.homo_mul_i(ca, ctx, negative=True), cb, ctx))
    assert np.max(np.abs(out - (-1j * a - b))) < TOL


def test_plain_multiply_and_rescale(env):
    fhe, client, ctx = env
    rng = np.random.default_rng(4)
    a = rng.normal(size=ctx.max_slots)
    w = rng.normal(scale=0.5, size=ctx.max_slots)
    ct = client.encrypt(a, cur_limbs=20)
    # plaintext at scale q_last so the rescaled product returns to the input scale
    st = fhe.CipherState(cur_limbs=20, scale_degree=1, scaling_factor=float(ctx.rescale_divisor_at(20)))
    pt = fhe.encode_plaintext(w, st, ctx.max_slots, ctx)
    prod = fhe.rescale(fhe.homo_mul_pt(ct, pt, ctx), ctx)
    assert prod.state.cur_limbs == 19
    assert abs(prod.state.scaling_factor - ct.state.scaling_factor) < 1e-6 * ct.state.scaling_factor
    out = client.decrypt(prod)
    assert np.max(np.abs(out.real - a * w)) < TOL


def test_batched_rotation_one_key_per_item(env):
    fhe, client, ctx = env
    rng = np.random.default_rng(5)
    v = rng.normal(size=(3, ctx.max_slots))
    ct = client.encrypt(v, cur_limbs=16)
    rots = [1, 5, -3]
    out = client.decrypt(fhe.homo_rotate_batch(ct, rots, ctx))
    for b, r in enumerate(rots):
        assert np.max(np.abs(out[b].real - np.roll(v[b], -r))) < TOL


def test_align_to_drops_limbs_only(env):
    fhe, client, ctx = env
    rng = np.random.default_rng(6)
    v = rng.normal(size=ctx.max_slots)
    ct = client.encrypt(v, cur_limbs=18)
    low = fhe.align_to(ct, ct.state.replace(cur_limbs=9), ctx)
    assert low.state.cur_limbs == 9
    assert np.max(np.abs(client.decrypt(low).real - v)) < TOL


def test_easyfhe_context_session_roundtrip():
    """The llama3fhe/backend.py session surface: create_sim_context, encrypt at a level,
    plaintext at a level, homo_mul_pt + rescale, decrypt."""

    from holmes_amd import backend
    from holmes_amd.config import SimulatorConfig

    cfg = SimulatorConfig(maxLevelsRemaining=5, dnum=2, dcrtBits=50, firstMod=50, scaleBits=40)
    sess = backend.create_sim_context(cfg, input_dim=16, block_out=8, rotations=(3,))
    assert sess.max_slots == 32768 and sess.context.L == 6
    rng = np.random.default_rng(11)
    v = rng.normal(size=sess.max_slots)
    w = rng.normal(size=sess.max_slots)
    ct = sess.encrypt(v, level=1)
    assert sess.level_for_cipher(ct) == 1 and ct.state.cur_limbs == 5
    pt = sess.plaintext(w, name="model.layers.3.w", level=1)
    prod = sess.fhe.rescale(sess.fhe.homo_mul_pt(ct, pt, sess.context), sess.context)
    assert sess.level_for_cipher(prod) == 2
    out = sess.decrypt(prod)
    assert np.max(np.abs(out.real - v * w)) < 2.0**-10  # scale 2^40 * 2^40 / q (~2^50) = 2^30
    rot = sess.decrypt(sess.fhe.homo_rotate(ct, 3, sess.context))
    assert np.max(np.abs(rot.real - np.roll(v, -3))) < TOL
    backend.release_if_supported(prod)
    assert prod.cv == []


def test_encryption_randomness_is_fresh_unless_deterministic():
    """Two clients of one spec (same keys) must not reuse (a, e): c0 - c0' would reveal m - m'.
    With deterministic_encryption the n-th encryptions coincide, for reproducible tests."""
    from holmes_amd import fhe

    v = np.linspace(-1.0, 1.0, 1 << 15)
    outs = []
    for det in (False, False, True, True):
        client, ctx = fhe.generate_client_context(fhe.CKKSContextSpec(depth=3, dnum=2, seed=99,
                                                                      deterministic_encryption=det))
        ct = client.encrypt(v, cur_limbs=2)
        assert np.max(np.abs(client.decrypt(ct).real - v)) < 2.0**-20
        outs.append(ct.cv[1].cpu().numpy())
    assert not np.array_equal(outs[0], outs[1])
    assert np.array_equal(outs[2], outs[3])
