"""GPU parity on the wide-prime path: the reference's production chain structure
(assets/feature_major.json: N = 2^16, 38 Q limbs -- q_0 of 60 bits, the other 37 of 59 bits -- dnum
5, 8 special primes of 60 bits), every kernel through the C ABI bit-exact against the CPU oracle
(exact 128-bit arithmetic for any prime below 2^62): NTT, automorphism, elementwise ops, key
generation, key switch at 38, 19 and 8 limbs (base conversion on either engine), rotation with and without addends, hoisted rotations,
the extended-basis
rotation and ModDown, rescale, ModRaise, tensor and relinearisation, the rotation and the product
with their ModDown fused into the rescale (against the unfused pair and the oracle), the BSGS MAC and the encoder
for coefficients up to 2^61.  Several checks are the FP64 path's own test bodies, run here on the
wide context."""

import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402

from . import test_gpu_bsgs as B  # noqa: E402
from . import test_gpu_mul as M  # noqa: E402
from . import test_gpu_parity as G  # noqa: E402
from .test_gpu_parity import _dev, _host, _key_pair, _rand  # noqa: E402

SEED = 20261207


@pytest.fixture(scope="module")
def env():
    from holmes_amd import fhe

    spec = fhe.CKKSContextSpec(depth=37, dnum=5, dcrt_bits=59, first_mod=60, scale_bits=59,
                               secret_key_dist="SPARSE_TERNARY", hamming_weight=192, seed=SEED)
    print("wide context: 38 Q limbs (60/59-bit), dnum 5, 8 special primes", flush=True)
    client, ctx = fhe.generate_client_context(spec, device="cuda")
    orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
    return fhe, client, ctx, orc


def test_chain_is_the_reference_structure(env):
    _, _, ctx, _ = env
    assert ctx.L == 38 and ctx.K == 8 and ctx.alpha == 8 and ctx.beta_max == 5
    assert ctx.q_primes[0].bit_length() == 60 and all(q.bit_length() == 59 for q in ctx.q_primes[1:])
    assert all(p.bit_length() == 60 for p in ctx.p_primes)
    P = O.gen_primes(16, 60, 8)
    q0 = O.gen_primes(16, 60, 1, exclude=P)
    assert ctx.p_primes == P and ctx.q_primes == q0 + O.gen_primes(16, 59, 37, exclude=P + q0)


def test_twiddles(env):
    G.test_twiddle_tables_match_oracle(env)


@pytest.mark.parametrize("limbs", [1, 38])
def test_ntt_forward_inverse(env, limbs):
    G.test_ntt_forward_inverse(env, limbs)


def test_ntt_special_primes_strided(env):
    G.test_ntt_on_special_primes_and_strided_batches(env)


@pytest.mark.parametrize("g", [5, pow(5, 12345, 1 << 17), (1 << 17) - 1])
def test_automorphism(env, g):
    G.test_automorphism(env, g)


def test_elementwise_ops(env):
    G.test_elementwise_ops(env)


def test_mul_xhalf(env):
    G.test_mul_xhalf_is_monomial_product(env)


def test_from_signed(env):
    G.test_from_signed(env)


def test_switching_key_generation(env):
    G.test_switching_key_generation(env)


@pytest.mark.parametrize("ell", [38, 19, 8])
def test_keyswitch(env, ell):
    print(f"wide key switch at {ell} limbs", flush=True)
    G.test_keyswitch(env, ell)


@pytest.mark.parametrize("ell", [38, 9, 1])
def test_conversion_engines_agree(env, ell):
    """The wide base conversion on the int8 matrix cores (the default: eight balanced base-256 digits
    per source, a 128-bit-free fold) and on the VALU (64-bit products, one Montgomery reduction) give
    bit-identical key switches and ModDowns, equal to the oracle's."""
    G.test_conversion_engines_agree(env, ell)


def test_rotate_and_rescale(env):
    _, client, ctx, orc = env
    ell = 38
    g = ctx.galois_element(1)
    gk, ok = _key_pair(client, ctx, orc, g)
    rng = np.random.default_rng(SEED)
    c0, c1 = _rand(ctx, rng, 1, ell), _rand(ctx, rng, 1, ell)
    c1[0, 0, :2] = [0, ctx.primes[0] - 1]
    o0, o1 = ctx.rotate_raw(_dev(c0), _dev(c1), ell, g, gk)
    w0, w1 = orc.rotate(ell, g, c0[0], c1[0], ok)
    assert np.array_equal(_host(o0)[0], w0) and np.array_equal(_host(o1)[0], w1)
    assert np.array_equal(_host(ctx.rescale_raw(o0, ell))[0], orc.rescale(ell, w0))


@pytest.mark.parametrize("ell,rot", [(19, 128), (3, -3)])
def test_rotate_accumulate_batch(env, ell, rot):
    G.test_rotate_accumulate_batch_matches_oracle(env, ell, rot)


@pytest.mark.parametrize("ell,inputs,per", [(38, 3, 4), (11, 2, 3), (1, 1, 2)])
def test_hoisted_rotations(env, ell, inputs, per):
    """Hoisted rotations on the wide path (one ModUp per input, the digits read through sigma in
    the inner product): bit-identical to the per-item key switch and to the oracle."""
    G.test_hoisted_rotations_equal_rotate_many(env, ell, inputs, per)


@pytest.mark.parametrize("ell", [38, 7])
def test_rotate_many(env, ell):
    G.test_rotate_many_matches_oracle(env, ell)


@pytest.mark.parametrize("ell", [38, 19, 2])
def test_rescale(env, ell):
    G.test_rescale(env, ell)


def test_rescale_in_place(env):
    G.test_rescale_in_place_and_rejected_overlaps(env)


@pytest.mark.parametrize("to", [38, 2])
def test_modraise(env, to):
    G.test_modraise(env, to)


def test_rotate_ext_then_moddown_equals_rotate(env):
    """The extended-basis rotation (P sigma(c0) + IP(sigma(c1)), no ModDown) followed by ModDown is the
    rotation bit for bit, and ModDown of random extended polynomials matches the oracle."""
    _, client, ctx, orc = env
    ell = 12
    g = ctx.galois_element(7)
    gk, ok = _key_pair(client, ctx, orc, g)
    rng = np.random.default_rng(SEED + 1)
    c0, c1 = _rand(ctx, rng, 2, ell), _rand(ctx, rng, 2, ell)
    e0, e1 = ctx.rotate_ext(_dev(c0), _dev(c1), ell, g, gk)
    d0, d1 = ctx.moddown(e0, ell), ctx.moddown(e1, ell)
    for b in range(2):
        w0, w1 = orc.rotate(ell, g, c0[b], c1[b], ok)
        assert np.array_equal(_host(d0)[b], w0) and np.array_equal(_host(d1)[b], w1), b
    idx = ctx.ext_prime_idx(ell)
    x = _rand(ctx, rng, 2, len(idx), idx)
    got = _host(ctx.moddown(_dev(x), ell))
    for b in range(2):
        assert np.array_equal(got[b], orc.moddown(ell, x[b])), b


@pytest.mark.parametrize("ell", [38, 9, 1])
def test_tensor(env, ell):
    M.test_tensor_bit_exact(env, ell)


def test_relin_key(env):
    M.test_relin_key_matches_oracle(env)


@pytest.mark.parametrize("ell", [38, 19, 2])
def test_mul_relin(env, ell):
    M.test_mul_relin_bit_exact(env, ell)


@pytest.mark.parametrize("ell", [38, 25, 2])
def test_rotate_rescale(env, ell):
    G.check_rotate_rescale(env, [ell], [ell], batch=2, rot=5)


def test_mul_relin_rescale_postop(env):
    M.check_mul_relin_rescale_postop(env, (38, 26, 2), batch=2)


@pytest.mark.parametrize("ell", [38, 25, 2])
def test_mul_relin_rescale(env, ell):
    M.check_mul_relin_rescale(env, [ell], [ell], batch=2)


def test_unfused_fallbacks_on_the_valu_engine(env):
    """With the VALU conversion engine the wide context has no fused kernels (wide_fused_ok is false,
    as on a chain with a prime at or above 2^60): the rotation and the product with their rescale run
    as two steps and grouped giant steps one member at a time.  Same residues as the oracle."""
    fhe, client, ctx, orc = env
    ctx.set_conversion_engine("valu")
    try:
        G.check_rotate_rescale(env, [38, 2], [38, 2], batch=2, rot=3)
        M.check_mul_relin_rescale(env, [9, 2], [9, 2], batch=2)
        G.test_grouped_ext_rotations_equal_sequential(env, 9, 3, 2)
    finally:
        ctx.set_conversion_engine("mfma")


def test_lincomb(env):
    M.test_lincomb_matches_oracle(env)


@pytest.mark.parametrize("limbs,G,T", [(38, 3, 5), (2, 2, 1), (24, 64, 1)])
def test_lincomb_rescale(env, limbs, G, T):
    M.check_lincomb_rescale(env, limbs, G, T)


@pytest.mark.parametrize("ni,nb,G_,limbs", [(3, 5, 6, 2), (2, 3, 2, 38), (5, 64, 2, 1), (4, 15, 9, 3), (2, 14, 4, 2)])
def test_bsgs_mac(env, ni, nb, G_, limbs):
    _, _, ctx, orc = env
    B.test_bsgs_mac((ctx, orc), ni, nb, G_, limbs)


def test_bsgs_mac_on_primes_above_2_60():
    """A context whose primes lie in [2^60, 2^61) (reachable through the C ABI; the Python spec stops
    at 60 bits) runs the 128-bit MAC, since the split MAC needs every prime below 2^60: bit-exact
    against the oracle over several folds, odd counts and clamped tiles."""
    import ctypes

    from holmes_amd import _native as nat
    from holmes_amd.params import ntt_primes

    primes = ntt_primes(16, 61, 3)  # two Q primes, one special prime
    assert all(p >= 1 << 60 for p in primes)
    L = nat.lib()
    h = ctypes.c_void_p()
    nat.check(L.hck_context_create(ctypes.byref(h), 16, 2, 1, 1, nat.u64_array(primes)), "hck_context_create")
    try:
        orc = O.OracleContext(16, 2, 1, 1, primes)
        ni, nb, G, limbs = 3, 11, 5, 2
        n = 1 << 16
        rng = np.random.default_rng(61)
        q = np.array(primes[:limbs], dtype=np.uint64).reshape(1, limbs, 1)
        pts = rng.integers(0, 2**62, size=(G * nb, limbs, n), dtype=np.uint64) % q
        babies = rng.integers(0, 2**62, size=(nb, 2, ni, limbs, n), dtype=np.uint64) % q.reshape(1, 1, 1, limbs, 1)
        pts[0, 0, :3] = primes[0] - 1
        babies[0, :, 0, 0, :3] = primes[0] - 1
        bt = torch.from_numpy(babies).cuda()
        pt = torch.from_numpy(pts).cuda()
        res = torch.empty((2, G, ni, limbs, n), dtype=torch.uint64, device="cuda")
        c0 = [bt[b, 0] for b in range(nb)]
        c1 = [bt[b, 1] for b in range(nb)]
        rc = L.hck_bsgs_mac(h, limbs, nat.int_array([0, 1]), ni, nb, G, nat.ptr_array([t.data_ptr() for t in c0]),
                            nat.ptr_array([t.data_ptr() for t in c1]), limbs * n, pt.data_ptr(), limbs * n,
                            res.data_ptr(), torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        got = _host(res)
        for i in range(ni):
            want = orc.bsgs_mac(limbs, nb, G, pts, np.ascontiguousarray(babies[:, :, i]))
            assert np.array_equal(got[:, :, i], want), f"input {i}"
    finally:
        torch.cuda.synchronize()
        L.hck_context_destroy(h)


@pytest.mark.parametrize("scale", [2.0**40, None])
def test_encode(env, scale):
    _, _, ctx, orc = env
    B.test_encode_real_bit_exact((ctx, orc), scale)


def test_encode_coefficients_up_to_2_61(env):
    """|v Delta| in [2^52, 2^61): residues equal the oracle's (a coefficient near 2^60 exceeds the
    59-bit primes, so the reduction is exercised), and 2^61 itself is refused."""
    _, _, ctx, orc = env
    B.test_encode_large_coefficients_bit_exact((ctx, orc))
    B.test_encode_overflow_is_reported((ctx, orc))


def test_encrypt_rotate_decrypt(env):
    """End to end on the wide chain at scale 2^59: encrypt, rotate by 3 (key switch at 38 limbs),
    multiply by a plaintext constant and rescale; the decrypted slots are the rotated products."""
    fhe, client, ctx, _ = env
    client.generate_rotation_keys([3])
    rng = np.random.default_rng(SEED + 2)
    x = rng.uniform(-1, 1, ctx.max_slots)
    ct = client.encrypt(x, cur_limbs=ctx.L, scaling_factor=2.0**59)
    r = fhe.homo_rotate(ct, 3, ctx)
    got = client.decrypt(r).real
    err = float(np.max(np.abs(got - np.roll(x, -3))))
    print(f"wide rotation: decrypted error 2^{math.log2(err):.1f}", flush=True)
    assert err < 2.0**-30
    sq = fhe.rescale(fhe.homo_mul_relin(r, r, ctx), ctx)
    err2 = float(np.max(np.abs(client.decrypt(sq).real - np.roll(x, -3) ** 2)))
    print(f"wide product + rescale: decrypted error 2^{math.log2(err2):.1f}", flush=True)
    assert err2 < 2.0**-30


@pytest.mark.parametrize("ell,outputs,group", [(19, 5, 3), (38, 4, 4), (3, 1, 2)])
def test_grouped_ext_rotations(env, ell, outputs, group):
    G.test_grouped_ext_rotations_equal_sequential(env, ell, outputs, group)
