"""GPU parity: every hot-path kernel, through the C ABI, bit-exact against the CPU oracle on the
same seeded inputs at N = 2^16 (24 x 50-bit Q primes, 8 special primes, dnum 3)."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402


@pytest.fixture(scope="module")
def env():
    from holmes_amd import fhe

    spec = fhe.CKKSContextSpec(depth=23, dnum=3, dcrt_bits=50, first_mod=50, seed=20261201)
    client, ctx = fhe.generate_client_context(spec, device="cuda")
    orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
    return fhe, client, ctx, orc


def _rand(ctx, rng, batch, limbs, prime_idx=None):
    prime_idx = list(range(limbs)) if prime_idx is None else prime_idx
    a = np.stack([np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in prime_idx])
                  for _ in range(batch)])
    return a


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_prime_chain_matches_oracle_rule(env):
    _, _, ctx, _ = env
    P = O.gen_primes(16, 50, ctx.K)
    Q = O.gen_primes(16, 50, ctx.L, exclude=P)
    assert ctx.p_primes == P and ctx.q_primes == Q


def test_twiddle_tables_match_oracle(env):
    from holmes_amd import _native as nat

    _, _, ctx, orc = env
    for pi in (0, 7, ctx.L, ctx.L + ctx.K - 1):
        fwd, inv = orc.tables(pi)
        got = np.zeros(ctx.N, dtype=np.uint64)
        nat.check(nat.lib().hck_context_twiddles(ctx.handle, pi, 0, got.ctypes.data_as(nat._u64p)), "tw")
        assert np.array_equal(got, fwd)
        nat.check(nat.lib().hck_context_twiddles(ctx.handle, pi, 1, got.ctypes.data_as(nat._u64p)), "tw")
        assert np.array_equal(got, inv)


@pytest.mark.parametrize("limbs", [1, 24])
def test_ntt_forward_inverse(env, limbs):
    _, _, ctx, orc = env
    rng = np.random.default_rng(1000 + limbs)
    idx = list(range(limbs))
    x = _rand(ctx, rng, 2, limbs)
    x[0, 0, :4] = [0, 1, ctx.primes[0] - 1, ctx.primes[0] - 2]
    t = _dev(x)
    out = ctx.empty(2, limbs, ctx.N)
    ctx.ntt(t, out, prime_idx=idx)
    want = np.stack([orc.ntt_fwd_limbs(x[b], idx) for b in range(2)])
    assert np.array_equal(_host(out), want)
    ctx.ntt(out, prime_idx=idx, inverse=True)  # in place
    assert np.array_equal(_host(out), x)


def test_ntt_on_special_primes_and_strided_batches(env):
    _, _, ctx, orc = env
    rng = np.random.default_rng(77)
    idx = [ctx.L + k for k in range(ctx.K)] + [3, 5]
    x = _rand(ctx, rng, 3, len(idx), idx)
    big = ctx.zeros(3, len(idx) + 2, ctx.N)  # batch stride larger than the limb count
    big[:, : len(idx)].copy_(_dev(x))
    view = big[:, : len(idx)]
    ctx.ntt(view, prime_idx=idx)
    got = _host(big)
    want = np.stack([orc.ntt_fwd_limbs(x[b], idx) for b in range(3)])
    assert np.array_equal(got[:, : len(idx)], want)
    assert not got[:, len(idx):].any()


@pytest.mark.parametrize("g", [5, pow(5, 16, 1 << 17), pow(5, 12345, 1 << 17), (1 << 17) - 1])
def test_automorphism(env, g):
    _, _, ctx, orc = env
    rng = np.random.default_rng(g)
    x = _rand(ctx, rng, 2, 3)
    out = ctx.automorphism(_dev(x), g, 3)
    got = _host(out)
    for b in range(2):
        for i in range(3):
            assert np.array_equal(got[b, i], O.automorph_ntt(x[b, i], 16, g))


def test_automorphism_power_of_two_rotations(env):
    """sigma_g for every power-of-two rotation 2^0 .. 2^14 in both directions (the BSGS and
    bootstrap offsets) and the conjugation, against the oracle's permutation."""
    _, _, ctx, orc = env
    x = _rand(ctx, np.random.default_rng(17), 1, 1)
    gs = [ctx.galois_element(s * (1 << k)) for k in range(15) for s in (1, -1)] + [ctx.M - 1]
    for g in gs:
        got = _host(ctx.automorphism(_dev(x), g, 1))
        assert np.array_equal(got[0, 0], O.automorph_ntt(x[0, 0], 16, g)), f"g = {g}"


def test_elementwise_ops(env):
    from holmes_amd import _native as nat

    _, _, ctx, _ = env
    rng = np.random.default_rng(5)
    idx = [0, 9, ctx.L + 2]
    a = _rand(ctx, rng, 2, 3, idx)
    b = _rand(ctx, rng, 2, 3, idx)
    a[0, 0, 0], b[0, 0, 0] = ctx.primes[0] - 1, ctx.primes[0] - 1
    ta, tb = _dev(a), _dev(b)
    out = ctx.empty(2, 3, ctx.N)
    qs = np.array([ctx.primes[i] for i in idx], dtype=object).reshape(1, 3, 1)
    A, B = a.astype(object), b.astype(object)
    ctx.poly_op(nat.HCK_OP_ADD, out, ta, tb, prime_idx=idx)
    assert np.array_equal(_host(out).astype(object), (A + B) % qs)
    ctx.poly_op(nat.HCK_OP_SUB, out, ta, tb, prime_idx=idx)
    assert np.array_equal(_host(out).astype(object), (A - B) % qs)
    ctx.poly_op(nat.HCK_OP_MUL, out, ta, tb, prime_idx=idx)
    assert np.array_equal(_host(out).astype(object), (A * B) % qs)
    ctx.poly_op(nat.HCK_OP_NEG, out, ta, prime_idx=idx)
    assert np.array_equal(_host(out).astype(object), (-A) % qs)
    sc = [int(rng.integers(0, ctx.primes[i])) for i in idx]
    ctx.poly_op(nat.HCK_OP_MUL_SCALAR, out, ta, prime_idx=idx, scalar=sc)
    assert np.array_equal(_host(out).astype(object), (A * np.array(sc, dtype=object).reshape(1, 3, 1)) % qs)
    out2 = _dev(b)
    ctx.poly_op(nat.HCK_OP_MAC, out2, ta, tb, prime_idx=idx)
    assert np.array_equal(_host(out2).astype(object), (B + A * B) % qs)


def test_mul_xhalf_is_monomial_product(env):
    from holmes_amd import _native as nat

    _, _, ctx, orc = env
    rng = np.random.default_rng(8)
    x = _rand(ctx, rng, 1, 2)
    out = ctx.empty(1, 2, ctx.N)
    ctx.poly_op(nat.HCK_OP_MUL_XHALF, out, _dev(x), prime_idx=[0, 1])
    got = _host(out)
    n = ctx.N
    for i in range(2):
        q = ctx.primes[i]
        coef = orc.ntt_inv_limbs(x[0, i:i + 1], [i])[0].astype(object)
        shifted = np.concatenate([(-coef[n // 2:]) % q, coef[: n // 2]]).astype(np.uint64)  # X^(N/2) * a
        assert np.array_equal(got[0, i], orc.ntt_fwd_limbs(shifted[None], [i])[0])


def test_from_signed(env):
    _, _, ctx, _ = env
    rng = np.random.default_rng(3)
    v = rng.integers(-(2**62), 2**62, size=(2, ctx.N), dtype=np.int64)
    v[0, :3] = [0, -1, np.iinfo(np.int64).min + 1]
    idx = [0, 5, ctx.L]
    out = _host(ctx.from_signed(_dev(v), idx))
    for j, i in enumerate(idx):
        q = ctx.primes[i]
        assert np.array_equal(out[:, j].astype(object), v.astype(object) % q)


def _key_pair(client, ctx, orc, g):
    s_from, s_to, a, e = client.key_inputs(g)
    gpu_key = ctx.make_switching_key(s_from, s_to, a, e)
    return gpu_key, orc.make_ksk(s_from, s_to, a, e)


def test_switching_key_generation(env):
    _, client, ctx, orc = env
    g = ctx.galois_element(1)
    gk, ok = _key_pair(client, ctx, orc, g)
    assert np.array_equal(_host(gk), ok)


@pytest.mark.parametrize("ell", [24, 20, 13, 8, 1])
def test_keyswitch(env, ell):
    _, client, ctx, orc = env
    g = ctx.galois_element(3)
    gk, ok = _key_pair(client, ctx, orc, g)
    rng = np.random.default_rng(ell)
    d = _rand(ctx, rng, 2, ell)
    d[1, 0, :2] = [0, ctx.primes[0] - 1]
    ob, oa = ctx.keyswitch(_dev(d), ell, gk)
    gb, ga = _host(ob), _host(oa)
    for b in range(2):
        wb, wa = orc.keyswitch(ell, d[b], ok)
        assert np.array_equal(gb[b], wb), f"b component, item {b}"
        assert np.array_equal(ga[b], wa), f"a component, item {b}"


@pytest.mark.parametrize("ell", [24, 9, 1])
def test_conversion_engines_agree(env, ell):
    """The ModUp / ModDown conversion sums on the int8 matrix cores (the default) and on FP64 VALU
    give bit-identical key switches and extended-basis ModDowns, equal to the oracle's."""
    _, client, ctx, orc = env
    g = ctx.galois_element(5)
    gk, ok = _key_pair(client, ctx, orc, g)
    rng = np.random.default_rng(900 + ell)
    d = _rand(ctx, rng, 3, ell)
    d[0, 0, :4] = [0, 1, ctx.primes[0] - 1, (ctx.primes[0] - 1) // 2]
    idx = ctx.ext_prime_idx(ell)
    x = _rand(ctx, rng, 2, len(idx), idx)
    got = {}
    try:
        for engine in ("valu", "mfma"):
            ctx.set_conversion_engine(engine)
            ob, oa = ctx.keyswitch(_dev(d), ell, gk)
            got[engine] = (_host(ob), _host(oa), _host(ctx.moddown(_dev(x), ell)))
    finally:
        ctx.set_conversion_engine("mfma")
    for a, b in zip(got["valu"], got["mfma"]):
        assert np.array_equal(a, b)
    for b in range(3):
        wb, wa = orc.keyswitch(ell, d[b], ok)
        assert np.array_equal(got["mfma"][0][b], wb) and np.array_equal(got["mfma"][1][b], wa), b
    for b in range(2):
        assert np.array_equal(got["mfma"][2][b], orc.moddown(ell, x[b])), b
    with pytest.raises(ValueError):
        ctx.set_conversion_engine("fp32")


@pytest.mark.parametrize("ell,inputs,per", [(24, 3, 5), (9, 2, 3), (1, 1, 4)])
def test_hoisted_rotations_equal_rotate_many(env, ell, inputs, per):
    """Rotations from hoisted ModUp digits (one ModUp per input, read through sigma) equal the
    per-item key switch bit for bit, item i = input i % inputs, and one of them equals the oracle."""
    _, client, ctx, orc = env
    rng = np.random.default_rng(1100 + ell)
    c0, c1 = _rand(ctx, rng, inputs, ell), _rand(ctx, rng, inputs, ell)
    c1[0, 0, :3] = [0, 1, ctx.primes[0] - 1]
    steps = [1, -3, 64, 4097, (1 << 15) - 1, 7][:per]
    gals = [ctx.galois_element(r) for r in steps for _ in range(inputs)]  # offset-major, then input
    pairs = {g: _key_pair(client, ctx, orc, g) for g in set(gals)}
    keys = [pairs[g][0] for g in gals]
    d0, d1 = _dev(c0), _dev(c1)
    digits = ctx.hoist_digits(d1, ell)
    h0, h1 = ctx.rotate_hoisted(d0, d1, ell, digits, gals, keys)
    idx = torch.tensor([i % inputs for i in range(len(gals))], device=d0.device)
    r0, r1 = (x.view(torch.int64).index_select(0, idx).view(torch.uint64) for x in (d0, d1))
    w0, w1 = ctx.rotate_raw(r0, r1, ell, gals, keys)
    assert torch.equal(h0, w0) and torch.equal(h1, w1)
    g = gals[1]
    o0, o1 = orc.rotate(ell, g, c0[1 % inputs], c1[1 % inputs], pairs[g][1])
    assert np.array_equal(_host(h0)[1], o0) and np.array_equal(_host(h1)[1], o1)


def test_rotate_matches_oracle(env):
    _, client, ctx, orc = env
    ell = 24
    g = ctx.galois_element(1)
    gk, ok = _key_pair(client, ctx, orc, g)
    rng = np.random.default_rng(20261201)
    c0, c1 = _rand(ctx, rng, 1, ell), _rand(ctx, rng, 1, ell)
    o0, o1 = ctx.rotate_raw(_dev(c0), _dev(c1), ell, g, gk)
    w0, w1 = orc.rotate(ell, g, c0[0], c1[0], ok)
    assert np.array_equal(_host(o0)[0], w0)
    assert np.array_equal(_host(o1)[0], w1)
    # then rescale (config C1: rotation by 5^1, key switch, rescale)
    r0 = ctx.rescale_raw(o0, ell)
    assert np.array_equal(_host(r0)[0], orc.rescale(ell, w0))


@pytest.mark.parametrize("engine", ["mfma", "valu"])
def test_rotate_rescale_equals_rotation_then_rescale(env, engine):
    """hck_rotate_rescale (one pass on the matrix-core engine, two steps on the FP64 one) gives the
    residues of hck_rotate followed by hck_rescale at every level (batch 3, one rotation amount),
    and the oracle's rotation-then-rescale at 24, 9 and 2 limbs (config C1's unit)."""
    _, client, ctx, orc = env
    ctx.set_conversion_engine(engine)
    try:
        check_rotate_rescale((None, client, ctx, orc), range(2, ctx.L + 1), (2, 9, ctx.L))
    finally:
        ctx.set_conversion_engine("mfma")


def check_rotate_rescale(env, levels, oracle_levels, batch=3, rot=1):
    _, client, ctx, orc = env
    g = ctx.galois_element(rot)
    gk, ok = _key_pair(client, ctx, orc, g)
    for ell in levels:
        rng = np.random.default_rng(900 + ell)
        c0, c1 = _dev(_rand(ctx, rng, batch, ell)), _dev(_rand(ctx, rng, batch, ell))
        f0, f1 = ctx.rotate_rescale_raw(c0, c1, ell, g, gk)
        o0, o1 = ctx.rotate_raw(c0, c1, ell, g, gk)
        w0, w1 = ctx.rescale_raw(o0, ell), ctx.rescale_raw(o1, ell)
        assert f0.shape == (batch, ell - 1, ctx.N)
        assert torch.equal(f0, w0) and torch.equal(f1, w1), f"{ell} limbs"
        if ell in oracle_levels:
            h0, h1, hc0, hc1 = _host(f0), _host(f1), _host(c0), _host(c1)
            for b in range(batch):
                r0, r1 = orc.rotate(ell, g, hc0[b], hc1[b], ok)
                assert np.array_equal(h0[b], orc.rescale(ell, r0)), (ell, b)
                assert np.array_equal(h1[b], orc.rescale(ell, r1)), (ell, b)


@pytest.mark.parametrize("ell,rot", [(20, 128), (9, -3), (3, 4096)])
def test_rotate_accumulate_batch_matches_oracle(env, ell, rot):
    """Batched rotation with a shared key and the fused addends: out = rot(c) + acc, written over
    acc (the BSGS Horner step), against the oracle rotation followed by exact addition."""
    _, client, ctx, orc = env
    g = ctx.galois_element(rot)
    gk, ok = _key_pair(client, ctx, orc, g)
    rng = np.random.default_rng(700 + ell)
    B = 5
    c0, c1 = _rand(ctx, rng, B, ell), _rand(ctx, rng, B, ell)
    a0, a1 = _rand(ctx, rng, B, ell), _rand(ctx, rng, B, ell)
    acc0, acc1 = _dev(a0), _dev(a1)
    o0, o1 = ctx.rotate_raw(_dev(c0), _dev(c1), ell, g, gk, out0=acc0, out1=acc1, acc=(acc0, acc1))
    assert o0.data_ptr() == acc0.data_ptr()
    h0, h1 = _host(o0), _host(o1)
    q = np.array(ctx.primes[:ell], dtype=object).reshape(ell, 1)
    for b in range(B):
        w0, w1 = orc.rotate(ell, g, c0[b], c1[b], ok)
        e0 = ((w0.astype(object) + a0[b].astype(object)) % q).astype(np.uint64)
        e1 = ((w1.astype(object) + a1[b].astype(object)) % q).astype(np.uint64)
        assert np.array_equal(h0[b], e0), f"b component, item {b}"
        assert np.array_equal(h1[b], e1), f"a component, item {b}"
    # plain batched rotation with the same key, no addends
    p0, p1 = ctx.rotate_raw(_dev(c0), _dev(c1), ell, g, gk)
    w0, w1 = orc.rotate(ell, g, c0[B - 1], c1[B - 1], ok)
    assert np.array_equal(_host(p0)[B - 1], w0) and np.array_equal(_host(p1)[B - 1], w1)


def test_rotate_rejects_aliased_output(env):
    _, client, ctx, orc = env
    from holmes_amd import _native as nat

    g = ctx.galois_element(1)
    gk, _ = _key_pair(client, ctx, orc, g)
    rng = np.random.default_rng(9)
    c0, c1 = _dev(_rand(ctx, rng, 1, 4)), _dev(_rand(ctx, rng, 1, 4))
    with pytest.raises(nat.NativeError):
        ctx.rotate_raw(c0, c1, 4, g, gk, out0=c0)


@pytest.mark.parametrize("ell", [24, 2])
def test_rescale(env, ell):
    _, _, ctx, orc = env
    rng = np.random.default_rng(40 + ell)
    x = _rand(ctx, rng, 3, ell)
    out = _host(ctx.rescale_raw(_dev(x), ell))
    for b in range(3):
        assert np.array_equal(out[b], orc.rescale(ell, x[b]))


def test_rescale_in_place_and_rejected_overlaps(env):
    """In place with equal strides is exact; an out buffer that overlaps the input at another
    stride, or strides below one poly, is an argument error (nothing launched), and a short out
    tensor is refused on the host."""
    from holmes_amd import _native as nat

    _, _, ctx, orc = env
    ell, polys = 6, 3
    rng = np.random.default_rng(46)
    x = _rand(ctx, rng, polys, ell)
    buf = _dev(x)
    want = [orc.rescale(ell, x[b]) for b in range(polys)]
    got = _host(ctx.rescale_raw(buf, ell, out=buf))  # same strides: in place
    for b in range(polys):
        assert np.array_equal(got[b, :ell - 1], want[b])
    L = nat.lib()
    n = ctx.N
    ws = ctx.workspace(L.hck_rescale_workspace_bytes(ctx.handle, ell, polys))
    base = buf.data_ptr()
    stream = torch.cuda.current_stream().cuda_stream
    # out packed at (ell - 1) limbs per poly over an input with ell limbs per poly: overlapping
    assert L.hck_rescale(ctx.handle, ell, polys, base, ell * n, base, (ell - 1) * n, ws.data_ptr(), ws.numel(),
                         stream) == nat.HCK_ERR_ARG
    other = ctx.empty(polys, ell, n)
    assert L.hck_rescale(ctx.handle, ell, polys, base, (ell - 1) * n, other.data_ptr(), ell * n, ws.data_ptr(),
                         ws.numel(), stream) == nat.HCK_ERR_ARG  # input stride below one poly
    with pytest.raises(ValueError):
        ctx.rescale_raw(buf, ell, out=ctx.empty(polys - 1, ell - 1, n))


def test_rotate_rescale_rejects_overlapping_outputs(env):
    """hck_rotate_rescale refuses outputs that share words with c0, c1 or each other at any offset
    (the fused pass reads c0 through the automorphism while other tiles store): HCK_ERR_ARG, nothing
    launched."""
    from holmes_amd import _native as nat

    _, client, ctx, orc = env
    ell, n = 4, ctx.N
    g = ctx.galois_element(3)
    gk, _ = _key_pair(client, ctx, orc, g)
    rng = np.random.default_rng(47)
    c0, c1 = _dev(_rand(ctx, rng, 1, ell)), _dev(_rand(ctx, rng, 1, ell))
    free0, free1 = ctx.empty(1, ell - 1, n), ctx.empty(1, ell - 1, n)
    L = nat.lib()
    ws = ctx.workspace(L.hck_rotate_rescale_workspace_bytes(ctx.handle, ell, 1))
    keys = nat.ptr_array([gk.data_ptr()])
    stream = torch.cuda.current_stream().cuda_stream

    def call(o0, o1):
        return L.hck_rotate_rescale(ctx.handle, ell, 1, g, c0.data_ptr(), c1.data_ptr(), ell * n, keys, o0, o1,
                                    (ell - 1) * n, ws.data_ptr(), ws.numel(), stream)

    assert call(c0.data_ptr() + 8 * n, free1.data_ptr()) == nat.HCK_ERR_ARG  # out0 one limb into c0
    assert call(free0.data_ptr(), c1.data_ptr() + 8 * n) == nat.HCK_ERR_ARG  # out1 one limb into c1
    assert call(free0.data_ptr(), free0.data_ptr() + 8 * n) == nat.HCK_ERR_ARG  # out1 inside out0
    assert call(free0.data_ptr(), free1.data_ptr()) == 0
    torch.cuda.synchronize()


def test_batched_keyswitch_sixteen_keys(env):
    """Config C2 shape: 16 ciphertexts at 24 limbs, 16 distinct rotation keys (steps 1..16)."""

    _, client, ctx, orc = env
    ell = 24
    keys_gpu, keys_orc = [], []
    for r in range(1, 17):
        g = ctx.galois_element(r)
        gk, ok = _key_pair(client, ctx, orc, g)
        keys_gpu.append(gk)
        keys_orc.append(ok)
    rng = np.random.default_rng(20261202)
    d = _rand(ctx, rng, 16, ell)
    ob, oa = ctx.keyswitch(_dev(d), ell, keys_gpu)
    wb, wa = orc.keyswitch_batch(ell, d, keys_orc)
    assert np.array_equal(_host(ob), wb)
    assert np.array_equal(_host(oa), wa)


@pytest.mark.parametrize("to", [24, 2])
def test_modraise(env, to):
    _, _, ctx, orc = env
    rng = np.random.default_rng(60 + to)
    x = _rand(ctx, rng, 3, 1)
    out = _host(ctx.modraise(_dev(x), to))
    for b in range(3):
        assert np.array_equal(out[b], orc.modraise(to, x[b]))


@pytest.mark.parametrize("ell", [24, 7])
def test_rotate_many_matches_oracle(env, ell):
    """Rotations by different amounts in one launch (a Galois element and a key per item), with and
    without the fused addends, against the oracle's rotation of each item; then one input rotated by
    every element (batch stride 0)."""
    _, client, ctx, orc = env
    gs = [ctx.galois_element(1), ctx.galois_element(-512), ctx.M - 1, ctx.galois_element(4096)]
    pairs = [_key_pair(client, ctx, orc, g) for g in gs]
    rng = np.random.default_rng(900 + ell)
    B = len(gs)
    c0, c1 = _rand(ctx, rng, B, ell), _rand(ctx, rng, B, ell)
    a0, a1 = _rand(ctx, rng, B, ell), _rand(ctx, rng, B, ell)
    o0, o1 = ctx.rotate_raw(_dev(c0), _dev(c1), ell, gs, [p[0] for p in pairs])
    h0, h1 = _host(o0), _host(o1)
    q = np.array(ctx.primes[:ell], dtype=object).reshape(ell, 1)
    want = [orc.rotate(ell, g, c0[b], c1[b], pairs[b][1]) for b, g in enumerate(gs)]
    for b in range(B):
        assert np.array_equal(h0[b], want[b][0]) and np.array_equal(h1[b], want[b][1]), f"item {b}"
    acc0, acc1 = _dev(a0), _dev(a1)
    ctx.rotate_raw(_dev(c0), _dev(c1), ell, gs, [p[0] for p in pairs], out0=acc0, out1=acc1, acc=(acc0, acc1))
    h0, h1 = _host(acc0), _host(acc1)
    for b in range(B):
        e0 = ((want[b][0].astype(object) + a0[b].astype(object)) % q).astype(np.uint64)
        e1 = ((want[b][1].astype(object) + a1[b].astype(object)) % q).astype(np.uint64)
        assert np.array_equal(h0[b], e0) and np.array_equal(h1[b], e1), f"accumulated item {b}"
    one0, one1 = _dev(c0[:1]), _dev(c1[:1])
    s0, s1 = ctx.rotate_raw(one0.expand(B, -1, -1), one1.expand(B, -1, -1), ell, gs, [p[0] for p in pairs])
    h0, h1 = _host(s0), _host(s1)
    for b, g in enumerate(gs):
        w0, w1 = orc.rotate(ell, g, c0[0], c1[0], pairs[b][1])
        assert np.array_equal(h0[b], w0) and np.array_equal(h1[b], w1), f"broadcast item {b}"


def test_rotate_ext_many_equals_single_rotations(env):
    _, client, ctx, orc = env
    ell = 10
    gs = [ctx.galois_element(3), ctx.galois_element(-1), ctx.galois_element(77)]
    keys = [_key_pair(client, ctx, orc, g)[0] for g in gs]
    rng = np.random.default_rng(31)
    c0, c1 = _dev(_rand(ctx, rng, 3, ell)), _dev(_rand(ctx, rng, 3, ell))
    m0, m1 = ctx.rotate_ext(c0, c1, ell, gs, keys)
    for b, g in enumerate(gs):
        s0, s1 = ctx.rotate_ext(c0[b:b + 1], c1[b:b + 1], ell, g, keys[b])
        assert torch.equal(m0[b:b + 1], s0) and torch.equal(m1[b:b + 1], s1), f"item {b}"
    from holmes_amd import _native as nat

    with pytest.raises(ValueError):
        ctx.rotate_raw(c0, c1, ell, gs[:2], keys)
    with pytest.raises(nat.NativeError):
        ctx.rotate_raw(c0, c1, ell, [gs[0], 4, gs[2]], keys)  # an even Galois element


def test_batches_spanning_launches(env):
    """66 items, more than one launch holds (64): a key switch and a rotation with a Galois
    element per item, every item against the oracle, items 64 and 65 in the second launch."""
    _, client, ctx, orc = env
    ell, B = 2, 66
    gs = [ctx.galois_element(1), ctx.galois_element(-7), ctx.M - 1]
    pairs = [_key_pair(client, ctx, orc, g) for g in gs]
    rng = np.random.default_rng(66)
    d = _rand(ctx, rng, B, ell)
    ob, oa = ctx.keyswitch(_dev(d), ell, [pairs[b % 3][0] for b in range(B)])
    gb, ga = _host(ob), _host(oa)
    for b in range(B):
        wb, wa = orc.keyswitch(ell, d[b], pairs[b % 3][1])
        assert np.array_equal(gb[b], wb) and np.array_equal(ga[b], wa), f"key switch item {b}"
    c0, c1 = _rand(ctx, rng, B, ell), _rand(ctx, rng, B, ell)
    o0, o1 = ctx.rotate_raw(_dev(c0), _dev(c1), ell, [gs[b % 3] for b in range(B)],
                            [pairs[b % 3][0] for b in range(B)])
    h0, h1 = _host(o0), _host(o1)
    for b in range(B):
        w0, w1 = orc.rotate(ell, gs[b % 3], c0[b], c1[b], pairs[b % 3][1])
        assert np.array_equal(h0[b], w0) and np.array_equal(h1[b], w1), f"rotation item {b}"


def test_empty_batch_is_a_no_op(env):
    """batch 0 returns success through the C ABI and writes nothing."""
    from holmes_amd import _native as nat

    _, client, ctx, orc = env
    gk, _ = _key_pair(client, ctx, orc, ctx.galois_element(1))
    d = _dev(_rand(ctx, np.random.default_rng(0), 1, 2))
    out_b = torch.full((1, 2, ctx.N), 7, dtype=torch.int64, device="cuda").view(torch.uint64)
    out_a = torch.full((1, 2, ctx.N), 9, dtype=torch.int64, device="cuda").view(torch.uint64)
    L = nat.lib()
    ws = ctx.workspace(L.hck_keyswitch_workspace_bytes(ctx.handle, 2, 1))
    rc = L.hck_keyswitch(ctx.handle, 2, 0, d.data_ptr(), 2 * ctx.N, nat.ptr_array([gk.data_ptr()]), None, 0,
                         out_b.data_ptr(), out_a.data_ptr(), 2 * ctx.N, ws.data_ptr(), ws.numel(), None)
    assert rc == 0
    torch.cuda.synchronize()
    assert bool((out_b.view(torch.int64) == 7).all()) and bool((out_a.view(torch.int64) == 9).all())


def test_every_level_keyswitch_and_rescale(env):
    """The per-level tables (ModUp digits, ModDown, rescale and ModRaise conversions, P^-1 and
    q_last^-1 factors) at every level: a key switch at each ell = 1 .. L, a rescale and a ModRaise
    to each ell = 2 .. L, against the oracle."""
    _, client, ctx, orc = env
    gk, ok = _key_pair(client, ctx, orc, ctx.galois_element(5))
    for ell in range(1, ctx.L + 1):
        rng = np.random.default_rng(7000 + ell)
        d = _rand(ctx, rng, 1, ell)
        ob, oa = ctx.keyswitch(_dev(d), ell, gk)
        wb, wa = orc.keyswitch(ell, d[0], ok)
        assert np.array_equal(_host(ob)[0], wb) and np.array_equal(_host(oa)[0], wa), f"key switch at {ell} limbs"
        if ell >= 2:
            x = _rand(ctx, rng, 2, ell)
            got = _host(ctx.rescale_raw(_dev(x), ell))
            for b in range(2):
                assert np.array_equal(got[b], orc.rescale(ell, x[b])), f"rescale at {ell} limbs, item {b}"
            y = _rand(ctx, rng, 1, 1)
            assert np.array_equal(_host(ctx.modraise(_dev(y), ell))[0], orc.modraise(ell, y[0])), f"ModRaise to {ell}"


@pytest.mark.parametrize("ell,outputs,group", [(20, 5, 3), (9, 16, 4), (24, 1, 2)])
def test_grouped_ext_rotations_equal_sequential(env, ell, outputs, group):
    """hck_rotate_ext_sum (a group of giant steps summed on chip, one accumulator pass) against
    `group` accumulating hck_rotate_ext calls, and its ModDown against the oracle's rotations."""
    _, client, ctx, orc = env
    rots = [1, -17, 4096, 333][:group]
    gs = [ctx.galois_element(r) for r in rots]
    pairs = [_key_pair(client, ctx, orc, g) for g in gs]
    rng = np.random.default_rng(1000 * ell + outputs)
    c0 = _rand(ctx, rng, group * outputs, ell).reshape(group, outputs, ell, ctx.N)
    c1 = _rand(ctx, rng, group * outputs, ell).reshape(group, outputs, ell, ctx.N)
    idx = ctx.ext_prime_idx(ell)
    a0, a1 = _rand(ctx, rng, outputs, len(idx), idx), _rand(ctx, rng, outputs, len(idx), idx)
    s0, s1 = _dev(a0), _dev(a1)
    for m in range(group):
        ctx.rotate_ext(_dev(c0[m]), _dev(c1[m]), ell, gs[m], pairs[m][0], out0=s0, out1=s1, acc=(s0, s1))
    g0, g1 = _dev(a0), _dev(a1)
    ctx.rotate_ext_sum(_dev(c0), _dev(c1), ell, gs, [p[0] for p in pairs], g0, g1, acc=(g0, g1))
    assert np.array_equal(_host(g0), _host(s0)) and np.array_equal(_host(g1), _host(s1))
    # no accumulator: the first member starts the sum (ModDown of a sum rounds once, so it is pinned
    # through the sequential rotate_ext, whose ModDown equals the oracle's rotation bit for bit)
    e0, e1 = ctx.empty(outputs, len(idx), ctx.N), ctx.empty(outputs, len(idx), ctx.N)
    ctx.rotate_ext_sum(_dev(c0), _dev(c1), ell, gs, [p[0] for p in pairs], e0, e1)
    r0, r1 = ctx.rotate_ext(_dev(c0[0]), _dev(c1[0]), ell, gs[0], pairs[0][0])
    for m in range(1, group):
        ctx.rotate_ext(_dev(c0[m]), _dev(c1[m]), ell, gs[m], pairs[m][0], out0=r0, out1=r1, acc=(r0, r1))
    assert np.array_equal(_host(e0), _host(r0)) and np.array_equal(_host(e1), _host(r1))
    w0, w1 = orc.rotate(ell, gs[0], c0[0, 0], c1[0, 0], pairs[0][1])
    one0, one1 = ctx.rotate_ext(_dev(c0[0, :1]), _dev(c1[0, :1]), ell, gs[0], pairs[0][0])
    assert np.array_equal(_host(ctx.moddown(one0, ell))[0], w0)
