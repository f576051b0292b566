"""GPU parity of the ciphertext product and the scalar surface (N = 2^16, 24 x 50-bit primes,
8 special primes, dnum 3), through the C ABI:

* bit-exact against the CPU oracle: the tensor product, the relinearisation key, the product with
  relinearisation, the grouped scalar-weighted sum;
* the secret's square (the relinearisation key's source) against the oracle's independent NTT;
* the reference's own residue check of the fused weighted sum: it must equal the loop of scalar
  products and additions residue for residue (llama3fhe/operators/nonlinear/polynomial.py:33-44,
  _FUSED_WSUM_CHECK);
* decrypted semantics within 2^-16: products, the Chebyshev step 2 T_a T_b - T_c of
  homo_mul_relin_rescale_postop, scalar multiply / add (double and integer modes), plaintext add.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402

TOL = 2.0**-16


@pytest.fixture(scope="module")
def env():
    from holmes_amd import fhe

    spec = fhe.CKKSContextSpec(depth=23, dnum=3, dcrt_bits=50, first_mod=50, seed=20261211)
    client, ctx = fhe.generate_client_context(spec, device="cuda")
    orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
    return fhe, client, ctx, orc


@pytest.fixture(scope="module")
def fixed_env():
    """A fixed-scale context (scale 2^50 = the prime size) for chains of products."""

    from holmes_amd import fhe

    spec = fhe.CKKSContextSpec(depth=7, dnum=2, dcrt_bits=50, first_mod=50, scale_bits=50, seed=20261212)
    client, ctx = fhe.generate_client_context(spec, device="cuda")
    orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
    return fhe, client, ctx, orc


def _rand(ctx, rng, batch, limbs):
    return np.stack([np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in range(limbs)])
                     for _ in range(batch)])


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_secret_square_matches_oracle_ntt(env):
    fhe, client, ctx, orc = env
    sq = client.secret_square()
    q = ctx.primes[0]
    s = np.asarray([[int(v) % q for v in client.secret]], dtype=np.uint64)
    sn = orc.ntt_fwd_limbs(s, [0])
    prod = (sn[0].astype(object) * sn[0].astype(object)) % q
    back = orc.ntt_inv_limbs(np.asarray([prod], dtype=np.uint64), [0])[0].astype(np.int64)
    want = np.where(back > q // 2, back - q, back)
    assert np.array_equal(sq, want)
    nz = int(np.count_nonzero(client.secret))
    assert int(np.max(np.abs(sq))) <= nz


def test_relin_key_matches_oracle(env):
    fhe, client, ctx, orc = env
    want = orc.make_ksk(*client.relin_key_inputs())
    assert np.array_equal(_host(ctx.relin_key), want)


@pytest.mark.parametrize("ell", [24, 7, 1])
def test_tensor_bit_exact(env, ell):
    fhe, client, ctx, orc = env
    rng = np.random.default_rng(ell)
    a0, a1, b0, b1 = (_rand(ctx, rng, 2, ell) for _ in range(4))
    # edge residues: 0 and q - 1 in the first coefficients
    for t in (a0, a1, b0, b1):
        t[:, :, 0] = 0
        for i in range(ell):
            t[:, i, 1] = ctx.primes[i] - 1
    d = ctx.tensor(*(_dev(x) for x in (a0, a1, b0, b1)), ell)
    for b in range(2):
        want = orc.tensor(ell, a0[b], a1[b], b0[b], b1[b])
        for c in range(3):
            assert np.array_equal(_host(d[c])[b], want[c]), (b, c)


@pytest.mark.parametrize("ell", [24, 9, 2])
def test_mul_relin_bit_exact(env, ell):
    fhe, client, ctx, orc = env
    rng = np.random.default_rng(100 + ell)
    a0, a1, b0, b1 = (_rand(ctx, rng, 2, ell) for _ in range(4))
    rlk = orc.make_ksk(*client.relin_key_inputs())
    o0, o1 = ctx.mul_relin_raw(*(_dev(x) for x in (a0, a1, b0, b1)), ell, ctx.relin_key)
    h0, h1 = _host(o0), _host(o1)
    for b in range(2):
        w0, w1 = orc.mul_relin(ell, a0[b], a1[b], b0[b], b1[b], rlk)
        assert np.array_equal(h0[b], w0) and np.array_equal(h1[b], w1), b


def test_mul_relin_every_level(env):
    """The product with relinearisation at every level ell = 1 .. L (one item each) against the
    oracle: every level's ModUp digits and ModDown factors under the relinearisation key."""
    fhe, client, ctx, orc = env
    rlk = orc.make_ksk(*client.relin_key_inputs())
    for ell in range(1, ctx.L + 1):
        rng = np.random.default_rng(300 + ell)
        a0, a1, b0, b1 = (_rand(ctx, rng, 1, ell) for _ in range(4))
        o0, o1 = ctx.mul_relin_raw(*(_dev(x) for x in (a0, a1, b0, b1)), ell, ctx.relin_key)
        w0, w1 = orc.mul_relin(ell, a0[0], a1[0], b0[0], b1[0], rlk)
        assert np.array_equal(_host(o0)[0], w0) and np.array_equal(_host(o1)[0], w1), f"{ell} limbs"


@pytest.mark.parametrize("engine", ["mfma", "valu"])
def test_mul_relin_rescale_equals_product_then_rescale(env, engine):
    """hck_mul_relin_rescale (the ModDown fused with the rescale on the matrix-core engine, the two
    steps on the FP64 one) gives the residues of hck_mul_relin followed by hck_rescale at every
    level, batch 3, and the oracle's product-then-rescale at three levels."""
    _, _, ctx, _ = env
    ctx.set_conversion_engine(engine)
    try:
        check_mul_relin_rescale(env, range(2, ctx.L + 1), (2, 9, ctx.L))
    finally:
        ctx.set_conversion_engine("mfma")


def check_mul_relin_rescale(env, levels, oracle_levels, batch=3):
    fhe, client, ctx, orc = env
    rlk = orc.make_ksk(*client.relin_key_inputs())
    for ell in levels:
        rng = np.random.default_rng(700 + ell)
        a0, a1, b0, b1 = (_dev(_rand(ctx, rng, batch, ell)) for _ in range(4))
        f0, f1 = ctx.mul_relin_rescale_raw(a0, a1, b0, b1, ell, ctx.relin_key)
        p0, p1 = ctx.mul_relin_raw(a0, a1, b0, b1, ell, ctx.relin_key)
        w0, w1 = ctx.rescale_raw(p0, ell), ctx.rescale_raw(p1, ell)
        assert f0.shape == (batch, ell - 1, ctx.N)
        assert torch.equal(f0, w0) and torch.equal(f1, w1), f"{ell} limbs"
        if ell in oracle_levels:
            h0, h1 = _host(f0), _host(f1)
            for b in range(batch):
                m0, m1 = orc.mul_relin(ell, *(_host(x)[b] for x in (a0, a1, b0, b1)), rlk)
                assert np.array_equal(h0[b], orc.rescale(ell, m0)), (ell, b)
                assert np.array_equal(h1[b], orc.rescale(ell, m1)), (ell, b)


def test_relinearize_of_tensor_equals_mul_relin(env):
    fhe, client, ctx, orc = env
    rng = np.random.default_rng(5)
    x, y = rng.uniform(-1, 1, (2, ctx.max_slots))
    cx = client.encrypt(x, cur_limbs=12)
    cy = client.encrypt(y, cur_limbs=12)
    three = fhe.homo_mul_no_relin(cx, cy, ctx)
    assert len(three.cv) == 3 and three.state.scale_degree == 2
    r1 = fhe.homo_relinearize(three, ctx)
    r2 = fhe.homo_mul_relin(cx, cy, ctx)
    for u, v in zip(r1.cv, r2.cv):
        assert torch.equal(u, v)


def test_product_decrypts_to_slot_product(fixed_env):
    # fixed-scale parameters (scale = prime size): the rescaled product keeps the scale.  (At scale
    # 2^40 with 50-bit primes a product rescales to scale 2^30, where a uniform-ternary key's
    # rescale noise alone is ~1e-5 per slot.)
    fhe, client, ctx, orc = fixed_env
    rng = np.random.default_rng(6)
    x, y = rng.uniform(-1, 1, (2, ctx.max_slots))
    cx = client.encrypt(x, cur_limbs=ctx.L)
    cy = client.encrypt(y, cur_limbs=ctx.L)
    prod = fhe.rescale(fhe.homo_mul_relin(cx, cy, ctx), ctx)
    assert prod.state.cur_limbs == ctx.L - 1 and prod.state.scale_degree == 1
    got = client.decrypt(prod).real
    assert np.max(np.abs(got - x * y)) < TOL
    # a three-component product decrypts too once relinearised after the rescale
    three = fhe.rescale(fhe.homo_mul_no_relin(cx, cy, ctx), ctx)
    got3 = client.decrypt(fhe.homo_relinearize(three, ctx)).real
    assert np.max(np.abs(got3 - x * y)) < TOL


def test_chebyshev_step_postop(fixed_env):
    fhe, client, ctx, orc = fixed_env
    rng = np.random.default_rng(7)
    x = rng.uniform(-1, 1, ctx.max_slots)
    t1 = client.encrypt(x, cur_limbs=ctx.L)

    def minus_one(l, r):
        limbs = min(l.state.cur_limbs, r.state.cur_limbs) - 1
        sf = l.state.scaling_factor * r.state.scaling_factor / ctx.rescale_divisor_at(limbs + 1)
        return fhe.encode_scalar(-1.0, cur_limbs=limbs, scale_degree=1, scaling_factor=sf, context=ctx)

    t2 = fhe.homo_mul_relin_rescale_postop(t1, t1, ctx, apply_double=True, scalar=minus_one(t1, t1))
    t3 = fhe.homo_mul_relin_rescale_postop(t1, t2, ctx, apply_double=True, sub=t1)
    t4 = fhe.homo_mul_relin_rescale_postop(t2, t2, ctx, apply_double=True, scalar=minus_one(t2, t2))
    th = np.arccos(x)
    for k, t in ((2, t2), (3, t3), (4, t4)):
        got = client.decrypt(t).real
        assert np.max(np.abs(got - np.cos(k * th))) < TOL, k
    assert t4.state.cur_limbs == ctx.L - 2


def test_scalar_ops(fixed_env):
    # fixed-scale context: a product by an encoded constant rescales back to the working scale
    fhe, client, ctx, orc = fixed_env
    rng = np.random.default_rng(8)
    x = rng.uniform(-1, 1, ctx.max_slots)
    ct = client.encrypt(x, cur_limbs=6)
    half = fhe.encode_scalar(0.5, cur_limbs=6, scale_degree=1, scaling_factor=ct.state.scaling_factor, context=ctx)
    r = fhe.homo_mul_scalar_rescale(ct, half, ctx)
    assert r.state.cur_limbs == 5
    assert np.max(np.abs(client.decrypt(r).real - 0.5 * x)) < TOL
    steps = fhe.rescale(fhe.homo_mul_scalar(ct, half, ctx), ctx)  # the fused call gives the steps' residues
    assert r.state == steps.state and all(torch.equal(a, b) for a, b in zip(r.cv, steps.cv))
    shift = fhe.encode_scalar(0.375, cur_limbs=6, scale_degree=1, scaling_factor=ct.state.scaling_factor,
                              context=ctx)
    assert np.max(np.abs(client.decrypt(fhe.homo_add_scalar(ct, shift, ctx)).real - (x + 0.375))) < TOL
    three = fhe.encode_scalar(3, cur_limbs=6, scale_degree=0, mode="integer", context=ctx)
    r3 = fhe.homo_mul_scalar(ct, three, ctx)
    assert r3.state.scaling_factor == ct.state.scaling_factor and r3.state.cur_limbs == 6
    assert np.max(np.abs(client.decrypt(r3).real - 3 * x)) < TOL
    # a scalar at the wrong scale is refused
    with pytest.raises(ValueError):
        fhe.homo_add_scalar(ct, three, ctx)


def test_add_pt(env):
    fhe, client, ctx, orc = env
    rng = np.random.default_rng(9)
    x, y = rng.uniform(-1, 1, (2, ctx.max_slots))
    ct = client.encrypt(x, cur_limbs=8)
    pt = fhe.encode_plaintext(y, ct.state, ctx.max_slots, ctx)
    assert np.max(np.abs(client.decrypt(fhe.homo_add_pt(ct, pt, ctx)).real - (x + y))) < TOL


def test_weighted_sum_equals_scalar_loop_and_oracle(fixed_env):
    fhe, client, ctx, orc = fixed_env
    rng = np.random.default_rng(10)
    n, limbs = 5, 6
    xs = rng.uniform(-1, 1, (n, ctx.max_slots))
    ws = rng.uniform(-2, 2, n)
    cts = [client.encrypt(v, cur_limbs=limbs) for v in xs]
    batch = fhe.pack_cipher_batch(cts)
    sf = cts[0].state.scaling_factor
    table = fhe.encode_scalar(ws, cur_limbs=limbs, scale_degree=1, scaling_factor=sf, context=ctx)
    acc = fhe.grouped_scalar_weighted_acc(batch, table, ctx)
    assert acc.batch_size == 1 and acc.state.scale_degree == 2
    # the loop of scalar products and additions (the reference's residue check)
    loop = None
    for c, w in zip(cts, ws):
        enc = fhe.encode_scalar(float(w), cur_limbs=limbs, scale_degree=1, scaling_factor=sf, context=ctx)
        term = fhe.homo_mul_scalar(c, enc, ctx)
        loop = term if loop is None else fhe.homo_add(loop, term, ctx)
    for u, v in zip(acc.cv, loop.cv):
        assert torch.equal(u[:, :limbs], v[:, :limbs])
    # the oracle's weighted sum
    w_tab = table.residues.numpy().reshape(1, n, limbs)
    for comp in range(2):
        x_h = np.stack([_host(c.cv[comp])[0, :limbs] for c in cts])
        assert np.array_equal(_host(acc.cv[comp])[0], orc.weighted_sum(limbs, x_h, w_tab)[0])
    got = client.decrypt(fhe.rescale(acc, ctx)).real
    assert np.max(np.abs(got - ws @ xs)) < TOL


def test_product_arguments_are_checked(env):
    fhe, client, ctx, orc = env
    ct = client.encrypt(np.zeros(ctx.max_slots), cur_limbs=4)
    three = fhe.homo_mul_no_relin(ct, ct, ctx)
    with pytest.raises(ValueError):
        fhe.homo_mul_relin(three, ct, ctx)
    from holmes_amd import _native as nat

    lib = nat.lib()
    t = ctx.empty(1, 4, ctx.N)
    ws = ctx.workspace(lib.hck_relinearize_workspace_bytes(ctx.handle, 4, 1))
    # the output may not alias d2
    rc = lib.hck_relinearize(ctx.handle, 4, 1, t.data_ptr(), t.data_ptr(), t.data_ptr(), 4 * ctx.N,
                             ctx.relin_key.data_ptr(), t.data_ptr(), ctx.empty(1, 4, ctx.N).data_ptr(), 4 * ctx.N,
                             ws.data_ptr(), ws.numel(), None)
    assert rc == -1


@pytest.mark.parametrize("engine", ["mfma", "valu"])
def test_aliased_products_are_refused(env, engine):
    """hck_mul_relin_rescale(_postop) refuses outputs that overlap an operand (in place on a0, a1,
    b0 or b1, or a view shifted by one limb) on both conversion engines, and
    hck_lincomb_rescale refuses an output that is any group's input: both before launching."""
    fhe, client, ctx, orc = env
    from holmes_amd import _native as nat

    lib = nat.lib()
    ctx.set_conversion_engine(engine)
    try:
        limbs, B, N = 4, 2, ctx.N
        a = ctx.empty(2, B, limbs, N)
        b = ctx.empty(2, B, limbs, N)
        fresh = ctx.empty(2, B, limbs - 1, N)
        ws = ctx.workspace(lib.hck_mul_relin_rescale_workspace_bytes(ctx.handle, limbs, B))
        st = limbs * N
        stream = torch.cuda.current_stream().cuda_stream

        def call(o0, o1, ostride):
            return lib.hck_mul_relin_rescale(ctx.handle, limbs, B, a[0].data_ptr(), a[1].data_ptr(), st,
                                             b[0].data_ptr(), b[1].data_ptr(), st, ctx.relin_key.data_ptr(),
                                             o0, o1, ostride, ws.data_ptr(), ws.numel(), stream)

        for target in (a[0], a[1], b[0], b[1]):
            assert call(target.data_ptr(), fresh[1].data_ptr(), st) == nat.HCK_ERR_ARG
            assert call(fresh[0].data_ptr(), target.data_ptr(), st) == nat.HCK_ERR_ARG
        assert call(a[0, 0, 1].data_ptr(), fresh[1].data_ptr(), st) == nat.HCK_ERR_ARG  # shifted by one limb
        assert call(fresh[0].data_ptr(), fresh[0, 0, 1].data_ptr(), (limbs - 1) * N) == nat.HCK_ERR_ARG
        rc = lib.hck_mul_relin_rescale_postop(ctx.handle, limbs, B, a[0].data_ptr(), a[1].data_ptr(), st,
                                              b[0].data_ptr(), b[1].data_ptr(), st, ctx.relin_key.data_ptr(), 1,
                                              None, None, 0, None, b[1].data_ptr(), fresh[1].data_ptr(), st,
                                              ws.data_ptr(), ws.numel(), stream)
        assert rc == nat.HCK_ERR_ARG
        x = [ctx.empty(limbs, N) for _ in range(4)]
        w = torch.zeros(2, limbs, dtype=torch.uint64, device="cuda")
        lws = ctx.workspace(lib.hck_lincomb_rescale_workspace_bytes(ctx.handle, limbs, 2))
        outs = [ctx.empty(limbs - 1, N), x[2]]  # group 1 writes over group 1's first input
        rc = lib.hck_lincomb_rescale(ctx.handle, limbs, 2, 2, nat.ptr_array([t.data_ptr() for t in x]), w.data_ptr(),
                                     nat.ptr_array([o.data_ptr() for o in outs]), None, 0, lws.data_ptr(),
                                     lws.numel(), stream)
        assert rc == nat.HCK_ERR_ARG
        outs = [x[3], ctx.empty(limbs - 1, N)]  # group 0 writes over group 1's input
        rc = lib.hck_lincomb_rescale(ctx.handle, limbs, 2, 2, nat.ptr_array([t.data_ptr() for t in x]), w.data_ptr(),
                                     nat.ptr_array([o.data_ptr() for o in outs]), None, 0, lws.data_ptr(),
                                     lws.numel(), stream)
        assert rc == nat.HCK_ERR_ARG
        torch.cuda.synchronize()
    finally:
        ctx.set_conversion_engine("mfma")


def test_lincomb_matches_oracle(env):
    """Pointer-list linear combinations (hck_lincomb): operands at different levels in separate
    allocations, weighted (against the oracle's weighted sum per group) and unit weights (against
    exact sums), an output aliasing its group's first input."""
    fhe, client, ctx, orc = env
    rng = np.random.default_rng(41)
    limbs, G, T = 6, 3, 9
    srcs = [[_dev(_rand(ctx, rng, 1, limbs + int(rng.integers(0, 5)))[0]) for _ in range(T)] for _ in range(G)]
    w = np.stack([[rng.integers(0, ctx.primes[l], dtype=np.uint64) for l in range(limbs)] for _ in range(T)])
    outs = [ctx.empty(limbs, ctx.N) for _ in range(G)]
    ctx.lincomb(srcs, limbs, outs, torch.from_numpy(w).cuda())
    for g in range(G):
        x = np.stack([_host(t)[:limbs] for t in srcs[g]])
        assert np.array_equal(_host(outs[g]), orc.weighted_sum(limbs, x, w[None])[0]), f"group {g}"
    q = np.array(ctx.primes[:limbs], dtype=object).reshape(limbs, 1)
    want = [sum(_host(t)[:limbs].astype(object) for t in srcs[g]) % q for g in range(G)]
    first = [_host(srcs[g][0]).copy() for g in range(G)]
    ctx.lincomb(srcs, limbs, [srcs[g][0] for g in range(G)])  # unit weights, in place
    for g in range(G):
        got = _host(srcs[g][0])
        assert np.array_equal(got[:limbs], want[g].astype(np.uint64)), f"unit group {g}"
        assert np.array_equal(got[limbs:], first[g][limbs:])  # limbs above the count untouched
    with pytest.raises(ValueError):
        ctx.lincomb(srcs, limbs, outs[:2])


@pytest.mark.parametrize("limbs,G,T", [(6, 3, 9), (24, 64, 4), (2, 5, 1)])
def test_lincomb_rescale_matches_oracle(env, limbs, G, T):
    check_lincomb_rescale(env, limbs, G, T)


def check_lincomb_rescale(env, limbs, G, T):
    """hck_lincomb_rescale: operands at different levels in separate allocations, weighted, a scalar
    added on every other group; equal to hck_lincomb + hck_rescale + the scalar add on the GPU, and
    to the oracle's weighted sum followed by its rescale."""
    fhe, client, ctx, orc = env
    from holmes_amd import _native as nat

    rng = np.random.default_rng(1000 + limbs + G)
    srcs = [[_dev(_rand(ctx, rng, 1, limbs + int(rng.integers(0, 3)))[0]) for _ in range(T)] for _ in range(G)]
    w = np.stack([[rng.integers(0, ctx.primes[i], dtype=np.uint64) for i in range(limbs)] for _ in range(T)])
    wd = torch.from_numpy(w).cuda()
    add = [int(rng.integers(0, ctx.primes[i])) for i in range(limbs - 1)]
    groups = range(0, G, 2)
    outs = [ctx.empty(limbs - 1, ctx.N) for _ in range(G)]
    ctx.lincomb_rescale(srcs, limbs, outs, wd, add=add, add_groups=groups)
    acc = [ctx.empty(limbs, ctx.N) for _ in range(G)]
    ctx.lincomb(srcs, limbs, acc, wd)
    for g in range(G):
        want = ctx.rescale_raw(acc[g][None], limbs)
        if g in groups:
            ctx.poly_op(nat.HCK_OP_ADD_SCALAR, want, want, prime_idx=ctx.q_prime_idx(limbs - 1), scalar=add)
        assert torch.equal(outs[g], want[0]), f"group {g}"
    for g in (0, G - 1):
        x = np.stack([_host(t)[:limbs] for t in srcs[g]])
        r = orc.rescale(limbs, orc.weighted_sum(limbs, x, w[None])[0])
        if g in groups:
            q = np.array(ctx.primes[:limbs - 1], dtype=object).reshape(-1, 1)
            r = ((r.astype(object) + np.array(add, dtype=object).reshape(-1, 1)) % q).astype(np.uint64)
        assert np.array_equal(_host(outs[g]), r), f"oracle group {g}"


@pytest.mark.parametrize("engine", ["mfma", "valu"])
def test_mul_relin_rescale_postop_equals_the_steps(env, engine):
    _, _, ctx, _ = env
    ctx.set_conversion_engine(engine)
    try:
        check_mul_relin_rescale_postop(env, (24, 9, 2))
    finally:
        ctx.set_conversion_engine("mfma")


def check_mul_relin_rescale_postop(env, levels, batch=3):
    """hck_mul_relin_rescale_postop (2 x product - sub, 2 x product + scalar, product - sub) equals the
    rescaled product followed by the additions, residue for residue."""
    from holmes_amd import _native as nat

    fhe, client, ctx, orc = env
    for ell in levels:
        rng = np.random.default_rng(1300 + ell)
        a0, a1, b0, b1 = (_dev(_rand(ctx, rng, batch, ell)) for _ in range(4))
        s0, s1 = (_dev(_rand(ctx, rng, batch, ell)) for _ in range(2))  # more limbs than needed
        sc = [int(rng.integers(0, ctx.primes[i])) for i in range(ell - 1)]
        base = ctx.mul_relin_rescale_raw(a0, a1, b0, b1, ell, ctx.relin_key, stacked=True)
        idx = ctx.q_prime_idx(ell - 1)
        for twice, sub, scalar in ((True, True, False), (True, False, True), (False, True, True)):
            want = base.clone()
            for c, sv in ((0, s0), (1, s1)):
                w = want[c]
                if twice:
                    ctx.poly_op(nat.HCK_OP_ADD, w, w, w, prime_idx=idx)
                if sub:
                    ctx.poly_op(nat.HCK_OP_SUB, w, w, sv[:, :ell - 1], prime_idx=idx)
                if scalar and c == 0:
                    ctx.poly_op(nat.HCK_OP_ADD_SCALAR, w, w, prime_idx=idx, scalar=sc)
            got = ctx.mul_relin_rescale_postop_raw(a0, a1, b0, b1, ell, ctx.relin_key, apply_double=twice,
                                                   sub=(s0, s1) if sub else None, scalar=sc if scalar else None)
            assert torch.equal(got, want), (ell, twice, sub, scalar)
