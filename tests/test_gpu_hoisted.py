"""Hoisted / extended-basis surface of the fhe namespace on the GPU: fast_rotate (both outputs),
moddown_from_ext, grouped_pairwise_mac, prepare_hoisted_baby_rotations (anchor composition),
hoisted_mac_sum (Horner and double-hoisted), GPU plaintext encode (real, complex, extended)."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402

LIMBS = 6


@pytest.fixture(scope="module")
def env():
    from holmes_amd import fhe

    rots = (1, 2, 3, 5, 8, 16, 24, 32, 40, 64, 128)
    spec = fhe.CKKSContextSpec(depth=23, dnum=3, seed=777, rotations=rots)
    client, ctx = fhe.generate_client_context(spec)
    rng = np.random.default_rng(3)
    x = rng.normal(size=ctx.max_slots)
    ct = client.encrypt(x, cur_limbs=LIMBS)
    return fhe, client, ctx, x, ct


def _h(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_fast_rotate_rows_equal_single_rotations(env):
    fhe, client, ctx, x, ct = env
    offs = (0, 1, 5, 128)
    batch = fhe.fast_rotate(ct, offs, ctx)
    assert batch.batch_size == len(offs) and not batch.is_ext
    for i, (row, off) in enumerate(zip(fhe.unpack_cipher_batch(batch), offs)):
        want = fhe.homo_rotate(ct, off, ctx)
        assert np.array_equal(_h(row.cv[0]), _h(want.cv[0][:, :LIMBS])), off
        assert np.array_equal(_h(row.cv[1]), _h(want.cv[1][:, :LIMBS])), off


def test_fast_rotate_ext_then_moddown_is_exact(env):
    fhe, client, ctx, x, ct = env
    offs = (0, 3, 64)
    ext = fhe.fast_rotate(ct, offs, ctx, output_ext=True)
    assert ext.is_ext and ext.cv[0].shape[1] == LIMBS + ctx.K
    back = fhe.moddown_from_ext(ext, ctx)
    plain = fhe.fast_rotate(ct, offs, ctx)
    assert np.array_equal(_h(back.cv[0]), _h(plain.cv[0]))
    assert np.array_equal(_h(back.cv[1]), _h(plain.cv[1]))


def test_rotate_ext_accumulates(env):
    fhe, client, ctx, x, ct = env
    g = ctx.galois_element(5)
    key = ctx.key_for_galois(g)
    c0, c1 = ct.cv[0][:, :LIMBS], ct.cv[1][:, :LIMBS]
    e0, e1 = ctx.rotate_ext(c0, c1, LIMBS, g, key)
    rng = np.random.default_rng(4)
    idx = ctx.ext_prime_idx(LIMBS)
    acc = [np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in idx])[None] for _ in range(2)]
    a0, a1 = (torch.from_numpy(a).cuda() for a in acc)
    s0, s1 = ctx.rotate_ext(c0, c1, LIMBS, g, key, out0=a0, out1=a1, acc=(a0, a1))
    q = np.array([ctx.primes[i] for i in idx], dtype=object).reshape(-1, 1)
    for got, base, add in ((s0, e0, acc[0]), (s1, e1, acc[1])):
        want = ((_h(base)[0].astype(object) + add[0].astype(object)) % q).astype(np.uint64)
        assert np.array_equal(_h(got)[0], want)


def test_moddown_matches_oracle(env):
    fhe, client, ctx, x, ct = env
    orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
    rng = np.random.default_rng(11)
    idx = ctx.ext_prime_idx(LIMBS)
    xs = np.stack([np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in idx])
                   for _ in range(3)])
    got = _h(ctx.moddown(torch.from_numpy(xs).cuda(), LIMBS))
    for b in range(3):
        assert np.array_equal(got[b], orc.moddown(LIMBS, xs[b]))


def test_moddown_every_level(env):
    """ModDown of an extended-basis poly at every level ell = 1 .. L against the oracle."""
    fhe, client, ctx, x, ct = env
    orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
    for ell in range(1, ctx.L + 1):
        rng = np.random.default_rng(500 + ell)
        xs = np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in ctx.ext_prime_idx(ell)])[None]
        got = _h(ctx.moddown(torch.from_numpy(xs).cuda(), ell))
        assert np.array_equal(got[0], orc.moddown(ell, xs[0])), f"{ell} limbs"


def test_grouped_pairwise_mac_ext_decrypts(env):
    fhe, client, ctx, x, ct = env
    offs = (0, 1, 2, 3)
    rng = np.random.default_rng(5)
    masks = rng.uniform(-1, 1, size=(len(offs), ctx.max_slots))
    st = ct.state.replace(scaling_factor=float(ctx.rescale_divisor_at(LIMBS)))
    want = sum(masks[i] * np.roll(x, -o) for i, o in enumerate(offs))
    for ext in (False, True):
        rot = fhe.fast_rotate(ct, offs, ctx, output_ext=ext)
        pts = fhe.encode_plaintext(masks, st, ctx.max_slots, ctx, is_ext=ext)
        prod = fhe.grouped_pairwise_mac(rot, pts, 1, ctx)
        total = fhe.moddown_from_ext(prod, ctx) if ext else prod
        got = client.decrypt(fhe.rescale(total, ctx)).real.reshape(-1)
        assert np.max(np.abs(got - want)) < 2.0**-16, ext


def test_encode_complex_plaintext(env):
    fhe, client, ctx, x, ct = env
    rng = np.random.default_rng(9)
    v = rng.uniform(-1, 1, size=ctx.max_slots) + 1j * rng.uniform(-1, 1, size=ctx.max_slots)
    st = ct.state.replace(scaling_factor=float(ctx.rescale_divisor_at(LIMBS)))
    pt = fhe.encode_plaintext(v, st, ctx.max_slots, ctx)
    got = client.decrypt(fhe.rescale(fhe.homo_mul_pt(ct, pt, ctx), ctx)).reshape(-1)
    assert np.max(np.abs(got - v * x)) < 2.0**-16
    # sparse slots: 1024 values tiled across the ring
    small = fhe.encode_plaintext(v[:1024].real, st, 1024, ctx)
    got = client.decrypt(fhe.rescale(fhe.homo_mul_pt(ct, small, ctx), ctx)).real.reshape(-1)
    assert np.max(np.abs(got - np.tile(v[:1024].real, ctx.max_slots // 1024) * x)) < 2.0**-16


def test_baby_rotations_anchor_composition(env):
    fhe, client, ctx, x, ct = env
    # offset 48 has no key: reached from the anchor 40 (key) plus 8 (key)
    offs = (0, 8, 16, 24, 40, 48)
    babies = fhe.prepare_hoisted_baby_rotations(ct, offs, ctx, baby_anchor_step=5)
    assert babies[0].cv[0].data_ptr() == ct.cv[0].data_ptr()
    for b, o in zip(babies, offs):
        got = client.decrypt(b).real.reshape(-1)
        assert np.max(np.abs(got - np.roll(x, -o))) < 2.0**-20, o


@pytest.mark.parametrize("strategy", ["normal", "ext_double_hoist"])
def test_hoisted_mac_sum_decrypts(env, strategy):
    fhe, client, ctx, x, ct = env
    offs, G, step = (0, 1, 2, 3), 3, 4  # giant offset 4: keys 4 (Horner) / 4, 8 (double hoist)
    for r in (4, 8):
        g = ctx.galois_element(r)
        if g not in ctx.rotation_keys:
            ctx.rotation_keys[g] = client.rotation_key(g)
    rng = np.random.default_rng(21)
    rows = rng.uniform(-1, 1, size=(G * len(offs), ctx.max_slots))
    st = ct.state.replace(scaling_factor=float(ctx.rescale_divisor_at(LIMBS)))
    pts = fhe.encode_plaintext(rows, st, ctx.max_slots, ctx)
    res = fhe.hoisted_mac_sum(ct, offs, pts, step, G, ctx, strategy=strategy)
    want = np.zeros(ctx.max_slots)
    for g in range(G):
        inner = sum(rows[g * len(offs) + b] * np.roll(x, -o) for b, o in enumerate(offs))
        want += np.roll(inner, -g * step)
    got = client.decrypt(fhe.rescale(res, ctx)).real.reshape(-1)
    assert np.max(np.abs(got - want)) < 2.0**-16
