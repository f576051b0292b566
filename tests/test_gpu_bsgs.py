"""GPU parity of the BSGS row kernels: diagonal packing, encode (special IFFT + round + NTT) and
the multi-input baby-step MAC, bit-exact against the oracle."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402


@pytest.fixture(scope="module")
def env():
    from holmes_amd import fhe

    spec = fhe.CKKSContextSpec(depth=23, dnum=3, seed=99)
    client, ctx = fhe.generate_client_context(spec)
    orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
    return ctx, orc


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("D,lanes,shift,B,base,G", [(4096, 8, 0, 16, 32, 4), (256, 8, 32, 16, 3, 2)])
def test_pack_diagonals(env, D, lanes, shift, B, base, G):
    ctx, _ = env
    rng = np.random.default_rng(D + base)
    W = rng.normal(scale=0.02, size=(D, D))
    got = _host(ctx.pack_diagonals(torch.from_numpy(W).cuda(), lanes=lanes, lane_shift=shift, baby_steps=B,
                                   giant_base=base, giant_count=G))
    want = O.pack_diagonals(W, lanes, shift, B, base, G, ctx.max_slots)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("scale", [2.0**40, None])
def test_encode_real_bit_exact(env, scale):
    ctx, orc = env
    limbs = 20
    scale = float(ctx.rescale_divisor_at(limbs)) if scale is None else scale
    rng = np.random.default_rng(7)
    vals = rng.normal(scale=0.05, size=(3, ctx.max_slots))
    vals[1, :5] = [0.0, 1.0, -1.0, 0.5 / scale, -0.5 / scale]  # rounding ties away from zero
    got = _host(ctx.encode_real(torch.from_numpy(vals).cuda(), scale, limbs))
    for r in range(3):
        want, ok = orc.encode_real(vals[r], scale, list(range(limbs)))
        assert ok
        assert np.array_equal(got[r], want), f"row {r}"


def test_encode_every_limb_count(env):
    """The fused encoder at every limb count 1 .. L (its per-limb column loop and the row pass's
    limb list), one row each at that level's prime scale, against the oracle."""
    ctx, orc = env
    rng = np.random.default_rng(71)
    for limbs in range(1, ctx.L + 1):
        scale = float(ctx.rescale_divisor_at(limbs))
        vals = rng.normal(scale=0.05, size=(1, ctx.max_slots))
        got = _host(ctx.encode_real(torch.from_numpy(vals).cuda(), scale, limbs))
        want, ok = orc.encode_real(vals[0], scale, list(range(limbs)))
        assert ok and np.array_equal(got[0], want), f"{limbs} limbs"


def test_encode_overflow_is_reported(env):
    ctx, _ = env
    vals = np.full((1, ctx.max_slots), 2.0**21)  # DC coefficient exactly 2^61: the first refused value
    with pytest.raises(ValueError, match="2\\^61"):
        ctx.encode_real(torch.from_numpy(vals).cuda(), 2.0**40, 4)


def test_encode_large_coefficients_bit_exact(env):
    """Coefficients in [2^52, 2^61) (the reference's encoder cap, softmax.py:559): a DC offset of
    1000 at scale 2^50 puts coefficient 0 near 2^60 and the noise rows' other coefficients past
    2^52; residues equal the oracle's, and the constant row's DC residue is 1000 * 2^50 mod q."""
    ctx, orc = env
    limbs, scale = 12, 2.0**50
    rng = np.random.default_rng(61)
    vals = np.stack([np.full(ctx.max_slots, 1000.0), 1000.0 + rng.normal(scale=8.0, size=ctx.max_slots),
                     rng.normal(scale=30.0, size=ctx.max_slots)])
    got = _host(ctx.encode_real(torch.from_numpy(vals).cuda(), scale, limbs))
    for r in range(3):
        want, ok = orc.encode_real(vals[r], scale, list(range(limbs)))
        assert ok and np.array_equal(got[r], want), f"row {r}"
    coef, _ = orc.encode_real(vals[0], scale, list(range(limbs)), ntt=False)
    assert [int(c) for c in coef[:, 0]] == [(1000 * 2**50) % q for q in ctx.primes[:limbs]]


@pytest.mark.parametrize("ni,nb,G,limbs", [(16, 16, 5, 3), (3, 5, 6, 2), (1, 1, 1, 1), (5, 64, 9, 1), (2, 3, 2, 24)])
def test_bsgs_mac(env, ni, nb, G, limbs):
    ctx, orc = env
    rng = np.random.default_rng(ni * 100 + nb)
    q = np.array(ctx.primes[:limbs], dtype=np.uint64).reshape(1, limbs, 1)
    pts = (rng.integers(0, 2**62, size=(G * nb, limbs, ctx.N), dtype=np.uint64) % q)
    babies = rng.integers(0, 2**62, size=(nb, 2, ni, limbs, ctx.N), dtype=np.uint64) % q.reshape(1, 1, 1, limbs, 1)
    pts[0, 0, :3] = [0, ctx.primes[0] - 1, ctx.primes[0] - 1]
    babies[0, :, 0, 0, :3] = ctx.primes[0] - 1
    bt = torch.from_numpy(babies).cuda()
    res = _host(ctx.bsgs_mac([bt[b, 0] for b in range(nb)], [bt[b, 1] for b in range(nb)],
                             torch.from_numpy(pts).cuda(), limbs, G))
    for i in range(ni):
        want = orc.bsgs_mac(limbs, nb, G, pts, np.ascontiguousarray(babies[:, :, i]))
        assert np.array_equal(res[:, :, i], want), f"input {i}"


def test_bsgs_mac_rejects_more_babies_than_a_launch_holds(env):
    """65 baby steps exceed the kernel's pointer table (64): an argument error, nothing launched."""
    from holmes_amd import _native as nat

    ctx, _ = env
    x = ctx.zeros(1, 1, ctx.N)
    with pytest.raises(nat.NativeError):
        ctx.bsgs_mac([x] * 65, [x] * 65, ctx.zeros(65, 1, ctx.N), 1, 1)
