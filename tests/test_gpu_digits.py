"""GPU parity of the fused key switch under other digit layouts than the dnum 3 / 24-limb chain:
dnum 4 at 24 limbs (6-limb digits, 6 special primes) and dnum 4 at 32 limbs (8-limb digits, 32
conversion targets per ModUp digit and per ModDown: the conversion kernel's variant with separate
exchange runs), bit-exact against the oracle at the full level and a partial one."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402


def _rand(ctx, rng, batch, limbs):
    return np.stack([np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in range(limbs)])
                     for _ in range(batch)])


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("depth,dnum", [(23, 4), (31, 4)])
def test_keyswitch_and_rescale_other_digit_layouts(depth, dnum):
    from holmes_amd import fhe

    spec = fhe.CKKSContextSpec(depth=depth, dnum=dnum, dcrt_bits=50, first_mod=50, seed=4000 + depth)
    client, ctx = fhe.generate_client_context(spec, device="cuda")
    orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
    assert ctx.alpha == -(-ctx.L // dnum) and ctx.K == ctx.alpha
    g = ctx.galois_element(9)
    s_from, s_to, a, e = client.key_inputs(g)
    gk = ctx.make_switching_key(s_from, s_to, a, e)
    ok = orc.make_ksk(s_from, s_to, a, e)
    assert np.array_equal(_host(gk), ok)
    for ell in (ctx.L, ctx.L - ctx.alpha - 1):
        rng = np.random.default_rng(ell)
        d = _rand(ctx, rng, 2, ell)
        ob, oa = ctx.keyswitch(torch.from_numpy(d).cuda(), ell, gk)
        gb, ga = _host(ob), _host(oa)
        for b in range(2):
            wb, wa = orc.keyswitch(ell, d[b], ok)
            assert np.array_equal(gb[b], wb) and np.array_equal(ga[b], wa), f"{ell} limbs, item {b}"
        x = _rand(ctx, rng, 1, ell)
        assert np.array_equal(_host(ctx.rescale_raw(torch.from_numpy(x).cuda(), ell))[0], orc.rescale(ell, x[0]))
    ctx.close()
