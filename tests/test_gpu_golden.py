"""The GPU path reproduces the committed production golden hashes (N = 2^16, 24 + 8 primes of
50 bits, dnum 3): NTT, INTT, key switch, rotation, rescale, encode and the BSGS MAC."""

import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from tests.golden import golden_inputs as G  # noqa: E402

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def env():
    from holmes_amd import fhe

    with open(os.path.join(HERE, "ckks_prod.json")) as f:
        doc = json.load(f)
    spec = fhe.CKKSContextSpec(depth=23, dnum=3, dcrt_bits=50, first_mod=50, seed=1)
    ctx = fhe.CKKSContext(spec)
    assert [int(p) for p in ctx.primes] == doc["primes"]
    return ctx, doc


def _h(t):
    torch.cuda.synchronize()
    return G.limb_hashes(t.cpu().numpy())


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_golden_ntt(env):
    ctx, doc = env
    L, n = ctx.L, ctx.N
    x = G.uniform(G.rng(G.SEED, "ntt"), ctx.primes[:L], (), n)
    idx = list(range(L))
    fwd = ctx.ntt(_dev(x)[None], prime_idx=idx)
    assert _h(fwd) == doc["hashes"]["ntt_fwd"]
    inv = ctx.ntt(_dev(x)[None], prime_idx=idx, inverse=True)
    assert _h(inv) == doc["hashes"]["ntt_inv"]


def test_golden_keyswitch_rotate_rescale(env):
    ctx, doc = env
    L, n = ctx.L, ctx.N
    s_from, s_to, a, e, g = G.key_inputs(G.PROD, ctx.primes, 1)
    key = ctx.make_switching_key(s_from, s_to, a, e)
    d = G.uniform(G.rng(G.SEED, "keyswitch"), ctx.primes[:L], (), n)
    b, aa = ctx.keyswitch(_dev(d)[None], L, key)
    assert _h(b) == doc["hashes"]["ks_b"]
    assert _h(aa) == doc["hashes"]["ks_a"]
    r = G.rng(G.SEED, "rotate")
    c0, c1 = G.uniform(r, ctx.primes[:L], (), n), G.uniform(r, ctx.primes[:L], (), n)
    o0, o1 = ctx.rotate_raw(_dev(c0)[None], _dev(c1)[None], L, g, key)
    assert _h(o0) == doc["hashes"]["rot_0"]
    assert _h(o1) == doc["hashes"]["rot_1"]
    assert _h(ctx.rescale_raw(o0, L)) == doc["hashes"]["rescale"]


def test_golden_encode_and_mac(env):
    ctx, doc = env
    L, n = ctx.L, ctx.N
    vals = G.rng(G.SEED, "encode").normal(size=n // 2)
    enc = ctx.encode_real(_dev(vals)[None], 2.0**40, L)
    assert _h(enc) == doc["hashes"]["encode"]
    r = G.rng(G.SEED, "mac")
    pts = G.uniform(r, ctx.primes[:2], (4,), n)
    baby = G.uniform(r, ctx.primes[:2], (2, 2), n)
    b0 = [_dev(baby[b, 0])[None] for b in range(2)]
    b1 = [_dev(baby[b, 1])[None] for b in range(2)]
    res = ctx.bsgs_mac(b0, b1, _dev(pts), 2, 2)  # [2][G][1][limbs][N]
    assert _h(res[:, :, 0]) == doc["hashes"]["mac"]
