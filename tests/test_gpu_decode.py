"""GPU checks of the encrypted decode step (config C5 at a reduced MLP width of 6144): one token
against a 256-token and a 200-token encrypted PairFold cache (three pages; the second appends into
a partly filled page through the four-sum), N = 2^16, 24 x 50-bit Q primes, scale 2^50, sparse
ternary secret.  The decrypted output must match decode_layer_numpy (the float64 semantics with
the same polynomials) within 2^-16 of the output's magnitude, and the token's key page must
decrypt to the RoPE'd, conjugated key fold of the float64 computation.  The slot simulator
(tests/test_decode_sim.py) holds the same dataflow to round-off on the CPU; here the remaining
difference is CKKS noise and the five refreshes."""

import types

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SEED = 20261205


@pytest.fixture(scope="module")
def env():
    from holmes_amd import bootstrap as B
    from holmes_amd import decode as Dm
    from holmes_amd import fhe

    spec = Dm.DecodeSpec(intermediate=6144)
    cs = fhe.CKKSContextSpec(depth=23, dnum=3, dcrt_bits=50, first_mod=50, scale_bits=50,
                             secret_key_dist="SPARSE_TERNARY", hamming_weight=192, seed=SEED)
    client, ctx = fhe.generate_client_context(cs, device="cuda")
    client.generate_rotation_keys(Dm.decode_key_rotations(pages=3))
    progs = [B.generate(ctx, b) for b in Dm.decode_bootstrap_specs()]
    ops = Dm.CipherOps(ctx, progs[0], progs[1])
    rng = np.random.default_rng(SEED)
    w = Dm.random_weights(spec, rng)
    layer = Dm.DecodeLayer(ops, w, spec)
    return Dm, fhe, client, ctx, ops, layer, w, spec, rng


@pytest.mark.timeout(900)
@pytest.mark.parametrize("history", [256, 200])
def test_decode_step_matches_float64(env, history):
    Dm, fhe, client, ctx, ops, layer, w, spec, rng = env
    x = rng.normal(size=spec.hidden_dim)
    ck = rng.normal(size=(history, 1024))
    cv = rng.normal(size=(history, 1024))
    S = float(ctx.scale_at(ctx.L))
    cache = Dm.encrypt_kv_history(client, ck, cv, spec, S)
    xin = client.encrypt(Dm.lr8(x), cur_limbs=ctx.L)
    cc = types.SimpleNamespace(fhe=fhe, context=ctx)
    print(f"decode step, history {history}", flush=True)
    out, stages, _ = layer.forward(xin, cache, position=history, crypto_context=cc)
    ref = Dm.decode_layer_numpy(x, ck, cv, w, spec, position=history)
    dec = client.decrypt(out)
    got = dec[::8].real
    err = float(np.max(np.abs(got - ref["output"])))
    mag = float(np.max(np.abs(ref["output"])))
    print(f"history {history}: max error {err:.3e} (2^{np.log2(err):.2f}) of magnitude {mag:.2f}; "
          f"limbs {out.state.cur_limbs}; stages {stages}", flush=True)
    assert err < 2.0**-16  # absolute, in decoded units (the slot scale)
    assert np.max(np.abs(dec.reshape(-1, 8)[:, 1:])) < 2.0**-16  # lanes 1..7 stay empty
    col = history % 128
    last = cache.pages[-1]
    assert last.occupied == col + 1 and cache.content_tokens == history + 1
    kdec = client.decrypt(last.key_groups[1])
    want = Dm.pack_key_page(np.vstack([ck[history - col:history], ref["k"][None, :]]), 1)
    assert np.max(np.abs(kdec - want)) <= 2.0**-20 * np.max(np.abs(want))
