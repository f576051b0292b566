"""GPU check of the encrypted MLP block (feature-major, 128 tokens x 4096 features, N = 2^16,
24 x 50-bit limbs, scale 2^50, sparse secret): RMSNorm (degree-15 inverse square root), gate/up
projections over two feature pages (the second half zero-padded), SiLU (degree-63 Chebyshev on
[-16, 16]), the product, the down projection, and the two-pass bootstrap of the output -- every
decrypted slot within 2^-16 of the float64 oracle that applies the same polynomials; both carriers
(token ciphertexts paired as x + i y with one gate + i up projection per page, and real pages)."""

import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def env():
    from holmes_amd import bootstrap as bs
    from holmes_amd import fhe, mlp

    spec = fhe.CKKSContextSpec(depth=23, dnum=3, dcrt_bits=50, first_mod=50, scale_bits=50,
                               secret_key_dist="SPARSE_TERNARY", hamming_weight=192, seed=20261204)
    client, ctx = fhe.generate_client_context(spec, device="cuda")
    mspec = mlp.MLPBlockSpec(intermediate_width=6144)
    bspec = bs.BootstrapSpec(log_slots=15, level_budget=(3, 3))
    from holmes_amd.layouts import FeatureMajorPrefillLayout

    layout = FeatureMajorPrefillLayout()
    cfg = mlp.default_config()
    rots = set(mlp.FeatureMajorMLPBlock.rotations(mspec, layout, cfg)) | set(bs.requirements(bspec, 16).rotations)
    client.generate_rotation_keys(sorted(rots))
    prog = bs.generate(ctx, bspec)
    rng = np.random.default_rng(7)
    D, Iw = 4096, mspec.intermediate_width
    gate, up = rng.normal(scale=0.02, size=(2, Iw, D))
    down = rng.normal(scale=0.02, size=(D, Iw))
    gamma = 1.0 + 0.1 * rng.normal(size=D)
    block = mlp.FeatureMajorMLPBlock(ctx, gate, up, down, norm_weight=gamma, spec=mspec, layout=layout, config=cfg,
                                     bootstrap_program=prog)
    x = rng.normal(size=(128, D))
    cts = [client.encrypt(row, cur_limbs=ctx.L) for row in layout.pack(x)]
    want = layout.pack(mlp.mlp_block_numpy(x, gate, up, down, gamma, mspec))
    real = mlp.FeatureMajorMLPBlock(ctx, gate, up, down, norm_weight=gamma, layout=layout, config=cfg,
                                    spec=mlp.MLPBlockSpec(intermediate_width=6144, paired=False))
    return mlp, client, ctx, block, cts, want, real


def test_real_pages_agree(env):
    # the separate gate / up projections on real token ciphertexts: the same block, the other carrier
    mlp, client, ctx, block, cts, want, real = env
    out, times = real.forward(cts)
    err = max(float(np.max(np.abs(client.decrypt(o).real - want[i]))) for i, o in enumerate(out))
    print(f"MLP block (real pages): max error 2^{math.log2(err):.1f}, stages {times}")
    assert err < 2.0**-16


def test_mlp_block_without_refresh(env):
    mlp, client, ctx, block, cts, want, real = env
    prog, block.bootstrap_program = block.bootstrap_program, None
    try:
        out, times = block.forward(cts)
    finally:
        block.bootstrap_program = prog
    assert len(out) == 16 and out[0].state.cur_limbs == 5
    err = max(float(np.max(np.abs(client.decrypt(o).real - want[i]))) for i, o in enumerate(out))
    print(f"MLP block (no refresh): max error 2^{math.log2(err):.1f}, stages {times}")
    assert err < 2.0**-16


def test_mlp_block_with_refresh(env):
    mlp, client, ctx, block, cts, want, real = env
    out, times = block.forward(cts)
    assert out[0].state.cur_limbs == 8
    err = max(float(np.max(np.abs(client.decrypt(o).real - want[i]))) for i, o in enumerate(out))
    print(f"MLP block: max error 2^{math.log2(err):.1f}, stages {times}")
    assert err < 2.0**-16
