"""CPU tests of the host-side boundary logic (no GPU): name normalisation, plaintext cache policy,
default rotation sets, configuration, the prime-chain rule and the encoder."""

import numpy as np
import pytest

from holmes_amd import backend, encoding
from holmes_amd.config import SimulatorConfig
from holmes_amd.params import CKKSContextSpec, ntt_primes
from oracle import oracle as O


def test_constant_names_normalise_layer_and_rank_prefixes():
    n = backend._normalized_constant_name
    assert n("model.layers.7.attn.mask") == n("model.layers.31.attn.mask")
    assert n("t2l.r3.i9.mask") == n("t2l.r0.i1.mask")
    assert n(("a", ["model.layers.1.x"])) == ("a", ("model.layers.*.x",))


def test_plaintext_cache_is_first_fit_and_capped():
    cache = backend.SessionPlaintextCache(limit_bytes=100, max_source_bytes=60)
    made = []

    def factory(admit):
        made.append(admit)
        return object()

    a = cache.get("a", factory, source_bytes=50)
    assert cache.get("a", factory, source_bytes=50) is a
    cache.get("b", factory, source_bytes=60)  # would cross 100: transient, not admitted
    assert made == [True, False]
    assert cache.info()["entries"] == 1 and cache.info()["hits"] == 1 and cache.info()["skips"] == 1
    assert not cache.accepts_source(61)
    cache.clear()
    with pytest.raises(RuntimeError):
        cache.get("c", factory, source_bytes=1)


def test_default_rotations_match_reference_rule():
    # block_out * 2^i for i < log2(input_dim), plus 2^i for i < log2(block_out)
    assert backend.default_rotations(16, 4) == {4, 8, 16, 32, 1, 2}
    with pytest.raises(ValueError):
        backend.default_rotations(12, 4)


def test_simulator_config_validation():
    cfg = SimulatorConfig()
    cfg.validate()
    assert cfg.rescale_policy() == "manual"
    # the reference's defaults (llama3fhe/config.py:18-22): depth 37, 59-bit primes, 60-bit first modulus
    assert (cfg.maxLevelsRemaining, cfg.dnum, cfg.dcrtBits, cfg.firstMod) == (37, 3, 59, 60)
    assert cfg.scale_bits() == 59 and SimulatorConfig(scaleBits=40).scale_bits() == 40
    with pytest.raises(ValueError):
        SimulatorConfig(rescaleTech="BOGUS").rescale_policy()


def test_spec_prime_chain_follows_oracle_rule():
    spec = CKKSContextSpec(depth=23, dnum=3)
    q, p = spec.prime_chain()
    assert len(q) == 24 and len(p) == 8 and spec.alpha == 8
    assert p == O.gen_primes(16, 50, 8)
    assert q == O.gen_primes(16, 50, 24, exclude=p)
    assert ntt_primes(16, 50, 3) == O.gen_primes(16, 50, 3)
    # the reference's production chain (assets/feature_major.json): 60-bit q_0 and specials, 59-bit rest
    wide = CKKSContextSpec(depth=37, dnum=5, dcrt_bits=59, first_mod=60)
    wide.validate()
    q, p = wide.prime_chain()
    assert len(q) == 38 and len(p) == 8 and wide.alpha == 8
    assert p == O.gen_primes(16, 60, 8) and q[:1] == O.gen_primes(16, 60, 1, exclude=p)
    assert q[1:] == O.gen_primes(16, 59, 37, exclude=p + q[:1])
    assert [x.bit_length() for x in q[:2]] == [60, 59] and all(x.bit_length() == 60 for x in p)
    for bits in (61, 31):
        with pytest.raises(ValueError):
            CKKSContextSpec(dcrt_bits=bits).validate()


@pytest.mark.parametrize("slots", [32768, 4096])
def test_encode_decode_roundtrip_and_rotation_group(slots):
    rng = np.random.default_rng(slots)
    z = rng.normal(size=slots) + 1j * rng.normal(size=slots)
    m = encoding.encode(z, 2.0**40, 16, slots)
    back = encoding.decode(m, 2.0**40, 16, slots)
    assert np.max(np.abs(back - z)) < 2.0**-30
    # X -> X^5 on the coefficients rotates the slots left by one
    n = 1 << 16
    idx = (np.arange(n) * 5) % (2 * n)
    m5 = np.zeros(n)
    wrap = idx >= n
    m5[idx[~wrap]] = m[~wrap]
    m5[idx[wrap] - n] = -m[wrap]
    rot = encoding.decode(m5, 2.0**40, 16, slots)
    assert np.max(np.abs(rot - np.roll(z, -1))) < 2.0**-30


def test_encoder_cap():
    with pytest.raises(ValueError):
        encoding.encode(np.full(8, 1e9), 2.0**40, 16, 8)


def test_feature_major_layout_roundtrip_and_slot_rule():
    from holmes_amd.layouts import FeatureMajorPrefillLayout

    lay = FeatureMajorPrefillLayout()
    assert lay.tokens_per_cipher == 8 and lay.cipher_count == 16
    rng = np.random.default_rng(1)
    rows = rng.normal(size=(128, 4096))
    packed = lay.pack(rows)
    assert packed.shape == (16, 32768)
    assert packed[3, lay.slot(17, 5)] == rows[3 * 8 + 5, 17]
    assert np.array_equal(lay.unpack(packed), rows)
    small = FeatureMajorPrefillLayout(seq_len=5, hidden_dim=16, slots=64)
    r = rng.normal(size=(5, 16))
    assert np.array_equal(small.unpack(small.pack(r)), r)
    with pytest.raises(ValueError):
        FeatureMajorPrefillLayout(hidden_dim=12)


def test_easyfhe_alias_binds_the_hot_path_surface():
    from holmes_amd import easyfhe_compat

    easyfhe_compat.install()
    try:
        from easyfhe import fhe  # noqa: F401  (the import llama3fhe's operators make)
        import easyfhe

        import holmes_amd.fhe as ours

        assert fhe is easyfhe.fhe and fhe.homo_rotate is ours.homo_rotate
        for name in ("CKKSContextSpec", "generate_client_context", "CipherState", "ConstantBundle", "PackedRaw",
                     "homo_rotate", "prepare_hoisted_baby_rotations", "hoisted_mac_sum", "rescale", "align_to",
                     "homo_add", "homo_sub", "homo_mul_i", "homo_mul_pt", "fast_rotate", "grouped_pairwise_mac",
                     "moddown_from_ext", "pack_cipher_batch", "unpack_cipher_batch"):
            assert callable(getattr(fhe, name)), name
        assert easyfhe.uint64 is not None and easyfhe.get_device_module("cuda") is not None
    finally:
        easyfhe_compat.uninstall()


def test_scalar_encoding_residues_and_rounding():
    from types import SimpleNamespace

    from holmes_amd import fhe

    primes = [1125899906826241, 1125899906629633, 1125899906301953]
    ctx = SimpleNamespace(q_primes=primes)
    sf = 2.0**40
    r = fhe._scalar_residues(0.5, 3, sf, False, ctx)
    assert [int(v) for v in r[0]] == [2**39 % q for q in primes]
    r = fhe._scalar_residues(-1.5, 2, sf, False, ctx)
    assert [int(v) for v in r[0]] == [(-3 * 2**39) % q for q in primes[:2]]
    # round half away from zero, as the encoder
    assert fhe._scaled_int(2.5, 1.0, False) == 3 and fhe._scaled_int(-2.5, 1.0, False) == -3
    assert fhe._scaled_int(7, 1.0, True) == 7
    with pytest.raises(ValueError):
        fhe._scaled_int(2.5, 1.0, True)  # integer mode needs an integral value
    with pytest.raises(ValueError):
        fhe._scaled_int(1.0, 2.0**61, False)  # beyond the 2^61 encoding cap
    # a scalar (one exactly reduced integer) may exceed 2^61 up to a quarter of the level's modulus
    big = fhe._scalar_residues(4.0, 2, 2.0**60, False, ctx)
    assert [int(v) for v in big[0]] == [2**62 % q for q in primes[:2]]
    with pytest.raises(ValueError):
        fhe._scalar_residues(1.0, 1, 2.0**62, False, ctx)  # one limb: 2^61 stays the limit
    tab = fhe._scalar_residues(np.array([1.0, -1.0]), 3, 4.0, False, ctx)
    assert tab.shape == (2, 3) and int(tab[1, 0]) == primes[0] - 4


def test_joined_components_view_without_copy():
    # components allocated back to back are rescaled as one batch through a strided view; anything
    # else is refused (and the caller falls back to a concatenation)
    import torch

    from holmes_amd.fhe import _joined

    n = 8
    buf = torch.arange(2 * 3 * 5 * n, dtype=torch.int64).reshape(2, 3, 5, n)
    v = _joined([buf[0], buf[1]], 4, n)
    assert v is not None and v.shape == (6, 4, n)
    assert torch.equal(v, torch.cat([buf[0, :, :4], buf[1, :, :4]], 0))
    one = torch.arange(2 * 1 * 5 * n, dtype=torch.int64).reshape(2, 1, 5, n)
    assert torch.equal(_joined([one[0], one[1]], 5, n), one.reshape(2, 5, n))
    other = torch.zeros(3, 5, n, dtype=torch.int64)
    assert _joined([buf[0], other], 4, n) is None
    assert _joined([buf[1], buf[0]], 4, n) is None
    gapped = torch.zeros(3, 3, 5, n, dtype=torch.int64)
    assert _joined([gapped[0], gapped[2]], 4, n) is None


def test_admitted_bundle_keeps_encodings_only_within_the_budget(monkeypatch):
    """An admitted bundle asks the session budget before it keeps an encoding: past the budget the
    encoding is returned but not kept, and the bundle stays cached."""
    from types import SimpleNamespace

    from holmes_amd import fhe

    class FakePt:
        def __init__(self, n):
            import torch

            self.cv = [torch.zeros(n, dtype=torch.int64)]

    sizes = iter([4, 4, 4])
    monkeypatch.setattr(fhe, "encode_plaintext", lambda v, state, slots, ctx, is_ext=False: FakePt(next(sizes)))
    cache = backend.SessionPlaintextCache(limit_bytes=100, max_source_bytes=100)
    sess = SimpleNamespace(plaintext_cache=cache)
    bundle = backend.EasyFHEContext.constant_bundle(sess, {"m": np.zeros(4)}, cache_key="model.layers.3.mask")
    assert cache.info()["bytes"] == 32  # the 4 float64 source values
    st = fhe.CipherState(cur_limbs=3, scale_degree=1, scaling_factor=2.0**40)
    a = bundle.plaintext("m", st, 8, None)
    assert bundle.plaintext("m", st, 8, None) is a and cache.info()["bytes"] == 64
    b = bundle.plaintext("m", st.replace(cur_limbs=2), 8, None)  # 32 more bytes: still fits (96)
    assert cache.info()["bytes"] == 96
    c = bundle.plaintext("m", st.replace(cur_limbs=1), 8, None)  # would reach 128: not kept
    assert bundle.plaintext("m", st.replace(cur_limbs=2), 8, None) is b and c is not None
    assert bundle.cache_info()["entries"] == 2
    # the same constant from another layer is a hit
    again = backend.EasyFHEContext.constant_bundle(sess, {"m": np.zeros(4)}, cache_key="model.layers.9.mask")
    assert again is bundle and cache.info()["hits"] == 1
