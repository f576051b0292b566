"""The ConstantBundle surface of the reference (llama3fhe/operators/linear/weight.py:458-469,
nonlinear/polynomial.py:274-291) on the host: UnpackedRaw packs lazily and once per slot count,
encoded_scalars is one residue table equal to encoding each name alone, honouring cache_mode."""

import types

import numpy as np

from holmes_amd import fhe
from holmes_amd.params import CKKSContextSpec


def _ctx():
    q, _ = CKKSContextSpec(depth=23, dcrt_bits=50, first_mod=50).prime_chain()
    return types.SimpleNamespace(q_primes=q, scale_at=lambda l: 2.0**40)


def test_unpacked_raw_packs_once_on_first_encode(monkeypatch):
    calls, seen = [], []

    def packer(src, slots, context):
        calls.append(slots)
        return np.full(slots, float(src))

    monkeypatch.setattr(fhe, "encode_plaintext", lambda v, state, slots, ctx, is_ext=False: seen.append(v) or v)
    raw = fhe.UnpackedRaw(3.0, packer)
    bundle = fhe.ConstantBundle(vectors={"w": raw}, cache_mode="none")
    assert calls == []
    st = fhe.CipherState(cur_limbs=4, scale_degree=1, scaling_factor=2.0**40)
    bundle.plaintext("w", st, 16, None)
    bundle.plaintext("w", st.replace(cur_limbs=3), 16, None)
    assert calls == [16] and len(seen) == 2 and np.all(seen[0] == 3.0)


def test_encoded_scalars_table_matches_single_encodings():
    ctx = _ctx()
    names = ("a", "b", "c")
    vals = {"a": 0.5, "b": -1.25, "c": 3e-3}
    bundle = fhe.ConstantBundle(scalars=vals, cache_mode="plain")
    enc = bundle.encoded_scalars(names, cur_limbs=5, scale_degree=1, context=ctx, scaling_factor=2.0**45)
    assert tuple(enc.residues.shape) == (3, 5) and enc.cur_limbs == 5 and enc.scaling_factor == 2.0**45
    for i, n in enumerate(names):
        one = fhe.encode_scalar(vals[n], 5, 1, 2.0**45, context=ctx)
        assert np.array_equal(enc.residues[i].numpy(), one.residues.numpy())
    assert bundle.encoded_scalars(names, cur_limbs=5, scale_degree=1, context=ctx, scaling_factor=2.0**45) is enc
    fresh = fhe.ConstantBundle(scalars=vals, cache_mode="none")
    e1 = fresh.encoded_scalars(names, cur_limbs=5, context=ctx, scaling_factor=2.0**45)
    assert fresh.encoded_scalars(names, cur_limbs=5, context=ctx, scaling_factor=2.0**45) is not e1
