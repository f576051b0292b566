"""The CPU oracle reproduces the committed golden vectors (tests/golden), bit for bit.

The small set holds every input and output in full; the production set (N = 2^16, 24 + 8
primes, dnum 3) holds per-limb hashes.  A change to the oracle that moves any residue fails
here; what the residues should be is pinned by the closed-form oracle tests."""

import json
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.golden import golden_inputs as G
from tests.golden import make_golden as M

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def oracle_built():
    O.build()
    return True


def test_small_vectors_full(oracle_built):
    want = np.load(os.path.join(HERE, "ckks_small.npz"))
    got = M.run(G.SMALL)
    assert set(want.files) == set(got)
    for k in want.files:
        assert np.array_equal(want[k], got[k]), k


def test_small_vectors_self_consistent(oracle_built):
    """Relations among the stored arrays that hold whatever the oracle's internals:
    INTT(NTT(x)) = x per limb, and the MAC is the plain modular sum of products."""

    v = np.load(os.path.join(HERE, "ckks_small.npz"))
    primes = [int(p) for p in v["primes"]]
    p = G.SMALL
    orc = O.OracleContext(p["log_n"], p["L"], p["K"], p["alpha"], primes)
    back = orc.ntt_inv_limbs(v["ntt_fwd"], list(range(p["L"])))
    assert np.array_equal(back, v["ntt_in"])
    q = np.array(primes[:2], dtype=object).reshape(2, 1)
    pts, baby, mac = v["mac_pts"], v["mac_baby"], v["mac"]
    for g in range(2):
        for c in range(2):
            acc = np.zeros((2, pts.shape[-1]), dtype=object)
            for b in range(2):
                acc = (acc + pts[g * 2 + b].astype(object) * baby[b, c].astype(object)) % q
            assert np.array_equal(mac[c, g].astype(object), acc)


def test_production_hashes(oracle_built):
    with open(os.path.join(HERE, "ckks_prod.json")) as f:
        doc = json.load(f)
    assert doc["params"] == G.PROD and doc["seed"] == G.SEED
    got = M.run(G.PROD)
    assert [int(x) for x in got["primes"]] == doc["primes"]
    for k, hashes in doc["hashes"].items():
        assert G.limb_hashes(got[k]) == hashes, k


def test_production_chain_matches_context_spec():
    from holmes_amd.params import CKKSContextSpec

    with open(os.path.join(HERE, "ckks_prod.json")) as f:
        doc = json.load(f)
    spec = CKKSContextSpec(depth=23, dnum=3, dcrt_bits=50, first_mod=50)
    q, p = spec.prime_chain()
    assert [int(x) for x in q + p] == doc["primes"]
