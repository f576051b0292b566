"""Writes the committed golden vectors with this repository's CPU oracle (oracle/ckks_oracle.c).

  ckks_small.npz  N = 2^8, 4 + 2 primes of 50 bits, alpha 2: every input and output in full
  ckks_prod.json  N = 2^16, 24 + 8 primes of 50 bits, alpha 8 (dnum 3): the prime chain and a
                  sha256 prefix of every output limb; inputs are rebuilt from the seed by
                  golden_inputs.py

The reference holds no residue-level vectors for this path (its tests pin decrypted values only),
so these files pin the oracle and the GPU path against regressions of each other; the oracle's
mathematics is pinned separately by the closed-form tests.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402
from tests.golden import golden_inputs as G  # noqa: E402


def chain(params: dict) -> list[int]:
    p = O.gen_primes(params["log_n"], params["bits"], params["K"])
    q = O.gen_primes(params["log_n"], params["bits"], params["L"], exclude=p)
    return list(q) + list(p)


def run(params: dict, seed: int = G.SEED) -> dict:
    """Every golden operation on one parameter set: {name: (inputs dict, outputs dict)}."""

    primes = chain(params)
    L, K, n = params["L"], params["K"], 1 << params["log_n"]
    orc = O.OracleContext(params["log_n"], L, K, params["alpha"], primes)
    qs = primes[:L]
    out: dict = {"primes": np.array(primes, dtype=np.uint64)}
    r = G.rng(seed, "ntt")
    x = G.uniform(r, qs, (), n)
    out["ntt_in"] = x
    out["ntt_fwd"] = orc.ntt_fwd_limbs(x, list(range(L)))
    out["ntt_inv"] = orc.ntt_inv_limbs(x, list(range(L)))
    s_from, s_to, a, e, g = G.key_inputs(params, primes, 1, seed)
    ksk = orc.make_ksk(s_from, s_to, a, e)
    out["ksk"] = ksk
    r = G.rng(seed, "keyswitch")
    d = G.uniform(r, qs, (), n)
    out["ks_d"] = d
    out["ks_b"], out["ks_a"] = orc.keyswitch(L, d, ksk)
    r = G.rng(seed, "rotate")
    c0, c1 = G.uniform(r, qs, (), n), G.uniform(r, qs, (), n)
    out["rot_c0"], out["rot_c1"] = c0, c1
    out["rot_0"], out["rot_1"] = orc.rotate(L, g, c0, c1, ksk)
    out["rescale"] = orc.rescale(L, out["rot_0"])
    r = G.rng(seed, "encode")
    vals = r.normal(size=n // 2)
    out["enc_values"] = vals
    enc, ok = orc.encode_real(vals, 2.0**40, list(range(L)))
    assert ok
    out["encode"] = enc
    r = G.rng(seed, "mac")
    lm, nb, gg = 2, 2, 2
    pts = G.uniform(r, qs[:lm], (gg * nb,), n)
    baby = G.uniform(r, qs[:lm], (nb, 2), n)
    out["mac_pts"], out["mac_baby"] = pts, baby
    out["mac"] = orc.bsgs_mac(lm, nb, gg, pts, baby)
    return out


OUTPUTS = ("ntt_fwd", "ntt_inv", "ks_b", "ks_a", "rot_0", "rot_1", "rescale", "encode", "mac")


def main() -> None:
    small = run(G.SMALL)
    np.savez_compressed(os.path.join(HERE, "ckks_small.npz"), **small)
    prod = run(G.PROD)
    doc = {
        "params": G.PROD,
        "seed": G.SEED,
        "primes": [int(p) for p in prod["primes"]],
        "hashes": {k: G.limb_hashes(prod[k]) for k in OUTPUTS},
        "note": "sha256(limb as little-endian uint64)[:16] per output limb; inputs from golden_inputs.py",
    }
    with open(os.path.join(HERE, "ckks_prod.json"), "w") as f:
        json.dump(doc, f, indent=1)
    print("wrote ckks_small.npz and ckks_prod.json")


if __name__ == "__main__":
    main()
