"""CPU tests of the decode layer (config C5): the float64 semantics against an independent
restatement of llama3fhe/approx/layer.py:768-906, the page layout, and the whole encrypted
dataflow run on the slot simulator (tests/slot_sim.py: the layer's own code with exact
(limbs, scale) bookkeeping on float64 slot vectors), which must reproduce the float64 output to
round-off and stay inside the level budget with five refreshes."""

from __future__ import annotations

import math

import numpy as np
import pytest

from holmes_amd import decode as Dm
from holmes_amd.kv_pages import PairFoldCipherPage, PairFoldLayerCache
from holmes_amd.params import CKKSContextSpec

from .slot_sim import SimCt, SlotOps, make_programs

SEED = 20261205


def _setup(intermediate=6144, history=256, seed=SEED):
    spec = Dm.DecodeSpec(intermediate=intermediate)
    rng = np.random.default_rng(seed)
    w = Dm.random_weights(spec, rng)
    x = rng.normal(size=spec.hidden_dim)
    ck = rng.normal(size=(history, 1024))
    cv = rng.normal(size=(history, 1024))
    return spec, w, x, ck, cv


def _chain():
    cs = CKKSContextSpec(depth=23, dnum=3, dcrt_bits=50, first_mod=50, scale_bits=50)
    q, _ = cs.prime_chain()
    return q, 2.0**50


def test_rope_phase_matches_rotate_half():
    """fold * e^(i theta) equals the reference's rotate-half RoPE (attention.py:41-59) written out."""

    spec = Dm.DecodeSpec()
    rng = np.random.default_rng(1)
    v = rng.normal(size=32 * 128)
    pos = 256
    hd = 128
    inv = 1.0 / (np.float32(spec.rope_theta) ** (np.arange(0, hd, 2, dtype=np.float32) / hd))
    ang = np.float32(pos) * inv.astype(np.float32)
    emb = np.concatenate([ang, ang]).astype(np.float32)
    cos, sin = np.cos(emb).astype(np.float64), np.sin(emb).astype(np.float64)
    h = v.reshape(32, 128)
    want = np.empty_like(h)
    want[:, :64] = h[:, :64] * cos[:64] - h[:, 64:] * sin[:64]
    want[:, 64:] = h[:, 64:] * cos[:64] + h[:, :64] * sin[:64]
    got = Dm._rope(v, 32, Dm.rope_phase(pos, spec))
    assert np.allclose(got, want.reshape(-1), atol=1e-12)


def test_numpy_layer_against_direct_restatement():
    """decode_layer_numpy equals a loop-level restatement (per-head dot products, GQA head // 4)
    and its softmax is close to the exact one when the polynomials are in range."""

    spec, w, x, ck, cv = _setup(intermediate=1024, history=20)
    P = Dm.DecodePolynomials.fit(spec)
    out = Dm.decode_layer_numpy(x, ck, cv, w, spec, position=20, polys=P)

    def cheb(v, c, iv):
        return np.polynomial.chebyshev.chebval((2 * v - iv[0] - iv[1]) / (iv[1] - iv[0]), c)

    xn = x * cheb(np.mean(x**2), P.rms, spec.rms_interval) * w.input_layernorm
    q, k, v = w.q_proj @ xn, w.k_proj @ xn, w.v_proj @ xn
    ph = Dm.rope_phase(20, spec)
    q, k = Dm._rope(q, 32, ph), Dm._rope(k, 8, ph)
    keys, vals = np.vstack([ck, k]), np.vstack([cv, v])
    o = np.zeros(4096)
    for h in range(32):
        kvh = h // 4
        s = np.array([q[128 * h:128 * h + 128] @ keys[t, 128 * kvh:128 * kvh + 128] for t in range(keys.shape[0])])
        y = cheb(s / math.sqrt(128) / 2, P.exp, spec.exp_interval)
        lam = cheb(np.sum(y * y), P.rsqrt, spec.rsqrt_interval)
        p = (y * lam) ** 2
        o[128 * h:128 * h + 128] = p @ vals[:, 128 * kvh:128 * kvh + 128]
    h1 = x + w.o_proj @ o
    xn2 = h1 * cheb(np.mean(h1**2), P.rms, spec.rms_interval) * w.post_attention_layernorm
    act = cheb(w.gate_proj @ xn2, P.silu, spec.silu_interval) * (w.up_proj @ xn2)
    want = h1 + w.down_proj @ act
    assert np.allclose(out["output"], want, rtol=1e-10, atol=1e-10)


def test_page_packing_and_matrices_agree():
    """The QKV channel rows read back the folded query / conjugated key / value of every head, the
    page packers put token t of head (g, pair, lane) at page_slot, and the W_O blocks undo the
    z-index fold."""

    spec, w, x, ck, cv = _setup(intermediate=1024, history=4)
    xn = np.random.default_rng(3).normal(size=4096)
    A = Dm.qkv_matrix(w)
    u = A @ xn
    q = w.q_proj @ (xn * w.input_layernorm)
    k = w.k_proj @ (xn * w.input_layernorm)
    g, pair, f, lane, o = 1, 0, 5, 1, 2
    hk = Dm.kv_head(g, pair, lane)
    h = Dm.query_head(g, pair, lane, o)
    assert np.isclose(u[2048 * pair + 32 * f + Dm._q_j(g, lane, o)], q[128 * h + f] + 1j * q[128 * h + 64 + f])
    assert np.isclose(u[2048 * pair + 32 * f + Dm._k_j(g, lane)], k[128 * hk + f] - 1j * k[128 * hk + 64 + f])
    page = Dm.pack_key_page(ck, g)
    assert np.isclose(page[Dm.page_slot(pair, f, 3, lane)], ck[3, 128 * hk + f] - 1j * ck[3, 128 * hk + 64 + f])
    # W_O over z equals the real product over the head outputs
    oa = np.random.default_rng(4).normal(size=4096)
    z = np.zeros(2048, dtype=complex)
    kk = np.arange(2048)
    pr, ff, jj = kk // 1024, (kk // 16) % 64, kk % 16
    hh = Dm.query_head((jj // 4) % 2, pr, jj // 8, jj % 4)
    z[:] = oa[128 * hh + ff] + 1j * oa[128 * hh + 64 + ff]
    b0, b1 = Dm.wo_blocks(w)
    y = np.empty(4096)
    y[0::2] = (b0 @ z).real
    y[1::2] = (b1 @ z).real
    assert np.allclose(y, w.o_proj @ oa)


def test_rotation_set_is_canonical():
    rots = Dm.decode_rotations(pages=3)
    assert all(0 < r < Dm.SLOTS for r in rots) and len(set(rots)) == len(rots)


@pytest.mark.parametrize("history", [256, 200])
def test_decode_layer_on_slot_simulator(history):
    """The encrypted dataflow on exact slot values: output, token page write and level schedule."""

    spec, w, x, ck, cv = _setup(history=history)
    q, S = _chain()
    prog, deep = make_programs(q, 24, S)
    ops = SlotOps(q, prog, deep)
    layer = Dm.DecodeLayer(ops, w, spec)
    pages = []
    for p in range(0, history, 128):
        kt, vt = ck[p:p + 128], cv[p:p + 128]
        kg = [SimCt(Dm.pack_key_page(kt, g), spec.key_limbs, S) for g in range(2)]
        vg = [SimCt(Dm.pack_value_page(vt, g), spec.value_limbs, S) for g in range(2)]
        pages.append(PairFoldCipherPage(kg, vg, kt.shape[0]))
    cache = PairFoldLayerCache(pages=tuple(pages), content_tokens=history)
    xin = SimCt(Dm.lr8(x), 24, S)

    class _CC:  # the cache's partial-page sum
        class fhe:
            @staticmethod
            def homo_add(a, b, ctx):
                return ops.add(a, b)
        context = None

    out, stages, token = layer.forward(xin, cache, position=history, crypto_context=_CC)
    ref = Dm.decode_layer_numpy(x, ck, cv, w, spec, position=history)
    assert all(ref["in_range"].values()), ref["in_range"]
    got = out.values[0, ::8].real
    assert np.max(np.abs(got - ref["output"])) < 1e-9 * np.max(np.abs(ref["output"]))
    assert np.max(np.abs(out.values[0].reshape(-1, 8)[:, 1:])) < 1e-9  # lanes 1..7 stay empty
    assert ops.refreshes == 5 and not ops.log
    assert ops.limbs(out) >= 2
    # the token landed in its page column with the oracle's RoPE'd key and value
    col = history % 128
    last = cache.pages[-1]
    assert last.occupied == col + 1 and cache.content_tokens == history + 1
    k_page = sum(c.values[0] for c in [last.key_groups[0]])
    want = Dm.pack_key_page(np.vstack([np.zeros((col, 1024)), ref["k"][None, :]]), 0)
    if col == 0:
        assert np.allclose(k_page, want, atol=1e-9)
    else:
        prev = Dm.pack_key_page(ck[history - col:history], 0)
        assert np.allclose(k_page, prev + want, atol=1e-9)
    assert ops.limbs(last.key_groups[0]) == spec.key_limbs and ops.limbs(last.value_groups[1]) == spec.value_limbs


def test_two_consecutive_steps_on_slot_simulator():
    """Step two reads the page the first step opened (column 1 of the third page): its output
    follows the float64 semantics over the grown history, and the first step's position-tagged
    constants are gone."""

    spec, w, x, ck, cv = _setup(history=256)
    q, S = _chain()
    prog, deep = make_programs(q, 24, S)
    ops = SlotOps(q, prog, deep)
    layer = Dm.DecodeLayer(ops, w, spec)
    pages = []
    for p in range(0, 256, 128):
        kg = [SimCt(Dm.pack_key_page(ck[p:p + 128], g), spec.key_limbs, S) for g in range(2)]
        vg = [SimCt(Dm.pack_value_page(cv[p:p + 128], g), spec.value_limbs, S) for g in range(2)]
        pages.append(PairFoldCipherPage(kg, vg, 128))
    cache = PairFoldLayerCache(pages=tuple(pages), content_tokens=256)

    class _CC:
        class fhe:
            @staticmethod
            def homo_add(a, b, ctx):
                return ops.add(a, b)
        context = None

    layer.forward(SimCt(Dm.lr8(x), 24, S), cache, position=256, crypto_context=_CC)
    first = Dm.decode_layer_numpy(x, ck, cv, w, spec, position=256)
    x2 = np.random.default_rng(7).normal(size=spec.hidden_dim)
    out, _, _ = layer.forward(SimCt(Dm.lr8(x2), 24, S), cache, position=257, crypto_context=_CC)
    ref = Dm.decode_layer_numpy(x2, np.vstack([ck, first["k"]]), np.vstack([cv, first["v"]]), w, spec,
                                position=257)
    got = out.values[0, ::8].real
    assert np.max(np.abs(got - ref["output"])) < 1e-9 * np.max(np.abs(ref["output"]))
    assert cache.content_tokens == 258 and cache.pages[-1].occupied == 2
    assert not any(isinstance(k, tuple) and k[0] == "route" and k[-1] == 256 for k in layer._consts)
