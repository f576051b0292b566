"""The ``fhe`` operation namespace Holmes' operators call (``from easyfhe import fhe``).

Same names and keywords as the calls in llama3fhe (CKKSContextSpec / generate_client_context:
llama3fhe/backend.py:574-588; homo_rotate: operators/linear/operator.py:446-453; rescale:
operator.py:387-394; align_to: operators/primitives.py:125-131; homo_add / homo_sub / homo_mul_i:
operators/linear/complex.py:29-74; homo_mul_pt: operators/linear/prefill/output.py:450).  Every
op returns a new owned ciphertext and enqueues HIP kernels on the current stream; nothing
synchronises the host.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _native as nat
from . import encoding
from .client import Client
from .context import Cipher, CipherState, CKKSContext
from .params import CKKSContextSpec

__all__ = [
    "CKKSContextSpec",
    "CipherState",
    "Cipher",
    "Plaintext",
    "generate_client_context",
    "homo_rotate",
    "homo_rotate_batch",
    "keyswitch_batch",
    "rescale",
    "align_to",
    "homo_add",
    "homo_sub",
    "homo_neg",
    "homo_mul_i",
    "homo_mul_pt",
    "encode_plaintext",
    "PackedRaw",
    "ConstantBundle",
]


class Plaintext:
    """An encoded plaintext: ``cv = [p]``, ``[batch][limbs][N]`` uint64 in the NTT domain."""

    __slots__ = ("cv", "state", "slots", "is_ext", "batch_size")

    def __init__(self, poly: torch.Tensor, state: CipherState, *, slots: int, is_ext: bool = False):
        self.cv = [poly]
        self.state = state
        self.slots = int(slots)
        self.is_ext = bool(is_ext)
        self.batch_size = int(poly.shape[0])

    def release(self) -> None:
        self.cv = []


def generate_client_context(spec: CKKSContextSpec, device: str = "cuda"):
    """Build the context (device tables) and the client (secret key); generate the requested
    rotation keys when ``spec.auto_load_keys``.  Returns ``(client, context)``."""

    ctx = CKKSContext(spec, device=device)
    client = Client(ctx)
    if spec.auto_load_keys and spec.rotations:
        client.generate_rotation_keys(spec.rotations)
    return client, ctx


def _limbs(ct) -> int:
    return int(ct.state.cur_limbs)


def _view(t: torch.Tensor, limbs: int) -> torch.Tensor:
    return t[:, :limbs]


def _galois(rotation: int, ctx: CKKSContext) -> int:
    r = int(rotation)
    if r == ctx.M - 1:
        return ctx.M - 1
    return ctx.galois_element(r)


def homo_rotate(ct: Cipher, k: int, ctx: CKKSContext) -> Cipher:
    """Left-rotate every slot vector of ``ct`` by ``k`` (``k = M - 1``: complex conjugation)."""

    if ct.is_ext:
        raise ValueError("homo_rotate expects a non-extended ciphertext")
    limbs = _limbs(ct)
    if int(k) % ctx.max_slots == 0 and int(k) != ctx.M - 1:
        return ct.deep_copy()
    g = _galois(k, ctx)
    key = ctx.key_for_galois(g)
    out0, out1 = ctx.rotate_raw(_view(ct.cv[0], limbs), _view(ct.cv[1], limbs), limbs, g, key)
    return ct.cipher_like([out0, out1])


def homo_rotate_batch(ct: Cipher, rotations, ctx: CKKSContext) -> Cipher:
    """Rotate batch item b of ``ct`` by ``rotations[b]`` in one batched key switch (each item its
    own key, as the batched giant step of bench/cmp/holmes_multi_mac.py:180-186)."""

    limbs = _limbs(ct)
    B = ct.batch_size
    rotations = list(rotations)
    if len(rotations) != B:
        raise ValueError("one rotation per batch item")
    gs = [_galois(r, ctx) for r in rotations]
    c0, c1 = _view(ct.cv[0], limbs), _view(ct.cv[1], limbs)
    r0 = ctx.empty(B, limbs, ctx.N)
    r1 = ctx.empty(B, limbs, ctx.N)
    for b, g in enumerate(gs):
        ctx.automorphism(c0[b:b + 1], g, limbs, out=r0[b:b + 1])
        ctx.automorphism(c1[b:b + 1], g, limbs, out=r1[b:b + 1])
    keys = [ctx.key_for_galois(g) for g in gs]
    out0, out1 = ctx.keyswitch(r1, limbs, keys, add=r0)
    return ct.cipher_like([out0, out1])


def keyswitch_batch(d: torch.Tensor, limbs: int, keys, ctx: CKKSContext):
    """(b, a) = KeySwitch(d[i], keys[i]) for every batch item: ModUp, key inner product, ModDown."""

    return ctx.keyswitch(d, int(limbs), keys)


def rescale(ct: Cipher, ctx: CKKSContext) -> Cipher:
    """Divide by the last prime: ``cur_limbs`` -> ``cur_limbs - 1``, scale / q_last."""

    limbs = _limbs(ct)
    if ct.is_ext or limbs < 2:
        raise ValueError("rescale needs a non-extended ciphertext with at least two limbs")
    both = torch.cat([_view(c, limbs) for c in ct.cv], 0) if len(ct.cv) > 1 else _view(ct.cv[0], limbs)
    out = ctx.rescale_raw(both.contiguous(), limbs)
    B = ct.batch_size
    parts = [out[i * B:(i + 1) * B] for i in range(len(ct.cv))]
    st = ct.state
    state = st.replace(
        cur_limbs=limbs - 1,
        scale_degree=max(1, int(st.scale_degree) - 1),
        scaling_factor=float(st.scaling_factor) / float(ctx.rescale_divisor_at(limbs)),
    )
    return ct.cipher_like(parts, state=state)


def align_to(ct: Cipher, state: CipherState, ctx: CKKSContext) -> Cipher:
    """Drop limbs (no depth consumed) down to ``state.cur_limbs``; the scale is unchanged."""

    limbs = _limbs(ct)
    target = int(state.cur_limbs)
    if target > limbs:
        raise ValueError(f"cannot raise a ciphertext from {limbs} to {target} limbs")
    return ct.cipher_like([_view(c, target).clone() for c in ct.cv], state=ct.state.replace(cur_limbs=target))


def _binary(a: Cipher, b: Cipher, ctx: CKKSContext, op: int) -> Cipher:
    if a.is_ext or b.is_ext:
        raise ValueError("add/sub expect non-extended ciphertexts")
    if int(a.state.scale_degree) != int(b.state.scale_degree):
        raise ValueError("scale degrees differ")
    fa, fb = float(a.state.scaling_factor), float(b.state.scaling_factor)
    if abs(fa - fb) > 1e-9 * max(fa, fb):
        raise ValueError(f"scaling factors differ ({fa} vs {fb})")
    limbs = min(_limbs(a), _limbs(b))
    idx = ctx.q_prime_idx(limbs)
    out = []
    for x, y in zip(a.cv, b.cv):
        o = ctx.empty(x.shape[0], limbs, ctx.N)
        ctx.poly_op(op, o, _view(x, limbs), _view(y, limbs), prime_idx=idx)
        out.append(o)
    return a.cipher_like(out, state=a.state.replace(cur_limbs=limbs))


def homo_add(a: Cipher, b: Cipher, ctx: CKKSContext) -> Cipher:
    return _binary(a, b, ctx, nat.HCK_OP_ADD)


def homo_sub(a: Cipher, b: Cipher, ctx: CKKSContext) -> Cipher:
    return _binary(a, b, ctx, nat.HCK_OP_SUB)


def homo_neg(a: Cipher, ctx: CKKSContext) -> Cipher:
    limbs = _limbs(a)
    idx = ctx.q_prime_idx(limbs)
    out = []
    for x in a.cv:
        o = ctx.empty(x.shape[0], limbs, ctx.N)
        ctx.poly_op(nat.HCK_OP_NEG, o, _view(x, limbs), prime_idx=idx)
        out.append(o)
    return a.cipher_like(out)


def homo_mul_i(ct: Cipher, ctx: CKKSContext, negative: bool = False) -> Cipher:
    """Multiply the slots by i (or -i): the monomial X^(N/2), exact, no depth."""

    limbs = _limbs(ct)
    idx = ctx.q_prime_idx(limbs)
    out = []
    for x in ct.cv:
        o = ctx.empty(x.shape[0], limbs, ctx.N)
        ctx.poly_op(nat.HCK_OP_MUL_XHALF, o, _view(x, limbs), prime_idx=idx)
        if negative:
            ctx.poly_op(nat.HCK_OP_NEG, o, o, prime_idx=idx)
        out.append(o)
    return ct.cipher_like(out)


def encode_plaintext(values, state: CipherState, slots: int, ctx: CKKSContext) -> Plaintext:
    """Encode real/complex ``values`` at ``state`` (limbs, scale) into the NTT domain."""

    vals = np.asarray(values)
    rows = vals.reshape(1, -1) if vals.ndim <= 1 else vals.reshape(vals.shape[0], -1)
    m = np.stack([encoding.encode(r, float(state.scaling_factor), ctx.logN, slots) for r in rows])
    limbs = int(state.cur_limbs)
    idx = ctx.q_prime_idx(limbs)
    poly = ctx.from_signed(torch.from_numpy(m).to(ctx.device), idx)
    ctx.ntt(poly, prime_idx=idx)
    return Plaintext(poly, state, slots=slots)


def homo_mul_pt(ct: Cipher, pt: Plaintext, ctx: CKKSContext) -> Cipher:
    """Slotwise ciphertext x plaintext product (scale degrees and factors multiply)."""

    limbs = min(_limbs(ct), int(pt.state.cur_limbs))
    idx = ctx.q_prime_idx(limbs)
    p = _view(pt.cv[0], limbs)
    if p.shape[0] not in (1, ct.batch_size):
        raise ValueError("plaintext batch must be 1 or the ciphertext batch")
    if p.shape[0] == 1 and ct.batch_size > 1:
        p = p.expand(ct.batch_size, -1, -1)
    p = p.contiguous()
    out = []
    for x in ct.cv:
        o = ctx.empty(x.shape[0], limbs, ctx.N)
        ctx.poly_op(nat.HCK_OP_MUL, o, _view(x, limbs), p, prime_idx=idx)
        out.append(o)
    st = ct.state
    state = st.replace(
        cur_limbs=limbs,
        scale_degree=int(st.scale_degree) + int(pt.state.scale_degree),
        scaling_factor=float(st.scaling_factor) * float(pt.state.scaling_factor),
    )
    return ct.cipher_like(out, state=state)


class PackedRaw:
    """Raw slot values of one constant (a float/complex vector or a [rows][slots] array)."""

    def __init__(self, values):
        self.values = values

    def numpy(self) -> np.ndarray:
        v = self.values
        if hasattr(v, "detach"):
            v = v.detach().cpu().numpy()
        return np.asarray(v)


class ConstantBundle:
    """Named constants encoded on demand (``bundle.plaintext(name, state, slots, context, ...)``,
    llama3fhe/backend.py:346-356, operators/linear/weight.py:458-469).  ``cache_mode="plain"``
    keeps each encoded plaintext for reuse; ``"none"`` encodes every call."""

    def __init__(self, vectors: dict, cache_mode: str = "none"):
        self.vectors = dict(vectors)
        self.cache_mode = str(cache_mode)
        self._cache: dict = {}

    def plaintext(self, name: str, state: CipherState, slots: int, context: CKKSContext,
                  is_ext: bool = False, cache: bool | None = None) -> Plaintext:
        if is_ext:
            raise ValueError("extended-basis plaintexts are not supported by this backend")
        key = (str(name), int(state.cur_limbs), float(state.scaling_factor), int(slots))
        keep = self.cache_mode in ("plain", "both") if cache is None else bool(cache)
        hit = self._cache.get(key)
        if hit is not None:
            return hit
        pt = encode_plaintext(self.vectors[str(name)].numpy(), state, int(slots), context)
        if keep:
            self._cache[key] = pt
        return pt

    def cache_info(self) -> dict:
        total = sum(int(pt.cv[0].numel()) * 8 for pt in self._cache.values())
        return {"entries": len(self._cache), "total_bytes": total}

    def clear_cache(self) -> None:
        self._cache.clear()
