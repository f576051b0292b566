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
from .client import Client
from .context import Cipher, CipherState, CKKSContext, u64_cat, u64_clone, u64_copy
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
    "pack_cipher_batch",
    "unpack_cipher_batch",
    "fast_rotate",
    "moddown_from_ext",
    "grouped_pairwise_mac",
    "prepare_hoisted_baby_rotations",
    "hoisted_mac_sum",
    "EncodedScalar",
    "encode_scalar",
    "homo_mul_scalar",
    "homo_mul_scalar_rescale",
    "homo_add_scalar",
    "homo_add_pt",
    "homo_mul_no_relin",
    "homo_relinearize",
    "homo_mul_relin",
    "homo_mul_relin_rescale",
    "homo_mul_relin_rescale_postop",
    "grouped_scalar_weighted_acc",
    "cipher_batch_item",
]

# Fixed-scale mode (scale_mode "fixed"): a product rescaled by a prime q_l carries the exact scale
# s_a s_b / q_l, which differs from the nominal scale by |q_l / 2^bits - 1| (below 2^-32 for the
# chain's NTT primes when the scale matches the prime size).  Additions accept scales equal to
# this relative tolerance and keep the left operand's scale, as the reference's Chebyshev
# recurrence requires (T_k = 2 T_a T_b - T_1, llama3fhe/operators/nonlinear/polynomial.py:140-160).
SCALE_RTOL = 2.0**-20


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
    """Build the context (device tables) and the client (secret key) with the relinearisation key;
    generate the requested rotation keys when ``spec.auto_load_keys``.  Returns
    ``(client, context)``."""

    ctx = CKKSContext(spec, device=device)
    client = Client(ctx)
    ctx.relin_key = client.relin_key()
    if spec.auto_load_keys and spec.rotations:
        client.generate_rotation_keys(spec.rotations)
    return client, ctx


def _limbs(ct) -> int:
    return int(ct.state.cur_limbs)


def _view(t: torch.Tensor, limbs: int) -> torch.Tensor:
    return t[:, :limbs]


def _alloc(ctx: CKKSContext, comps: int, batch: int, limbs: int) -> list:
    """Output components as views of one [comps][batch][limbs][N] buffer: back to back, so a later
    rescale (or any per-poly kernel) takes them as one batch without a copy."""

    buf = ctx.empty(comps, batch, limbs, ctx.N)
    return [buf[c] for c in range(comps)]


def _joined(cv, limbs: int, n: int):
    """The components as one [comps * batch][limbs][N] view when they sit back to back in one buffer
    with one item stride (as ``_alloc`` leaves them); None otherwise."""

    t0 = cv[0]
    B = int(t0.shape[0])
    if len(cv) == 1:
        return t0[:, :limbs]
    gap = (cv[1].data_ptr() - t0.data_ptr()) // 8
    if gap <= 0 or gap % B:
        return None
    s = gap // B  # item stride in elements
    if s < limbs * n:
        return None
    for i, t in enumerate(cv):
        if (t.shape != t0.shape or t.dtype != t0.dtype or t.stride(1) != n or t.stride(2) != 1
                or (B > 1 and t.stride(0) != s) or t.data_ptr() != t0.data_ptr() + i * gap * 8
                or t.untyped_storage().data_ptr() != t0.untyped_storage().data_ptr()):
            return None
    return torch.as_strided(t0, (len(cv) * B, limbs, n), (s, n, 1))


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
    both = _joined(ct.cv, limbs, ctx.N)
    B = ct.batch_size
    if both is not None:
        out = ctx.rescale_raw(both, limbs)
    else:
        # components in separate buffers: each rescaled into its half of one output (no copy of
        # the input into a joint buffer first)
        out = ctx.empty(len(ct.cv) * B, limbs - 1, ctx.N)
        for i, c in enumerate(ct.cv):
            ctx.rescale_raw(_view(c, limbs), limbs, out=out[i * B:(i + 1) * B])
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
    out = _alloc(ctx, len(ct.cv), ct.batch_size if not ct.is_ext else int(ct.cv[0].shape[0]), target)
    for o, c in zip(out, ct.cv):
        u64_copy(o, _view(c, target))
    return ct.cipher_like(out, state=ct.state.replace(cur_limbs=target))


def _same_scale(fa: float, fb: float) -> bool:
    return abs(fa - fb) <= SCALE_RTOL * max(abs(fa), abs(fb))


def _binary(a: Cipher, b: Cipher, ctx: CKKSContext, op: int) -> Cipher:
    """a op b componentwise; a two-component operand meets a three-component one (a product before
    relinearisation) with a zero third component."""

    if a.is_ext or b.is_ext:
        raise ValueError("add/sub expect non-extended ciphertexts")
    if int(a.state.scale_degree) != int(b.state.scale_degree):
        raise ValueError("scale degrees differ")
    fa, fb = float(a.state.scaling_factor), float(b.state.scaling_factor)
    if not _same_scale(fa, fb):
        raise ValueError(f"scaling factors differ ({fa} vs {fb})")
    if a.batch_size != b.batch_size:
        raise ValueError("batch sizes differ")
    limbs = min(_limbs(a), _limbs(b))
    idx = ctx.q_prime_idx(limbs)
    comps = max(len(a.cv), len(b.cv))
    bufs = _alloc(ctx, comps, a.batch_size, limbs)
    if len(a.cv) == len(b.cv) == comps > 1:
        # components back to back in both operands: one launch over comps * batch rows
        ja, jb = _joined(a.cv, limbs, ctx.N), _joined(b.cv, limbs, ctx.N)
        if ja is not None and jb is not None:
            ctx.poly_op(op, _joined(bufs, limbs, ctx.N), ja, jb, prime_idx=idx)
            return a.cipher_like(bufs, state=a.state.replace(cur_limbs=limbs))
    out = []
    for c in range(comps):
        o = bufs[c]
        if c < len(a.cv) and c < len(b.cv):
            ctx.poly_op(op, o, _view(a.cv[c], limbs), _view(b.cv[c], limbs), prime_idx=idx)
        elif c < len(a.cv):
            u64_copy(o, _view(a.cv[c], limbs))
        elif op == nat.HCK_OP_SUB:
            ctx.poly_op(nat.HCK_OP_NEG, o, _view(b.cv[c], limbs), prime_idx=idx)
        else:
            u64_copy(o, _view(b.cv[c], limbs))
        out.append(o)
    return a.cipher_like(out, state=a.state.replace(cur_limbs=limbs))


def homo_add(a: Cipher, b: Cipher, ctx: CKKSContext) -> Cipher:
    return _binary(a, b, ctx, nat.HCK_OP_ADD)


def homo_sub(a: Cipher, b: Cipher, ctx: CKKSContext) -> Cipher:
    return _binary(a, b, ctx, nat.HCK_OP_SUB)


def homo_neg(a: Cipher, ctx: CKKSContext) -> Cipher:
    limbs = _limbs(a)
    idx = ctx.q_prime_idx(limbs)
    out = _alloc(ctx, len(a.cv), int(a.cv[0].shape[0]), limbs)
    for o, x in zip(out, a.cv):
        ctx.poly_op(nat.HCK_OP_NEG, o, _view(x, limbs), prime_idx=idx)
    return a.cipher_like(out)


def homo_mul_i(ct: Cipher, ctx: CKKSContext, negative: bool = False) -> Cipher:
    """Multiply the slots by i (or -i): the monomial X^(N/2), exact, no depth."""

    limbs = _limbs(ct)
    idx = ctx.q_prime_idx(limbs)
    out = _alloc(ctx, len(ct.cv), int(ct.cv[0].shape[0]), limbs)
    for o, x in zip(out, ct.cv):
        ctx.poly_op(nat.HCK_OP_MUL_XHALF, o, _view(x, limbs), prime_idx=idx)
        if negative:
            ctx.poly_op(nat.HCK_OP_NEG, o, o, prime_idx=idx)
    return ct.cipher_like(out)


def encode_plaintext(values, state: CipherState, slots: int, ctx: CKKSContext, is_ext: bool = False) -> Plaintext:
    """Encode real/complex ``values`` at ``state`` (limbs, scale) into the NTT domain on the GPU
    (special IFFT, rounding and per-limb reduction, forward NTT); ``is_ext`` adds the special
    primes (a plaintext for extended-basis products)."""

    re, im = ctx.slot_rows(values, slots)
    limbs = int(state.cur_limbs)
    idx = ctx.ext_prime_idx(limbs) if is_ext else ctx.q_prime_idx(limbs)
    poly = ctx.encode(re, float(state.scaling_factor), len(idx), values_im=im, prime_idx=idx)
    return Plaintext(poly, state, slots=slots, is_ext=is_ext)


def homo_mul_pt(ct: Cipher, pt: Plaintext, ctx: CKKSContext) -> Cipher:
    """Slotwise ciphertext x plaintext product (scale degrees and factors multiply)."""

    limbs = min(_limbs(ct), int(pt.state.cur_limbs))
    idx = ctx.q_prime_idx(limbs)
    p = _view(pt.cv[0], limbs)
    if p.shape[0] not in (1, ct.batch_size):
        raise ValueError("plaintext batch must be 1 or the ciphertext batch")
    if p.shape[0] == 1 and ct.batch_size > 1:
        p = p.expand(ct.batch_size, -1, -1)  # batch stride 0: one plaintext for every item
    out = _alloc(ctx, len(ct.cv), int(ct.cv[0].shape[0]), limbs)
    jx = _joined(ct.cv, limbs, ctx.N) if len(ct.cv) > 1 and pt.cv[0].shape[0] == 1 else None
    if jx is not None:
        # one plaintext for every row of the joined components (batch stride 0)
        pj = _view(pt.cv[0], limbs).expand(jx.shape[0], -1, -1)
        ctx.poly_op(nat.HCK_OP_MUL, _joined(out, limbs, ctx.N), jx, pj, prime_idx=idx)
    else:
        for o, x in zip(out, ct.cv):
            ctx.poly_op(nat.HCK_OP_MUL, o, _view(x, limbs), p, prime_idx=idx)
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


class UnpackedRaw:
    """A constant whose slot values a packer builds on first use: ``packer(source, slots,
    context)`` (llama3fhe/operators/linear/weight.py:458-465), so a bundle that is never encoded
    never packs."""

    def __init__(self, source, packer):
        self.source, self.packer = source, packer
        self._packed: dict = {}

    def values(self, slots: int, context: CKKSContext):
        key = int(slots)
        if key not in self._packed:
            self._packed[key] = self.packer(self.source, int(slots), context)
        return self._packed[key]


class ConstantBundle:
    """Named constants encoded on demand (``bundle.plaintext(name, state, slots, context, ...)``,
    llama3fhe/backend.py:346-356, operators/linear/weight.py:458-469), and named scalars encoded
    as one residue table (``encoded_scalars``, llama3fhe/operators/nonlinear/polynomial.py:
    274-291).  ``cache_mode="plain"`` keeps each encoded plaintext for reuse; ``"none"`` encodes
    every call.  ``keep`` (optional) is asked with an encoding's byte size before it is kept: a
    session byte budget answers False once it is spent, and the encoding is then only returned."""

    def __init__(self, vectors: dict | None = None, cache_mode: str = "none", scalars: dict | None = None,
                 keep=None):
        self.vectors = dict(vectors or {})
        self.scalars = dict(scalars or {})
        self.cache_mode = str(cache_mode)
        self._keep = keep
        self._cache: dict = {}

    @staticmethod
    def _nbytes(entry) -> int:
        tensors = getattr(entry, "cv", None) or [getattr(entry, "residues", None)]
        return sum(int(t.numel()) * int(t.element_size()) for t in tensors if hasattr(t, "numel"))

    def _store(self, key, entry) -> None:
        if self._keep is None or self._keep(self._nbytes(entry)):
            self._cache[key] = entry

    def encoded_scalars(self, names, cur_limbs: int, scale_degree: int = 1, context: CKKSContext | None = None,
                        scaling_factor: float | None = None, cache: bool | None = None,
                        mode: str = "double") -> EncodedScalar:
        """The named scalars as one EncodedScalar whose residues are [len(names)][cur_limbs]."""

        names = tuple(str(n) for n in names)
        key = ("scalars", names, int(cur_limbs), int(scale_degree), scaling_factor, str(mode))
        hit = self._cache.get(key)
        if hit is not None:
            return hit
        enc = encode_scalar(np.array([float(self.scalars[n]) for n in names]), int(cur_limbs), int(scale_degree),
                            scaling_factor, context=context, mode=mode)
        if (self.cache_mode in ("plain", "both")) if cache is None else bool(cache):
            self._store(key, enc)
        return enc

    def plaintext(self, name: str, state: CipherState, slots: int, context: CKKSContext,
                  is_ext: bool = False, cache: bool | None = None) -> Plaintext:
        key = (str(name), int(state.cur_limbs), float(state.scaling_factor), int(slots), bool(is_ext))
        keep = self.cache_mode in ("plain", "both") if cache is None else bool(cache)
        hit = self._cache.get(key)
        if hit is not None:
            return hit
        v = self.vectors[str(name)]
        if isinstance(v, UnpackedRaw):
            v = v.values(int(slots), context)
        v = v.values if isinstance(v, PackedRaw) else v
        pt = encode_plaintext(v, state, int(slots), context, is_ext=bool(is_ext))
        if keep:
            self._store(key, pt)
        return pt

    def cache_info(self) -> dict:
        return {"entries": len(self._cache), "total_bytes": sum(map(self._nbytes, self._cache.values()))}

    def clear_cache(self) -> None:
        self._cache.clear()


# ---------------------------------------------------------------------- hoisted / batched surface
def pack_cipher_batch(ciphers) -> Cipher:
    """Stack ciphertexts (same level, scale and basis) into one batch cipher, rows in order."""

    ciphers = tuple(ciphers)
    if not ciphers:
        raise ValueError("pack_cipher_batch needs at least one ciphertext")
    first = ciphers[0]
    for c in ciphers[1:]:
        if (c.is_ext != first.is_ext or int(c.state.cur_limbs) != int(first.state.cur_limbs)
                or int(c.state.scale_degree) != int(first.state.scale_degree)):
            raise ValueError("pack_cipher_batch: ciphertexts differ in level, scale degree or basis")
    rows = int(first.cv[0].shape[1]) if first.is_ext else _limbs(first)
    total = sum(int(c.cv[0].shape[0]) for c in ciphers)
    buf = first.cv[0].new_empty((2, total, rows, first.cv[0].shape[2]))
    for i in range(2):
        u64_cat([c.cv[i][:, :rows] for c in ciphers], 0, out=buf[i])
    return first.cipher_like([buf[0], buf[1]], batch_size=total)


def unpack_cipher_batch(batch: Cipher) -> tuple:
    """One cipher per batch row (views of the batch tensors: no copy)."""

    return tuple(batch.cipher_like([c[i:i + 1] for c in batch.cv], batch_size=1) for i in range(batch.batch_size))


def _lift_ext(x: torch.Tensor, limbs: int, ctx: CKKSContext) -> torch.Tensor:
    """[B][limbs][N] -> its extended-basis form P * x: [B][limbs + K][N], zero on the special
    primes (ModDown returns x exactly)."""

    P = 1
    for p in ctx.primes[ctx.L:ctx.L + ctx.K]:
        P *= int(p)
    out = ctx.zeros(x.shape[0], limbs + ctx.K, ctx.N)
    ctx.poly_op(nat.HCK_OP_MUL_SCALAR, out[:, :limbs], _view(x, limbs), prime_idx=ctx.q_prime_idx(limbs),
                scalar=[P % int(q) for q in ctx.primes[:limbs]])
    return out


def fast_rotate(ct: Cipher, offsets, ctx: CKKSContext, output_ext: bool = False) -> Cipher:
    """Rotations of ``ct`` by each offset as one batch cipher (row o * B + b = item b rotated by
    offsets[o]).  ``output_ext`` stops every rotation in the extended basis (no ModDown): the
    rows are then summed or multiplied there and closed by one ``moddown_from_ext``
    (llama3fhe/operators/attention/prefill/input.py:1669-1687, shifted_lane.py:76)."""

    if ct.is_ext:
        raise ValueError("fast_rotate expects a non-extended ciphertext")
    offsets = [int(o) for o in offsets]
    if not offsets:
        raise ValueError("fast_rotate needs at least one offset")
    limbs = _limbs(ct)
    c0, c1 = _view(ct.cv[0], limbs), _view(ct.cv[1], limbs)
    B = ct.batch_size
    rows = limbs + (ctx.K if output_ext else 0)
    out0 = ctx.empty(len(offsets) * B, rows, ctx.N)
    out1 = ctx.empty(len(offsets) * B, rows, ctx.N)
    for i, off in enumerate(offsets):
        o0, o1 = out0[i * B:(i + 1) * B], out1[i * B:(i + 1) * B]
        if off % ctx.max_slots == 0 and off != ctx.M - 1:
            if output_ext:
                u64_copy(o0, _lift_ext(c0, limbs, ctx))
                u64_copy(o1, _lift_ext(c1, limbs, ctx))
            else:
                u64_copy(o0, c0)
                u64_copy(o1, c1)
            continue
        g = _galois(off, ctx)
        key = ctx.key_for_galois(g)
        if output_ext:
            ctx.rotate_ext(c0, c1, limbs, g, key, out0=o0, out1=o1)
        else:
            ctx.rotate_raw(c0, c1, limbs, g, key, out0=o0, out1=o1)
    return ct.cipher_like([out0, out1], is_ext=bool(output_ext), batch_size=len(offsets) * B)


def moddown_from_ext(ct: Cipher, ctx: CKKSContext) -> Cipher:
    """Close an extended-basis cipher: divide by P (rounded) back to its Q limbs."""

    if not ct.is_ext:
        raise ValueError("moddown_from_ext expects an extended-basis ciphertext")
    limbs = _limbs(ct)
    out = [ctx.moddown(c, limbs) for c in ct.cv]
    return ct.cipher_like(out, is_ext=False)


def grouped_pairwise_mac(batch: Cipher, pts: Plaintext, groups: int, ctx: CKKSContext) -> Cipher:
    """Row-wise products summed within ``groups`` equal consecutive groups of rows:
    out[g] = sum_{r in group g} pts[r] * batch[r] (exact residues; extended-basis rows need an
    extended-basis plaintext).  Scale degrees and factors multiply."""

    groups = int(groups)
    R = batch.batch_size
    if groups < 1 or R % groups:
        raise ValueError(f"{R} rows do not split into {groups} groups")
    if bool(pts.is_ext) != bool(batch.is_ext):
        raise ValueError("plaintext and ciphertext bases differ (extended vs not)")
    if pts.batch_size != R:
        raise ValueError(f"expected {R} plaintext rows, got {pts.batch_size}")
    limbs = _limbs(batch)
    idx = ctx.ext_prime_idx(limbs) if batch.is_ext else ctx.q_prime_idx(limbs)
    n = len(idx)
    m = R // groups
    if pts.state.cur_limbs < limbs:
        raise ValueError("plaintext has fewer limbs than the ciphertext")
    p = pts.cv[0]
    if batch.is_ext and pts.state.cur_limbs != limbs:
        raise ValueError("an extended-basis plaintext must match the ciphertext level exactly")
    out0 = ctx.empty(groups, n, ctx.N)
    out1 = ctx.empty(groups, n, ctx.N)
    for g in range(groups):
        b0 = [batch.cv[0][g * m + b:g * m + b + 1] for b in range(m)]
        b1 = [batch.cv[1][g * m + b:g * m + b + 1] for b in range(m)]
        res = ctx.bsgs_mac(b0, b1, p[g * m:(g + 1) * m], n, 1, prime_idx=idx)
        u64_copy(out0[g], res[0, 0, 0])
        u64_copy(out1[g], res[1, 0, 0])
    st = batch.state
    state = st.replace(scale_degree=int(st.scale_degree) + int(pts.state.scale_degree),
                       scaling_factor=float(st.scaling_factor) * float(pts.state.scaling_factor))
    return batch.cipher_like([out0, out1], state=state, batch_size=groups)


def _has_key(ctx: CKKSContext, offset: int) -> bool:
    return _galois(offset, ctx) in ctx.rotation_keys


def prepare_hoisted_baby_rotations(ct: Cipher, offsets, ctx: CKKSContext, strategy: str = "normal",
                                   baby_anchor_step: int = -1) -> tuple:
    """The baby basis of a BSGS product: one cipher per offset (the input batch rotated by it),
    offset 0 sharing the input's tensors.  The offsets with their own keys come from one hoisted
    ModUp per input (``CKKSContext.rotate_hoisted``); an offset without its own key is reached from
    the largest smaller offset already built whose difference has a key (the anchor blocks of
    llama3fhe/operators/linear/config.py:235-268)."""

    if ct.is_ext:
        raise ValueError("baby rotations start from a non-extended ciphertext")
    limbs = _limbs(ct)
    c0, c1 = _view(ct.cv[0], limbs), _view(ct.cv[1], limbs)
    if c0.shape[0] > 1 and (c0.stride(0) != limbs * ctx.N or c1.stride(0) != limbs * ctx.N):
        # the MAC needs one batch stride across the basis: drop the stored limbs above the level
        c0, c1 = c0.contiguous(), c1.contiguous()
    built: dict[int, tuple] = {}
    offsets = [int(o) for o in offsets]
    direct = [o for o in dict.fromkeys(offsets) if o % ctx.max_slots and _has_key(ctx, o)]
    if ctx.supports_hoisting and len(direct) > 1:
        # one ModUp per input; every offset with its own key read from the hoisted digits
        B = int(c0.shape[0])
        gals = [_galois(o, ctx) for o in direct for _ in range(B)]
        digits = ctx.hoist_digits(c1, limbs)
        h0, h1 = ctx.rotate_hoisted(c0, c1, limbs, digits, gals, [ctx.key_for_galois(g) for g in gals])
        del digits
        for i, o in enumerate(direct):
            built[o] = (h0[i * B:(i + 1) * B], h1[i * B:(i + 1) * B])
    out = []
    for off in offsets:
        if off in built:
            pair = built[off]
        elif off % ctx.max_slots == 0:
            pair = (c0, c1)
        elif _has_key(ctx, off):
            g = _galois(off, ctx)
            pair = ctx.rotate_raw(c0, c1, limbs, g, ctx.key_for_galois(g))
        else:
            base = max((b for b in built if b < off and _has_key(ctx, off - b)), default=None)
            if base is None:
                raise KeyError(f"no rotation key reaches baby offset {off}")
            g = _galois(off - base, ctx)
            pair = ctx.rotate_raw(built[base][0], built[base][1], limbs, g, ctx.key_for_galois(g))
        built[off] = pair
        out.append(ct.cipher_like(list(pair)))
    return tuple(out)


GIANT_GROUP = 4  # giant steps per grouped extended-basis launch (hck_rotate_ext_sum); 1: one per launch


def hoisted_mac_sum(ct: Cipher, baby_offsets, plaintexts: Plaintext, giant_offset: int, giant_count: int,
                    ctx: CKKSContext, strategy: str = "normal", baby_anchor_step: int = -1,
                    baby_rotations=None) -> Cipher:
    """One BSGS chunk: sum_g rot(sum_b pt[g B + b] * baby_b, g * giant_offset) for every batch row
    of ``ct`` (llama3fhe/operators/linear/operator.py:434-444).  The baby MAC runs over all rows
    and giants at once (hck_bsgs_mac).  ``strategy="normal"`` closes the giants by Horner steps
    acc <- rot(acc, giant_offset) + partial_g, each one fused rotate-and-add; with
    ``"ext_double_hoist"`` every partial is rotated by its own multiple of giant_offset in the
    extended basis and the sum is closed by one ModDown.  The result keeps the input level with
    the plaintext's scale multiplied in (not rescaled)."""

    strategy = str(strategy).lower()
    if strategy not in ("normal", "ext_normal", "ext_double_hoist"):
        raise ValueError("strategy must be 'normal', 'ext_normal' or 'ext_double_hoist'")
    limbs = _limbs(ct)
    offsets = [int(o) for o in baby_offsets]
    nb, G = len(offsets), int(giant_count)
    if baby_rotations is None:
        baby_rotations = prepare_hoisted_baby_rotations(ct, offsets, ctx, strategy=strategy,
                                                        baby_anchor_step=baby_anchor_step)
    babies = tuple(baby_rotations)
    if len(babies) != nb:
        raise ValueError(f"expected {nb} baby rotations, got {len(babies)}")
    pts = plaintexts.cv[0] if isinstance(plaintexts, Plaintext) else plaintexts
    pt_state = plaintexts.state if isinstance(plaintexts, Plaintext) else None
    if pts.shape[0] != nb * G:
        raise ValueError(f"expected {nb * G} plaintext rows, got {pts.shape[0]}")
    part = ctx.bsgs_mac([_view(b.cv[0], limbs) for b in babies], [_view(b.cv[1], limbs) for b in babies],
                        pts, limbs, G)  # [2][G][B][limbs][N]
    idx = ctx.q_prime_idx(limbs)
    if strategy == "ext_double_hoist" and G > 1:
        ext0 = _lift_ext(part[0, 0], limbs, ctx)
        ext1 = _lift_ext(part[1, 0], limbs, ctx)
        B = int(part.shape[2])
        step = max(1, min(GIANT_GROUP, 64 // B))  # giants per grouped launch (<= 64 items)
        for g0 in range(1, G, step):
            # each partial rotated by its own giant multiple, summed in the extended basis; a group of
            # giants keeps its running sum on chip and touches the accumulator once
            gs = list(range(g0, min(G, g0 + step)))
            gals = [_galois(g * int(giant_offset), ctx) for g in gs]
            keys = [ctx.key_for_galois(gg) for gg in gals]
            if len(gs) == 1:
                ctx.rotate_ext(part[0, gs[0]], part[1, gs[0]], limbs, gals[0], keys[0], out0=ext0, out1=ext1,
                               acc=(ext0, ext1))
            else:
                ctx.rotate_ext_sum(part[0, gs[0]:gs[-1] + 1], part[1, gs[0]:gs[-1] + 1], limbs, gals, keys,
                                   ext0, ext1, acc=(ext0, ext1))
        acc0, acc1 = ctx.moddown(ext0, limbs), ctx.moddown(ext1, limbs)
    else:
        acc0, acc1 = part[0, G - 1], part[1, G - 1]
        gk = _galois(int(giant_offset), ctx) if G > 1 else None
        for g in range(G - 2, -1, -1):
            acc0, acc1 = ctx.rotate_raw(acc0, acc1, limbs, gk, ctx.key_for_galois(gk), out0=part[0, g],
                                        out1=part[1, g], acc=(part[0, g], part[1, g]))
        acc0, acc1 = u64_clone(acc0), u64_clone(acc1)
    del part
    st = ct.state
    deg = int(pt_state.scale_degree) if pt_state is not None else 1
    fac = float(pt_state.scaling_factor) if pt_state is not None else 1.0
    state = st.replace(scale_degree=int(st.scale_degree) + deg, scaling_factor=float(st.scaling_factor) * fac)
    return ct.cipher_like([acc0, acc1], state=state)


# ---------------------------------------------------------------------------- scalars
MAX_ENCODED_BITS = 61  # |value * scale| must stay below 2^61 (llama3fhe/operators/attention/prefill/softmax.py:559)


class EncodedScalar:
    """A constant encoded for one level: ``residues`` holds round(value * scaling_factor) (or the
    integer itself) modulo each of the ``cur_limbs`` Q primes, last axis = limb; the leading axes
    index groups / entries of a table (fhe.EncodedScalar, llama3fhe/operators/nonlinear/
    polynomial.py:286-291).  A constant polynomial takes the same value at every NTT evaluation
    point, so these residues act on every coefficient of an NTT-domain limb."""

    __slots__ = ("residues", "cur_limbs", "scale_degree", "scaling_factor")

    def __init__(self, residues, cur_limbs: int, scale_degree: int, scaling_factor: float):
        self.residues = residues
        self.cur_limbs = int(cur_limbs)
        self.scale_degree = int(scale_degree)
        self.scaling_factor = float(scaling_factor)


def _scaled_int(value, scaling_factor: float, integer: bool, limit: int = 1 << MAX_ENCODED_BITS) -> int:
    if integer:
        if float(value) != int(value):
            raise ValueError(f"integer mode needs an integral value, got {value!r}")
        m = int(value)
    else:
        x = float(value) * float(scaling_factor)
        if not np.isfinite(x):
            raise ValueError("scalar * scale is not finite")
        m = int(np.sign(x) * np.floor(abs(x) + 0.5))  # round half away from zero, as the encoder
    if abs(m) >= limit:
        raise ValueError(f"encoded scalar {value!r} x {scaling_factor} exceeds the limit 2^{limit.bit_length() - 1}")
    return m


def _scalar_limit(primes) -> int:
    """A scalar is one integer reduced exactly modulo each prime, so it is not bound by the
    polynomial encoder's 2^61: it may reach a quarter of the level's modulus (its residues then
    name it with a factor-2 margin), and 2^61 at any level.  The reference chain's 59-bit scales
    need this for the Chebyshev evaluator's coefficients (|c| * 2^59 above 2^61)."""

    Q = 1
    for q in primes:
        Q *= int(q)
    return max(1 << MAX_ENCODED_BITS, Q >> 2)


def _scalar_residues(values, cur_limbs: int, scaling_factor: float, integer: bool, ctx: CKKSContext) -> np.ndarray:
    vals = np.atleast_1d(np.asarray(values, dtype=np.float64 if not integer else object))
    primes = ctx.q_primes[: int(cur_limbs)]
    limit = _scalar_limit(primes)
    out = np.empty(vals.shape + (len(primes),), dtype=np.uint64)
    for pos in np.ndindex(vals.shape):
        m = _scaled_int(vals[pos], scaling_factor, integer, limit)
        out[pos] = [m % q for q in primes]
    return out


def encode_scalar(value, cur_limbs: int, scale_degree: int = 1, scaling_factor: float | None = None,
                  context: CKKSContext | None = None, mode: str = "double") -> EncodedScalar:
    """Encode a constant for a ciphertext at ``cur_limbs`` limbs.  ``mode="double"`` (scale_degree
    >= 1): round(value * scaling_factor), the scaling factor defaulting to the level's scale;
    ``mode="integer"`` or scale_degree 0: the integer itself (scale 1).  Keywords as
    llama3fhe/operators/nonlinear/polynomial.py:72-97, bootstrap.py:604-623."""

    ctx = context
    if ctx is None:
        raise ValueError("encode_scalar needs the context")
    integer = str(mode) == "integer" or int(scale_degree) == 0
    sf = 1.0 if integer else (ctx.scale_at(int(cur_limbs)) if scaling_factor is None else float(scaling_factor))
    res = _scalar_residues(value, int(cur_limbs), sf, integer, ctx)
    if np.ndim(value) == 0:
        res = res[0]
    return EncodedScalar(torch.from_numpy(res), int(cur_limbs), 0 if integer else int(scale_degree), sf)


def _scalar_list(enc: EncodedScalar, limbs: int):
    r = enc.residues.cpu().numpy() if hasattr(enc.residues, "cpu") else np.asarray(enc.residues)
    r = np.asarray(r, dtype=np.uint64).reshape(-1)
    if r.size < limbs:
        raise ValueError(f"encoded scalar has {r.size} limbs, need {limbs}")
    return [int(v) for v in r[:limbs]]


def homo_mul_scalar(ct: Cipher, enc: EncodedScalar, ctx: CKKSContext) -> Cipher:
    """Multiply every slot by the encoded constant (exact residue products); scale degrees add and
    scaling factors multiply."""

    limbs = min(_limbs(ct), enc.cur_limbs)
    idx = ctx.q_prime_idx(limbs)
    sc = _scalar_list(enc, limbs)
    out = _alloc(ctx, len(ct.cv), int(ct.cv[0].shape[0]), limbs)
    jx = _joined(ct.cv, limbs, ctx.N) if len(ct.cv) > 1 else None
    if jx is not None:
        ctx.poly_op(nat.HCK_OP_MUL_SCALAR, _joined(out, limbs, ctx.N), jx, prime_idx=idx, scalar=sc)
    else:
        for o, x in zip(out, ct.cv):
            ctx.poly_op(nat.HCK_OP_MUL_SCALAR, o, _view(x, limbs), prime_idx=idx, scalar=sc)
    st = ct.state
    state = st.replace(cur_limbs=limbs, scale_degree=int(st.scale_degree) + enc.scale_degree,
                       scaling_factor=float(st.scaling_factor) * enc.scaling_factor)
    return ct.cipher_like(out, state=state)


def homo_mul_scalar_rescale(ct: Cipher, enc: EncodedScalar, ctx: CKKSContext) -> Cipher:
    """homo_mul_scalar followed by rescale (softmax.py:720-729, norm/refresh.py:21-31), as one
    hck_lincomb_rescale of a single term: the product is never stored; the same residues."""

    limbs = min(_limbs(ct), enc.cur_limbs)
    if ct.is_ext or limbs < 2:
        raise ValueError("rescale needs a non-extended ciphertext with at least two limbs")
    B = int(ct.cv[0].shape[0])
    w = ctx.resident(np.asarray(_scalar_list(enc, limbs), dtype=np.uint64).reshape(1, limbs))
    out = _alloc(ctx, len(ct.cv), B, limbs - 1)
    ctx.lincomb_rescale([[x[b]] for x in ct.cv for b in range(B)], limbs, [o[b] for o in out for b in range(B)], w)
    st = ct.state
    sd = int(st.scale_degree) + enc.scale_degree
    state = st.replace(cur_limbs=limbs - 1, scale_degree=max(1, sd - 1),
                       scaling_factor=float(st.scaling_factor) * enc.scaling_factor
                       / float(ctx.rescale_divisor_at(limbs)))
    return ct.cipher_like(out, state=state)


def homo_add_scalar(ct: Cipher, enc: EncodedScalar, ctx: CKKSContext) -> Cipher:
    """Add the encoded constant to every slot (to c0 only); the constant must carry the
    ciphertext's scale (softmax.py:1053-1064)."""

    if not _same_scale(float(ct.state.scaling_factor), enc.scaling_factor):
        raise ValueError(f"scalar scale {enc.scaling_factor} != ciphertext scale {ct.state.scaling_factor}")
    limbs = min(_limbs(ct), enc.cur_limbs)
    idx = ctx.q_prime_idx(limbs)
    out = _alloc(ctx, len(ct.cv), ct.batch_size, limbs)
    ctx.poly_op(nat.HCK_OP_ADD_SCALAR, out[0], _view(ct.cv[0], limbs), prime_idx=idx,
                scalar=_scalar_list(enc, limbs))
    for o, x in zip(out[1:], ct.cv[1:]):
        u64_copy(o, _view(x, limbs))
    return ct.cipher_like(out, state=ct.state.replace(cur_limbs=limbs))


def homo_add_pt(ct: Cipher, pt: Plaintext, ctx: CKKSContext) -> Cipher:
    """Add a plaintext (same scale) to every slot: c0 + pt (softmax.py:290-298, rmsnorm.py:793)."""

    if not _same_scale(float(ct.state.scaling_factor), float(pt.state.scaling_factor)):
        raise ValueError(f"plaintext scale {pt.state.scaling_factor} != ciphertext scale {ct.state.scaling_factor}")
    limbs = min(_limbs(ct), int(pt.state.cur_limbs))
    idx = ctx.q_prime_idx(limbs)
    p = _view(pt.cv[0], limbs)
    if p.shape[0] not in (1, ct.batch_size):
        raise ValueError("plaintext batch must be 1 or the ciphertext batch")
    if p.shape[0] == 1 and ct.batch_size > 1:
        p = p.expand(ct.batch_size, -1, -1)
    c0 = ctx.empty(ct.batch_size, limbs, ctx.N)
    ctx.poly_op(nat.HCK_OP_ADD, c0, _view(ct.cv[0], limbs), p.contiguous(), prime_idx=idx)
    rest = [u64_clone(_view(x, limbs)) for x in ct.cv[1:]]
    return ct.cipher_like([c0] + rest, state=ct.state.replace(cur_limbs=limbs))


# ---------------------------------------------------------------------------- ciphertext products
def _product_state(a: Cipher, b: Cipher, limbs: int) -> CipherState:
    return a.state.replace(cur_limbs=limbs,
                           scale_degree=int(a.state.scale_degree) + int(b.state.scale_degree),
                           scaling_factor=float(a.state.scaling_factor) * float(b.state.scaling_factor))


def _mul_operands(a: Cipher, b: Cipher):
    if a.is_ext or b.is_ext or len(a.cv) != 2 or len(b.cv) != 2:
        raise ValueError("products take two-component, non-extended ciphertexts")
    if a.batch_size != b.batch_size:
        raise ValueError("batch sizes differ")
    limbs = min(_limbs(a), _limbs(b))
    return limbs, [_view(x, limbs) for x in a.cv], [_view(x, limbs) for x in b.cv]


def homo_mul_no_relin(a: Cipher, b: Cipher, ctx: CKKSContext) -> Cipher:
    """Tensor product: the three-component ciphertext (a0 b0, a0 b1 + a1 b0, a1 b1) decrypting
    under (1, s, s^2) (qk.py:460-464, pv.py:544-548)."""

    limbs, (a0, a1), (b0, b1) = _mul_operands(a, b)
    d0, d1, d2 = ctx.tensor(a0, a1, b0, b1, limbs)
    return a.cipher_like([d0, d1, d2], state=_product_state(a, b, limbs))


def _relin_key(ctx: CKKSContext) -> torch.Tensor:
    if ctx.relin_key is None:
        raise RuntimeError("the context holds no relinearisation key (generate_client_context makes one)")
    return ctx.relin_key


def homo_relinearize(ct: Cipher, ctx: CKKSContext) -> Cipher:
    """Three components back to two: (d0, d1) + KeySwitch_{s^2 -> s}(d2) (kernel_helpers.py:146-152)."""

    if len(ct.cv) == 2:
        return ct.cipher_like([u64_clone(x) for x in ct.cv])
    if len(ct.cv) != 3 or ct.is_ext:
        raise ValueError("relinearize takes a three-component, non-extended ciphertext")
    limbs = _limbs(ct)
    d0, d1, d2 = (_view(x, limbs) for x in ct.cv)
    o0, o1 = ctx.relinearize_raw(d0, d1, d2, limbs, _relin_key(ctx))
    return ct.cipher_like([o0, o1])


def homo_mul_relin(a: Cipher, b: Cipher, ctx: CKKSContext) -> Cipher:
    """Product with relinearisation (tensor product and key switch, the tensor components kept in
    the workspace)."""

    limbs, (a0, a1), (b0, b1) = _mul_operands(a, b)
    both = ctx.mul_relin_raw(a0, a1, b0, b1, limbs, _relin_key(ctx), stacked=True)
    return a.cipher_like([both[0], both[1]], state=_product_state(a, b, limbs))


def homo_mul_relin_rescale(a: Cipher, b: Cipher, ctx: CKKSContext) -> Cipher:
    """rescale(homo_mul_relin(a, b)) in one native call (hck_mul_relin_rescale: the relinearisation's
    ModDown and the rescale share one conversion pass), the same residues and state."""

    limbs, (a0, a1), (b0, b1) = _mul_operands(a, b)
    if limbs < 2:
        raise ValueError("rescale needs a non-extended ciphertext with at least two limbs")
    both = ctx.mul_relin_rescale_raw(a0, a1, b0, b1, limbs, _relin_key(ctx), stacked=True)
    st = _product_state(a, b, limbs)
    state = st.replace(cur_limbs=limbs - 1, scale_degree=max(1, int(st.scale_degree) - 1),
                       scaling_factor=float(st.scaling_factor) / float(ctx.rescale_divisor_at(limbs)))
    return a.cipher_like([both[0], both[1]], state=state)


def homo_mul_relin_rescale_postop(lhs: Cipher, rhs: Cipher, ctx: CKKSContext, apply_double: bool = False,
                                  sub: Cipher | None = None, scalar: EncodedScalar | None = None) -> Cipher:
    """rescale(lhs * rhs) (relinearised), then x 2 when ``apply_double``, minus ``sub`` (dropped to
    the result's level), plus the encoded ``scalar``: the Chebyshev step T_{a+b} = 2 T_a T_b -
    T_{|a-b|} (llama3fhe/operators/nonlinear/polynomial.py:140-190).  One native call
    (hck_mul_relin_rescale_postop): the post-ops ride on the product's last kernel."""

    limbs, (a0, a1), (b0, b1) = _mul_operands(lhs, rhs)
    if limbs < 2:
        raise ValueError("rescale needs a non-extended ciphertext with at least two limbs")
    st = _product_state(lhs, rhs, limbs)
    state = st.replace(cur_limbs=limbs - 1, scale_degree=max(1, int(st.scale_degree) - 1),
                       scaling_factor=float(st.scaling_factor) / float(ctx.rescale_divisor_at(limbs)))
    pair = None
    if sub is not None:
        if sub.is_ext or len(sub.cv) != 2 or sub.batch_size != lhs.batch_size or _limbs(sub) < limbs - 1:
            raise ValueError("postop sub must be a two-component ciphertext of the batch with the result's limbs")
        pair = tuple(_view(x, limbs - 1) for x in sub.cv)
    sc = None
    if scalar is not None:
        if not _same_scale(float(state.scaling_factor), scalar.scaling_factor):
            raise ValueError(f"scalar scale {scalar.scaling_factor} != product scale {state.scaling_factor}")
        sc = _scalar_list(scalar, limbs - 1)
    both = ctx.mul_relin_rescale_postop_raw(a0, a1, b0, b1, limbs, _relin_key(ctx), apply_double=bool(apply_double),
                                            sub=pair, scalar=sc)
    return lhs.cipher_like([both[0], both[1]], state=state)


def grouped_scalar_weighted_acc(batch: Cipher, table: EncodedScalar, ctx: CKKSContext) -> Cipher:
    """out[g] = sum_j table[g][j] * batch[j] over the items of a cipher batch (one kernel per
    component); ``table.residues`` is [groups][items][limbs] (or [items][limbs] for one group).
    Scale degrees add and scaling factors multiply, as for homo_mul_scalar; the caller rescales
    (polynomial.py:256-300)."""

    if batch.is_ext:
        raise ValueError("weighted sums take non-extended ciphertexts")
    limbs = min(_limbs(batch), table.cur_limbs)
    r = table.residues if isinstance(table.residues, torch.Tensor) else torch.from_numpy(np.asarray(table.residues))
    r = r.to(torch.uint64)
    if r.dim() == 2:
        r = r.unsqueeze(0)
    n = batch.batch_size
    if r.dim() != 3 or int(r.shape[1]) != n:
        raise ValueError(f"weight table must be [groups][{n}][limbs]")
    w = r[:, :, :limbs].contiguous()
    out = [ctx.weighted_sum(_view(x, limbs), w, limbs) for x in batch.cv]
    st = batch.state
    state = st.replace(cur_limbs=limbs, scale_degree=int(st.scale_degree) + table.scale_degree,
                       scaling_factor=float(st.scaling_factor) * table.scaling_factor)
    return batch.cipher_like(out, state=state, batch_size=int(w.shape[0]))


def cipher_batch_item(batch: Cipher, index: int) -> Cipher:
    """Item ``index`` of a cipher batch as a one-item cipher (views; easyfhe.fhe.ops.layout,
    polynomial.py:293-296)."""

    i = int(index)
    if not 0 <= i < batch.batch_size:
        raise IndexError(f"item {i} of a batch of {batch.batch_size}")
    return batch.cipher_like([x[i:i + 1] for x in batch.cv], batch_size=1)
