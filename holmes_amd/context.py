"""Device-resident CKKS context and ciphertext containers.

Mirrors the EasyFHE native context and cipher objects that Holmes' operators touch
(attributes L, N, M, K, alpha, max_slots, device, logN, scale_at, rescale_divisor_at, primes,
get_rotation_key_for_limbs: llama3fhe/parallel/prefill/keys.py:39-47; cipher fields cv, state,
is_ext, slots, batch_size, cipher_like, deep_copy: bench/cmp/holmes_multi_mac.py:61-89).
Every arithmetic operation runs in libholmes_ckks (HIP, gfx950); tensors are PyTorch-ROCm
buffers used only as device memory.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, replace

import numpy as np
import torch

from . import _native as nat
from .params import CKKSContextSpec

N_LOG = 16


@dataclass(frozen=True)
class CipherState:
    """Ciphertext metadata (easyfhe.fhe.CipherState: cur_limbs, scale_degree, scaling_factor)."""

    cur_limbs: int
    scale_degree: int = 1
    scaling_factor: float = float(2**40)

    def replace(self, **changes) -> "CipherState":
        return replace(self, **changes)


class Cipher:
    """A batch of CKKS ciphertexts: ``cv = [c0, c1]``, each ``[batch][limbs][N]`` uint64.

    Limb l of every polynomial is a residue modulo prime l of the Q chain (or, with
    ``is_ext``, Q limbs 0..cur_limbs-1 followed by the K special primes).
    """

    __slots__ = ("cv", "state", "slots", "is_ext", "batch_size", "_released")

    def __init__(self, cv, state: CipherState, *, slots: int, is_ext: bool = False, batch_size: int | None = None):
        self.cv = list(cv)
        self.state = state
        self.slots = int(slots)
        self.is_ext = bool(is_ext)
        self.batch_size = int(batch_size if batch_size is not None else self.cv[0].shape[0])
        self._released = False

    @property
    def device(self):
        return self.cv[0].device

    def cipher_like(self, cv, *, state=None, slots=None, is_ext=None, batch_size=None) -> "Cipher":
        return Cipher(
            cv,
            self.state if state is None else state,
            slots=self.slots if slots is None else slots,
            is_ext=self.is_ext if is_ext is None else is_ext,
            batch_size=batch_size,
        )

    def deep_copy(self) -> "Cipher":
        return self.cipher_like([u64_clone(c) for c in self.cv])

    def release(self) -> None:
        self.cv = []
        self._released = True

    def __repr__(self) -> str:
        return (f"Cipher(batch={self.batch_size}, limbs={self.state.cur_limbs}, "
                f"scale_degree={self.state.scale_degree}, ext={self.is_ext})")


def u64_copy(dst: torch.Tensor, src: torch.Tensor) -> torch.Tensor:
    """dst <- src for uint64 tensors through int64 views: torch's vectorised copy kernels (its
    uint64 copies take a slow generic path)."""

    dst.view(torch.int64).copy_(src.view(torch.int64))
    return dst


def u64_clone(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int64).clone().view(torch.uint64)


def u64_cat(parts, dim: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    if out is not None:
        torch.cat([x.view(torch.int64) for x in parts], dim, out=out.view(torch.int64))
        return out
    return torch.cat([x.view(torch.int64) for x in parts], dim).view(torch.uint64)


def _bstride(t: torch.Tensor) -> int:
    """Batch stride passed to the kernels: a single-item batch may carry any stride (a size-1
    axis from numpy has stride 0), so it is reported as the dense item size."""

    return int(t.stride(0)) if t.shape[0] > 1 else int(t[0].numel())


def _stream_ptr(device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


# EasyFHE's Encode.cu constant MAX_64BIT_VALUE: the encode sidecar stores a negative coefficient c
# as MAX + c and subtracts MAX mod p after the reduction (bench/cmp/kernels/holmes_encode.cu:15,133-159).
_MAX64 = 9223372036854775295


class ResidueTable(list):
    """A table of residues or moduli as Python ints (host arithmetic indexes and slices it like a
    list) with a device copy: ``data_ptr()`` is the address of a uint64 tensor of the same values on
    the context's device, which is how the reference's ctypes bindings pass EasyFHE's context
    tables (``ctx.primes.data_ptr()``, bench/cmp/holmes_multi_mac.py:139)."""

    def __init__(self, values, device):
        super().__init__(int(v) for v in values)
        self._device = device
        self._tensor = None

    @property
    def tensor(self) -> torch.Tensor:
        if self._tensor is None:
            self._tensor = torch.tensor(np.array(list(self), dtype=np.uint64), device=self._device)
        return self._tensor

    def data_ptr(self) -> int:
        return int(self.tensor.data_ptr())


class _PerLimbTables:
    """``table[limbs]``: a device uint64 tensor over q_0 .. q_(limbs-1) followed by the K special
    primes, built once per limb count -- the shape of EasyFHE's ``QplusP_map`` family
    (bench/cmp/holmes_fast_stage2.py:74-77)."""

    def __init__(self, ctx: "CKKSContext", value_of):
        self._ctx, self._value_of, self._cache = ctx, value_of, {}

    def __getitem__(self, limbs: int) -> torch.Tensor:
        limbs = int(limbs)
        if not 1 <= limbs <= self._ctx.L:
            raise KeyError(f"limb count {limbs} outside [1, {self._ctx.L}]")
        hit = self._cache.get(limbs)
        if hit is None:
            primes = list(self._ctx.q_primes[:limbs]) + list(self._ctx.p_primes)
            vals = np.array([self._value_of(int(p)) for p in primes], dtype=np.uint64)
            hit = self._cache[limbs] = torch.tensor(vals, device=self._ctx.device)
        return hit


def barrett_k(p: int) -> int:
    """The Barrett shift of EasyFHE's tables: floor(log2 p) + 63 (bench/cmp/kernels/holmes_mac.cu:56-58)."""

    return int(p).bit_length() - 1 + 63


def barrett_ratio(p: int) -> int:
    """floor(2^k / p) with k = barrett_k(p), below 2^64 (bench/cmp/kernels/holmes_mac.cu:56-58)."""

    return (1 << barrett_k(p)) // int(p)


class CKKSContext:
    """Prime chain + device tables (libholmes_ckks context) + evaluation keys in HBM.

    Besides the host lists the library needs, the context carries EasyFHE's native-context tables
    as device uint64 tensors, with the reference's definitions, so code that binds them by address
    runs unchanged: ``primes`` (Q then P; a ResidueTable, so ``primes.data_ptr()``), ``barret_ratio``
    and ``barret_k`` (per prime), ``PModq`` (P mod q_i), ``QplusP_map`` /
    ``QmaxdiffplusPmaxdiff_map`` / ``QbarretRatioplusPbarretRatio_map`` / ``QbarretKplusPbarretK_map``
    (per limb count) and ``power_of_roots`` / ``power_of_roots_shoup`` ([L + K][N])."""

    def __init__(self, spec: CKKSContextSpec, device: str = "cuda"):
        spec.validate()
        if not torch.cuda.is_available():
            raise RuntimeError("holmes_amd needs a ROCm GPU: no device is visible (no CPU fallback)")
        self.spec = spec
        self.device = torch.device(device if device != "cuda" else "cuda:0")
        self.logN = N_LOG
        self.N = 1 << N_LOG
        self.M = 2 * self.N
        self.max_slots = self.N // 2
        q, p = spec.prime_chain()
        self.q_primes, self.p_primes = q, p
        self.primes = ResidueTable(q + p, self.device)
        self.L = len(q)
        self.K = len(p)
        self.alpha = spec.alpha
        self.dnum = int(spec.dnum)
        self.beta_max = -(-self.L // self.alpha)
        self._scale = float(2 ** int(spec.scale_bits))
        L = nat.lib()
        h = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            nat.check(
                L.hck_context_create(ctypes.byref(h), N_LOG, self.L, self.K, self.alpha,
                                     nat.u64_array(self.primes)),
                "hck_context_create",
            )
        self._h = h
        # hoisted rotations (hck_rotate_hoisted) run on both prime widths
        self.supports_hoisting = True
        self._ws: torch.Tensor | None = None
        self.rotation_keys: dict[int, torch.Tensor] = {}
        self.relin_key: torch.Tensor | None = None

    # ------------------------------------------------------------------ EasyFHE's native tables
    @property
    def barret_ratio(self) -> torch.Tensor:
        return self._table("barret_ratio", lambda: [barrett_ratio(p) for p in self.primes])

    @property
    def barret_k(self) -> torch.Tensor:
        return self._table("barret_k", lambda: [barrett_k(p) for p in self.primes])

    @property
    def PModq(self) -> torch.Tensor:  # noqa: N802 -- EasyFHE's attribute name
        P = 1
        for p in self.p_primes:
            P *= int(p)
        return self._table("PModq", lambda: [P % int(q) for q in self.q_primes])

    @property
    def QplusP_map(self) -> _PerLimbTables:  # noqa: N802
        return self._limb_tables("QplusP_map", lambda p: p)

    @property
    def QmaxdiffplusPmaxdiff_map(self) -> _PerLimbTables:  # noqa: N802
        return self._limb_tables("QmaxdiffplusPmaxdiff_map", lambda p: _MAX64 % p)

    @property
    def QbarretRatioplusPbarretRatio_map(self) -> _PerLimbTables:  # noqa: N802
        return self._limb_tables("QbarretRatioplusPbarretRatio_map", barrett_ratio)

    @property
    def QbarretKplusPbarretK_map(self) -> _PerLimbTables:  # noqa: N802
        return self._limb_tables("QbarretKplusPbarretK_map", barrett_k)

    @property
    def power_of_roots(self) -> torch.Tensor:
        return self._root_tables()[0]

    @property
    def power_of_roots_shoup(self) -> torch.Tensor:
        return self._root_tables()[1]

    def _table(self, name: str, values) -> torch.Tensor:
        cache = self.__dict__.setdefault("_native_tables", {})
        if name not in cache:
            cache[name] = torch.tensor(np.array(values(), dtype=np.uint64), device=self.device)
        return cache[name]

    def _limb_tables(self, name: str, value_of) -> _PerLimbTables:
        cache = self.__dict__.setdefault("_native_tables", {})
        if name not in cache:
            cache[name] = _PerLimbTables(self, value_of)
        return cache[name]

    def _root_tables(self) -> tuple[torch.Tensor, torch.Tensor]:
        """psi^brv(k) and its Shoup companions floor(w 2^64 / p), [L + K][N] each (hck_context_root_tables)."""

        cache = self.__dict__.setdefault("_native_tables", {})
        if "roots" not in cache:
            roots = torch.empty(len(self.primes), self.N, dtype=torch.uint64, device=self.device)
            shoup = torch.empty_like(roots)
            with torch.cuda.device(self.device):
                nat.check(nat.lib().hck_context_root_tables(self._h, roots.data_ptr(), shoup.data_ptr()),
                          "hck_context_root_tables")
            cache["roots"] = (roots, shoup)
        return cache["roots"]

    # ------------------------------------------------------------------ lifetime
    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            nat.lib().hck_context_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    def set_conversion_engine(self, engine: str) -> None:
        """Engine of the key switch's ModUp / ModDown conversion sums: "mfma" (default, int8 matrix
        cores on balanced base-256 digits) or "valu" (FP64 multiply-accumulates).  Same results."""

        codes = {"valu": 0, "mfma": 1}
        if engine not in codes:
            raise ValueError(f"conversion engine must be one of {sorted(codes)}, got {engine!r}")
        nat.check(nat.lib().hck_context_set_conv_engine(self._h, codes[engine]), "hck_context_set_conv_engine")

    # ------------------------------------------------------------------ parameters
    def scale_at(self, cur_limbs: int) -> float:
        """Default encoding scale at a limb count (fixed scale mode)."""

        return self._scale

    def rescale_divisor_at(self, limbs: int) -> int:
        """The prime a rescale from ``limbs`` limbs divides by (q_{limbs-1})."""

        return int(self.q_primes[int(limbs) - 1])

    def q_prime_idx(self, limbs: int) -> list[int]:
        return list(range(int(limbs)))

    def ext_prime_idx(self, limbs: int) -> list[int]:
        return list(range(int(limbs))) + [self.L + k for k in range(self.K)]

    def galois_element(self, rotation: int) -> int:
        """5^r mod 2N for a left rotation by r slots (r taken mod N/2); 2N - 1 for conjugation."""

        r = int(rotation) % self.max_slots
        return pow(5, r, self.M)

    # ------------------------------------------------------------------ memory
    def workspace(self, nbytes: int) -> torch.Tensor:
        nbytes = max(int(nbytes), 256)
        if self._ws is None or self._ws.numel() < nbytes:
            self._ws = None
            self._ws = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        return self._ws

    def empty(self, *shape) -> torch.Tensor:
        return torch.empty(shape, dtype=torch.uint64, device=self.device)

    def zeros(self, *shape) -> torch.Tensor:
        return torch.zeros(shape, dtype=torch.uint64, device=self.device)

    # ------------------------------------------------------------------ kernels
    @staticmethod
    def _check_poly(t: torch.Tensor, limbs: int, n: int) -> None:
        if t.dtype != torch.uint64 or t.dim() != 3:
            raise ValueError("expected a [batch][limbs][N] uint64 tensor")
        if t.shape[1] < limbs or t.shape[2] != n or t.stride(2) != 1 or t.stride(1) != n:
            raise ValueError("limb-major [batch][>=limbs][N] layout with contiguous limbs required")
        if t.device.type != "cuda":
            raise ValueError("tensors must live on the GPU")

    def ntt(self, src: torch.Tensor, dst: torch.Tensor | None = None, *, prime_idx, inverse: bool = False) -> torch.Tensor:
        limbs = len(prime_idx)
        self._check_poly(src, limbs, self.N)
        dst = src if dst is None else dst
        self._check_poly(dst, limbs, self.N)
        fn = nat.lib().hck_ntt_inverse if inverse else nat.lib().hck_ntt_forward
        nat.check(fn(self._h, src.data_ptr(), dst.data_ptr(), src.shape[0], _bstride(src), _bstride(dst),
                     limbs, nat.int_array(prime_idx), _stream_ptr(self.device)),
                  "hck_ntt_inverse" if inverse else "hck_ntt_forward")
        return dst

    def automorphism(self, src: torch.Tensor, galois: int, limbs: int, out: torch.Tensor | None = None) -> torch.Tensor:
        self._check_poly(src, limbs, self.N)
        if out is None:
            out = self.empty(src.shape[0], limbs, self.N)
        self._check_poly(out, limbs, self.N)
        nat.check(nat.lib().hck_automorphism(self._h, src.data_ptr(), out.data_ptr(), src.shape[0],
                                             _bstride(src), _bstride(out), limbs, int(galois),
                                             _stream_ptr(self.device)), "hck_automorphism")
        return out

    def poly_op(self, op: int, out: torch.Tensor, a: torch.Tensor, b: torch.Tensor | None = None, *,
                prime_idx, scalar=None) -> torch.Tensor:
        limbs = len(prime_idx)
        for t in (out, a) + ((b,) if b is not None else ()):
            self._check_poly(t, limbs, self.N)
        bb = b if b is not None else a
        sc = nat.u64_array(scalar) if scalar is not None else None
        nat.check(nat.lib().hck_poly_op(self._h, int(op), out.data_ptr(), a.data_ptr(), bb.data_ptr(),
                                        a.shape[0], _bstride(out), _bstride(a), _bstride(bb), limbs,
                                        nat.int_array(prime_idx), sc, _stream_ptr(self.device)),
                  "hck_poly_op")
        return out

    def from_signed(self, coeffs: torch.Tensor, prime_idx) -> torch.Tensor:
        """int64 coefficient vectors [batch][N] -> residues [batch][limbs][N] (coefficient domain)."""

        if coeffs.dtype != torch.int64 or coeffs.dim() != 2 or coeffs.shape[1] != self.N:
            raise ValueError("expected [batch][N] int64 coefficients")
        coeffs = coeffs.contiguous()
        out = self.empty(coeffs.shape[0], len(prime_idx), self.N)
        nat.check(nat.lib().hck_poly_from_signed(self._h, coeffs.data_ptr(), out.data_ptr(), coeffs.shape[0],
                                                 _bstride(coeffs), _bstride(out), len(prime_idx),
                                                 nat.int_array(prime_idx), _stream_ptr(self.device)),
                  "hck_poly_from_signed")
        return out

    def keyswitch(self, d: torch.Tensor, limbs: int, keys, *, add: torch.Tensor | None = None,
                  out_b: torch.Tensor | None = None, out_a: torch.Tensor | None = None):
        """Batched hybrid key switch; ``keys`` is one key tensor per batch item (or one for all)."""

        self._check_poly(d, limbs, self.N)
        B = d.shape[0]
        if isinstance(keys, torch.Tensor):
            keys = [keys] * B
        if len(keys) != B:
            raise ValueError("one key per batch item")
        for k in keys:
            self._check_key(k)
        out_b = self.empty(B, limbs, self.N) if out_b is None else out_b
        out_a = self.empty(B, limbs, self.N) if out_a is None else out_a
        if _bstride(out_b) != _bstride(out_a):
            raise ValueError("out_b and out_a need the same batch stride")
        if add is not None:
            self._check_poly(add, limbs, self.N)
        L = nat.lib()
        ws_bytes = L.hck_keyswitch_workspace_bytes(self._h, limbs, B)
        ws = self.workspace(ws_bytes)
        nat.check(L.hck_keyswitch(self._h, limbs, B, d.data_ptr(), _bstride(d),
                                  nat.ptr_array([k.data_ptr() for k in keys]),
                                  add.data_ptr() if add is not None else None,
                                  _bstride(add) if add is not None else 0,
                                  out_b.data_ptr(), out_a.data_ptr(), _bstride(out_b),
                                  ws.data_ptr(), ws.numel(), _stream_ptr(self.device)), "hck_keyswitch")
        return out_b, out_a

    def rotate_raw(self, c0: torch.Tensor, c1: torch.Tensor, limbs: int, galois: int, keys,
                   out0: torch.Tensor | None = None, out1: torch.Tensor | None = None,
                   acc: tuple[torch.Tensor, torch.Tensor] | None = None):
        """(sigma(c0) + KS_b(sigma(c1)), KS_a(sigma(c1))), plus ``acc`` = (acc0, acc1) when given.
        Outputs may be the ``acc`` tensors themselves, never c0 / c1.  ``galois`` is one element
        for every item or a sequence of one per item (then one key per item too); c0 / c1 with
        batch stride 0 (an expanded view) rotate one input by every element."""

        self._check_poly(c0, limbs, self.N)
        self._check_poly(c1, limbs, self.N)
        if _bstride(c0) != _bstride(c1):
            raise ValueError("c0 and c1 need the same batch stride")
        B = c0.shape[0]
        if isinstance(keys, torch.Tensor):
            keys = [keys] * B
        if len(keys) != B:
            raise ValueError("one key per batch item")
        for k in keys:
            self._check_key(k)
        out0 = self.empty(B, limbs, self.N) if out0 is None else out0
        out1 = self.empty(B, limbs, self.N) if out1 is None else out1
        for o in (out0, out1):
            self._check_poly(o, limbs, self.N)
            if o.shape[0] != B:
                raise ValueError("outputs need one row per input")
        if _bstride(out0) != _bstride(out1):
            raise ValueError("out0 and out1 need the same batch stride")
        a0 = a1 = None
        a_stride = 0
        if acc is not None:
            a0, a1 = acc
            for a in (a0, a1):
                self._check_poly(a, limbs, self.N)
                if a.shape[0] != B:
                    raise ValueError("accumulators need one row per input")
            if _bstride(a0) != _bstride(a1):
                raise ValueError("acc0 and acc1 need the same batch stride")
            a_stride = _bstride(a0)
        L = nat.lib()
        ws = self.workspace(L.hck_rotate_workspace_bytes(self._h, limbs, B))
        fn, gal, name = self._galois_arg(L, galois, B, "hck_rotate")
        nat.check(fn(self._h, limbs, B, gal, c0.data_ptr(), c1.data_ptr(), _bstride(c0),
                     nat.ptr_array([k.data_ptr() for k in keys]),
                     a0.data_ptr() if a0 is not None else None,
                     a1.data_ptr() if a1 is not None else None, a_stride,
                     out0.data_ptr(), out1.data_ptr(), _bstride(out0), ws.data_ptr(), ws.numel(),
                     _stream_ptr(self.device)), name)
        return out0, out1

    def rotate_rescale_raw(self, c0: torch.Tensor, c1: torch.Tensor, limbs: int, galois: int, keys):
        """``rotate_raw`` by one Galois element followed by the rescale, in one native call (the same
        residues): outputs [batch][limbs - 1][N]."""

        self._check_poly(c0, limbs, self.N)
        self._check_poly(c1, limbs, self.N)
        if limbs < 2:
            raise ValueError("a rescaled rotation needs at least two limbs")
        if _bstride(c0) != _bstride(c1):
            raise ValueError("c0 and c1 need the same batch stride")
        B = c0.shape[0]
        if isinstance(keys, torch.Tensor):
            keys = [keys] * B
        if len(keys) != B:
            raise ValueError("one key per batch item")
        for k in keys:
            self._check_key(k)
        out0, out1 = self.empty(B, limbs - 1, self.N), self.empty(B, limbs - 1, self.N)
        L = nat.lib()
        ws = self.workspace(L.hck_rotate_rescale_workspace_bytes(self._h, limbs, B))
        nat.check(L.hck_rotate_rescale(self._h, limbs, B, int(galois), c0.data_ptr(), c1.data_ptr(), _bstride(c0),
                                       nat.ptr_array([k.data_ptr() for k in keys]), out0.data_ptr(), out1.data_ptr(),
                                       (limbs - 1) * self.N, ws.data_ptr(), ws.numel(), _stream_ptr(self.device)),
                  "hck_rotate_rescale")
        return out0, out1

    def hoist_digits(self, c1: torch.Tensor, limbs: int) -> torch.Tensor:
        """The extended ModUp digits of every c1 ([inputs][limbs][N]) in the full NTT domain, as
        [inputs][beta][limbs + K][N] uint64 (hck_rotate_hoist_prepare): computed once, they serve
        any number of ``rotate_hoisted`` calls on these inputs."""

        self._check_poly(c1, limbs, self.N)
        B = int(c1.shape[0])
        L = nat.lib()
        beta = -(-int(limbs) // self.alpha)
        digits = torch.empty((B, beta, int(limbs) + self.K, self.N), dtype=torch.uint64, device=self.device)
        if digits.numel() * 8 != L.hck_rotate_hoist_digits_bytes(self._h, limbs, B):
            raise RuntimeError("hoisted digit layout disagrees with the library")
        ws = self.workspace(L.hck_rotate_hoist_workspace_bytes(self._h, limbs, B, 0))
        nat.check(L.hck_rotate_hoist_prepare(self._h, limbs, B, c1.data_ptr(), _bstride(c1), digits.data_ptr(),
                                             ws.data_ptr(), ws.numel(), _stream_ptr(self.device)),
                  "hck_rotate_hoist_prepare")
        return digits

    def rotate_hoisted(self, c0: torch.Tensor, c1: torch.Tensor, limbs: int, digits: torch.Tensor, galois, keys,
                       out0: torch.Tensor | None = None, out1: torch.Tensor | None = None):
        """Item i < len(galois): input i % inputs of (c0, c1) rotated by galois[i] with keys[i], from
        the digits ``hoist_digits(c1, limbs)`` (hck_rotate_hoisted); bit-identical to ``rotate_raw``
        with a Galois element per item on the repeated inputs."""

        self._check_poly(c0, limbs, self.N)
        self._check_poly(c1, limbs, self.N)
        if _bstride(c0) != _bstride(c1) or c0.shape[0] != c1.shape[0]:
            raise ValueError("c0 and c1 need the same inputs and batch stride")
        B = int(c0.shape[0])
        beta = -(-int(limbs) // self.alpha)
        if (digits.dtype != torch.uint64 or tuple(digits.shape) != (B, beta, int(limbs) + self.K, self.N)
                or not digits.is_contiguous()):
            raise ValueError("digits must come from hoist_digits of these inputs at this level")
        items = len(galois)
        if len(keys) != items:
            raise ValueError("one key per rotated item")
        for k in keys:
            self._check_key(k)
        out0 = self.empty(items, limbs, self.N) if out0 is None else out0
        out1 = self.empty(items, limbs, self.N) if out1 is None else out1
        for o in (out0, out1):
            self._check_poly(o, limbs, self.N)
            if o.shape[0] != items:
                raise ValueError("outputs need one row per rotated item")
        if _bstride(out0) != _bstride(out1):
            raise ValueError("out0 and out1 need the same batch stride")
        L = nat.lib()
        ws = self.workspace(L.hck_rotate_hoist_workspace_bytes(self._h, limbs, B, items))
        nat.check(L.hck_rotate_hoisted(self._h, limbs, B, items, nat.u32_array(galois), c0.data_ptr(), c1.data_ptr(),
                                       _bstride(c0), digits.data_ptr(), nat.ptr_array([k.data_ptr() for k in keys]),
                                       out0.data_ptr(), out1.data_ptr(), _bstride(out0), ws.data_ptr(), ws.numel(),
                                       _stream_ptr(self.device)), "hck_rotate_hoisted")
        return out0, out1

    @staticmethod
    def _galois_arg(L, galois, batch: int, base: str):
        """(entry point, galois argument, name): the per-item variant for a sequence."""

        if isinstance(galois, (list, tuple, np.ndarray)):
            if len(galois) != batch:
                raise ValueError("one Galois element per item")
            return getattr(L, base + "_many"), nat.u32_array(galois), base + "_many"
        return getattr(L, base), int(galois), base

    def rotate_ext(self, c0: torch.Tensor, c1: torch.Tensor, limbs: int, galois: int, keys,
                   out0: torch.Tensor | None = None, out1: torch.Tensor | None = None,
                   acc: tuple[torch.Tensor, torch.Tensor] | None = None):
        """Hoisted-form rotation ending in the extended basis: (P sigma(c0) + IP_b, IP_a) as
        [batch][limbs + K][N] tensors (Q limbs, then the special primes), plus the extended-basis
        ``acc`` pair when given (the outputs may be the ``acc`` tensors); ``moddown`` of each
        component gives ``rotate_raw``'s result bit for bit."""

        self._check_poly(c0, limbs, self.N)
        self._check_poly(c1, limbs, self.N)
        if _bstride(c0) != _bstride(c1):
            raise ValueError("c0 and c1 need the same batch stride")
        B = c0.shape[0]
        if isinstance(keys, torch.Tensor):
            keys = [keys] * B
        if len(keys) != B:
            raise ValueError("one key per batch item")
        for k in keys:
            self._check_key(k)
        ext = limbs + self.K
        out0 = self.empty(B, ext, self.N) if out0 is None else out0
        out1 = self.empty(B, ext, self.N) if out1 is None else out1
        for o in (out0, out1):
            self._check_poly(o, ext, self.N)
            if o.shape[0] != B:
                raise ValueError("outputs need one row per input")
        if _bstride(out0) != _bstride(out1):
            raise ValueError("out0 and out1 need the same batch stride")
        a0 = a1 = None
        a_stride = 0
        if acc is not None:
            a0, a1 = acc
            for a in (a0, a1):
                self._check_poly(a, ext, self.N)
                if a.shape[0] != B:
                    raise ValueError("accumulators need one row per input")
            if _bstride(a0) != _bstride(a1):
                raise ValueError("acc0 and acc1 need the same batch stride")
            a_stride = _bstride(a0)
        L = nat.lib()
        ws = self.workspace(L.hck_keyswitch_workspace_bytes(self._h, limbs, B))
        fn, gal, name = self._galois_arg(L, galois, B, "hck_rotate_ext")
        nat.check(fn(self._h, limbs, B, gal, c0.data_ptr(), c1.data_ptr(), _bstride(c0),
                     nat.ptr_array([k.data_ptr() for k in keys]),
                     a0.data_ptr() if a0 is not None else None,
                     a1.data_ptr() if a1 is not None else None, a_stride,
                     out0.data_ptr(), out1.data_ptr(), _bstride(out0), ws.data_ptr(), ws.numel(),
                     _stream_ptr(self.device)), name)
        return out0, out1

    def rotate_ext_sum(self, c0: torch.Tensor, c1: torch.Tensor, limbs: int, galois, keys, out0: torch.Tensor,
                       out1: torch.Tensor, acc: tuple[torch.Tensor, torch.Tensor] | None = None):
        """Grouped extended-basis rotations: c0 / c1 are [group][outputs][limbs][N] (any strides with
        a uniform item step), member m rotated by ``galois[m]`` with ``keys[m]``;
        out[o] = acc[o] + sum_m (P sigma_m(c0[m][o]) + IP(sigma_m(c1[m][o]))) as [outputs][limbs + K][N]
        (the outputs may be the ``acc`` tensors).  Equals ``len(galois)`` accumulating ``rotate_ext``
        calls bit for bit."""

        G, B = int(c0.shape[0]), int(c0.shape[1])
        if tuple(c1.shape[:2]) != (G, B) or len(galois) != G or len(keys) != G:
            raise ValueError("one Galois element and one key per member, matching c0 / c1")
        items = []
        for c in (c0, c1):
            flat = c.reshape(G * B, *c.shape[2:]) if c.is_contiguous() else None
            if flat is None or flat.data_ptr() != c.data_ptr():
                raise ValueError("grouped rotations need contiguous [group][outputs] inputs")
            self._check_poly(flat, limbs, self.N)
            items.append(flat)
        for k in keys:
            self._check_key(k)
        ext = limbs + self.K
        for o in (out0, out1):
            self._check_poly(o, ext, self.N)
            if o.shape[0] != B:
                raise ValueError("outputs need one row per output")
        a0 = a1 = None
        a_stride = 0
        if acc is not None:
            a0, a1 = acc
            for a in (a0, a1):
                self._check_poly(a, ext, self.N)
                if a.shape[0] != B:
                    raise ValueError("accumulators need one row per output")
            a_stride = _bstride(a0)
        L = nat.lib()
        ws = self.workspace(L.hck_keyswitch_workspace_bytes(self._h, limbs, G * B))
        nat.check(L.hck_rotate_ext_sum(self._h, limbs, B, G, nat.u32_array(galois), items[0].data_ptr(),
                                       items[1].data_ptr(), _bstride(items[0]),
                                       nat.ptr_array([k.data_ptr() for k in keys]),
                                       a0.data_ptr() if a0 is not None else None,
                                       a1.data_ptr() if a1 is not None else None, a_stride,
                                       out0.data_ptr(), out1.data_ptr(), _bstride(out0), ws.data_ptr(), ws.numel(),
                                       _stream_ptr(self.device)), "hck_rotate_ext_sum")
        return out0, out1

    def _pair(self, c0: torch.Tensor, c1: torch.Tensor, limbs: int, what: str) -> int:
        self._check_poly(c0, limbs, self.N)
        self._check_poly(c1, limbs, self.N)
        if c0.shape[0] != c1.shape[0] or _bstride(c0) != _bstride(c1):
            raise ValueError(f"{what}: both components need one shape and batch stride")
        return _bstride(c0)

    def tensor(self, a0, a1, b0, b1, limbs: int):
        """(a0 b0, a0 b1 + a1 b0, a1 b1) over ``limbs`` Q limbs, as [batch][limbs][N] tensors."""

        sa = self._pair(a0, a1, limbs, "tensor lhs")
        sb = self._pair(b0, b1, limbs, "tensor rhs")
        B = a0.shape[0]
        if b0.shape[0] != B:
            raise ValueError("tensor operands need the same batch")
        d = self.empty(3, B, limbs, self.N)
        nat.check(nat.lib().hck_tensor(self._h, limbs, B, a0.data_ptr(), a1.data_ptr(), sa, b0.data_ptr(),
                                       b1.data_ptr(), sb, d[0].data_ptr(), d[1].data_ptr(), d[2].data_ptr(),
                                       limbs * self.N, _stream_ptr(self.device)), "hck_tensor")
        return d[0], d[1], d[2]

    def relinearize_raw(self, d0, d1, d2, limbs: int, key: torch.Tensor):
        """(d0, d1) + KeySwitch(d2) with the s^2 -> s key."""

        self._check_key(key)
        s01 = self._pair(d0, d1, limbs, "relinearize")
        self._check_poly(d2, limbs, self.N)
        if d2.shape[0] != d0.shape[0] or _bstride(d2) != s01:
            raise ValueError("relinearize: d2 needs the shape and batch stride of d0 / d1")
        B = d0.shape[0]
        out = self.empty(2, B, limbs, self.N)
        L = nat.lib()
        ws = self.workspace(L.hck_relinearize_workspace_bytes(self._h, limbs, B))
        nat.check(L.hck_relinearize(self._h, limbs, B, d0.data_ptr(), d1.data_ptr(), d2.data_ptr(), s01,
                                    key.data_ptr(), out[0].data_ptr(), out[1].data_ptr(), limbs * self.N,
                                    ws.data_ptr(), ws.numel(), _stream_ptr(self.device)), "hck_relinearize")
        return out[0], out[1]

    def mul_relin_raw(self, a0, a1, b0, b1, limbs: int, key: torch.Tensor, stacked: bool = False):
        """Tensor product followed by relinearisation: a two-component [batch][limbs][N] pair (or,
        with ``stacked``, the one [2][batch][limbs][N] tensor holding both)."""

        self._check_key(key)
        sa = self._pair(a0, a1, limbs, "mul lhs")
        sb = self._pair(b0, b1, limbs, "mul rhs")
        B = a0.shape[0]
        if b0.shape[0] != B:
            raise ValueError("mul operands need the same batch")
        out = self.empty(2, B, limbs, self.N)
        L = nat.lib()
        ws = self.workspace(L.hck_mul_relin_workspace_bytes(self._h, limbs, B))
        nat.check(L.hck_mul_relin(self._h, limbs, B, a0.data_ptr(), a1.data_ptr(), sa, b0.data_ptr(), b1.data_ptr(),
                                  sb, key.data_ptr(), out[0].data_ptr(), out[1].data_ptr(), limbs * self.N,
                                  ws.data_ptr(), ws.numel(), _stream_ptr(self.device)), "hck_mul_relin")
        return out if stacked else (out[0], out[1])

    def mul_relin_rescale_raw(self, a0, a1, b0, b1, limbs: int, key: torch.Tensor, stacked: bool = False):
        """mul_relin_raw followed by the rescale, in one native call (the same residues): outputs at
        ``limbs - 1`` limbs."""

        self._check_key(key)
        if limbs < 2:
            raise ValueError("a rescaled product needs at least two limbs")
        sa = self._pair(a0, a1, limbs, "mul lhs")
        sb = self._pair(b0, b1, limbs, "mul rhs")
        B = a0.shape[0]
        if b0.shape[0] != B:
            raise ValueError("mul operands need the same batch")
        out = self.empty(2, B, limbs - 1, self.N)
        L = nat.lib()
        ws = self.workspace(L.hck_mul_relin_rescale_workspace_bytes(self._h, limbs, B))
        nat.check(L.hck_mul_relin_rescale(self._h, limbs, B, a0.data_ptr(), a1.data_ptr(), sa, b0.data_ptr(),
                                          b1.data_ptr(), sb, key.data_ptr(), out[0].data_ptr(), out[1].data_ptr(),
                                          (limbs - 1) * self.N, ws.data_ptr(), ws.numel(),
                                          _stream_ptr(self.device)), "hck_mul_relin_rescale")
        return out if stacked else (out[0], out[1])

    def mul_relin_rescale_postop_raw(self, a0, a1, b0, b1, limbs: int, key: torch.Tensor, *, apply_double: bool = False,
                                     sub: tuple | None = None, scalar=None):
        """``mul_relin_rescale_raw`` then (apply_double ? 2 : 1) * product - sub (+ the ``limbs - 1``
        canonical residues ``scalar`` on the c0 component) in the product's last kernel
        (hck_mul_relin_rescale_postop): a [2][batch][limbs - 1][N] tensor.  ``sub`` is a (c0, c1)
        pair of [batch][>= limbs - 1][N] tensors with one batch stride."""

        self._check_key(key)
        if limbs < 2:
            raise ValueError("a rescaled product needs at least two limbs")
        sa = self._pair(a0, a1, limbs, "mul lhs")
        sb = self._pair(b0, b1, limbs, "mul rhs")
        B = a0.shape[0]
        if b0.shape[0] != B:
            raise ValueError("mul operands need the same batch")
        s0 = s1 = None
        ss = 0
        if sub is not None:
            s0, s1 = sub
            ss = self._pair(s0, s1, limbs - 1, "postop sub")
            if s0.shape[0] != B:
                raise ValueError("postop sub needs one row per product")
        sc = None if scalar is None else nat.u64_array([int(v) for v in list(scalar)[:limbs - 1]])
        out = self.empty(2, B, limbs - 1, self.N)
        L = nat.lib()
        ws = self.workspace(L.hck_mul_relin_rescale_workspace_bytes(self._h, limbs, B))
        nat.check(L.hck_mul_relin_rescale_postop(
            self._h, limbs, B, a0.data_ptr(), a1.data_ptr(), sa, b0.data_ptr(), b1.data_ptr(), sb, key.data_ptr(),
            1 if apply_double else 0, s0.data_ptr() if s0 is not None else None,
            s1.data_ptr() if s1 is not None else None, ss, sc, out[0].data_ptr(), out[1].data_ptr(),
            (limbs - 1) * self.N, ws.data_ptr(), ws.numel(), _stream_ptr(self.device)), "hck_mul_relin_rescale_postop")
        return out

    def resident(self, table: np.ndarray) -> torch.Tensor:
        """A small host table (residue weights, constants) on the device, uploaded once: a later
        call with the same bytes reuses the device copy, so repeated evaluations (every bootstrap's
        EvalMod, every step's polynomials) issue no host-to-device copy."""

        a = np.ascontiguousarray(table)
        key = (a.dtype.str, a.shape, a.tobytes())
        cache = self.__dict__.setdefault("_resident", {})
        t = cache.get(key)
        if t is None:
            if len(cache) >= 4096:
                cache.clear()
            t = cache[key] = torch.from_numpy(a.copy()).to(self.device)
        return t

    def weighted_sum(self, x: torch.Tensor, weights: torch.Tensor, limbs: int) -> torch.Tensor:
        """out[g] = sum_j weights[g][j][l] x[j] per limb l: x [n][>= limbs][N], weights a uint64
        tensor [groups][n][limbs] of residues (moved to the device here)."""

        self._check_poly(x, limbs, self.N)
        n = int(x.shape[0])
        w = weights.to(self.device, torch.uint64).contiguous()
        if w.dim() != 3 or int(w.shape[1]) != n or int(w.shape[2]) != limbs:
            raise ValueError(f"weights must be [groups][{n}][{limbs}]")
        G = int(w.shape[0])
        out = self.empty(G, limbs, self.N)
        nat.check(nat.lib().hck_weighted_sum(self._h, limbs, n, G, x.data_ptr(), _bstride(x), w.data_ptr(),
                                             out.data_ptr(), limbs * self.N, _stream_ptr(self.device)),
                  "hck_weighted_sum")
        return out

    def _check_single(self, t: torch.Tensor, limbs: int, what: str) -> None:
        if t.dim() == 3 and t.shape[0] == 1:
            t = t[0]
        if (t.dtype != torch.uint64 or t.dim() != 2 or t.shape[0] < limbs or t.shape[1] != self.N
                or t.stride(1) != 1 or t.stride(0) != self.N or t.device.type != "cuda"):
            raise ValueError(f"{what}: expected one [>= {limbs}][N] uint64 GPU polynomial with contiguous limbs")

    def lincomb(self, xs, limbs: int, outs, weights: torch.Tensor | None = None):
        """out[g] = sum_t w[t] * xs[g][t] over the first ``limbs`` Q primes: ``xs`` is [groups][terms]
        single polynomials ([limbs'][N] or [1][limbs'][N] views, limbs' >= limbs, any allocation),
        ``outs`` one polynomial per group, ``weights`` a [terms][limbs] uint64 GPU table of residues
        (None: unit weights).  One hck_lincomb launch per 64 groups (or 256 operands)."""

        G = len(xs)
        if G != len(outs) or G < 1:
            raise ValueError("one output per group")
        T = len(xs[0])
        if T > 256:
            raise ValueError("at most 256 terms per linear combination")
        ptrs = []
        for row in xs:
            if len(row) != T:
                raise ValueError("every group needs the same number of terms")
            for t in row:
                self._check_single(t, limbs, "lincomb input")
                ptrs.append(t.data_ptr())
        for o in outs:
            self._check_single(o, limbs, "lincomb output")
        wp = None
        if weights is not None:
            if (weights.dtype != torch.uint64 or tuple(weights.shape) != (T, limbs) or not weights.is_contiguous()
                    or weights.device.type != "cuda"):
                raise ValueError(f"weights must be a contiguous [{T}][{limbs}] uint64 GPU table")
            wp = weights.data_ptr()
        per = max(1, min(64, 256 // T))  # the kernel's pointer-list capacity per launch
        optr = [o.data_ptr() for o in outs]
        for g0 in range(0, G, per):
            g1 = min(G, g0 + per)
            nat.check(nat.lib().hck_lincomb(self._h, int(limbs), g1 - g0, T, nat.ptr_array(ptrs[g0 * T:g1 * T]), wp,
                                            nat.ptr_array(optr[g0:g1]), _stream_ptr(self.device)), "hck_lincomb")
        return outs

    def lincomb_rescale(self, xs, limbs: int, outs, weights: torch.Tensor, add=None, add_groups=()) -> None:
        """outs[g] = rescale(sum_t w[t] * xs[g][t]) from ``limbs`` to ``limbs - 1`` limbs, plus the
        residues ``add`` (``limbs - 1`` canonical values) on the groups listed in ``add_groups``
        (hck_lincomb_rescale: the combination is never stored).  ``xs`` as for ``lincomb`` (at least
        ``limbs`` limbs each), ``outs`` [limbs - 1][N] polynomials, ``weights`` a [terms][limbs]
        uint64 GPU table."""

        G = len(xs)
        if G != len(outs) or G < 1:
            raise ValueError("one output per group")
        if limbs < 2:
            raise ValueError("a rescaled combination needs at least two limbs")
        T = len(xs[0])
        if T > 256:
            raise ValueError("at most 256 terms per linear combination")
        ptrs = []
        for row in xs:
            if len(row) != T:
                raise ValueError("every group needs the same number of terms")
            for t in row:
                self._check_single(t, limbs, "lincomb input")
                ptrs.append(t.data_ptr())
        for o in outs:
            self._check_single(o, limbs - 1, "lincomb output")
        if (weights.dtype != torch.uint64 or tuple(weights.shape) != (T, limbs) or not weights.is_contiguous()
                or weights.device.type != "cuda"):
            raise ValueError(f"weights must be a contiguous [{T}][{limbs}] uint64 GPU table")
        addv = None if add is None else nat.u64_array([int(v) for v in list(add)[:limbs - 1]])
        groups_with_add = {int(g) for g in add_groups}
        per = max(1, min(64, 256 // T))
        optr = [o.data_ptr() for o in outs]
        L = nat.lib()
        stream = _stream_ptr(self.device)
        for g0 in range(0, G, per):
            g1 = min(G, g0 + per)
            mask = sum(1 << (g - g0) for g in range(g0, g1) if g in groups_with_add)
            ws = self.workspace(L.hck_lincomb_rescale_workspace_bytes(self._h, limbs, g1 - g0))
            nat.check(L.hck_lincomb_rescale(self._h, int(limbs), g1 - g0, T, nat.ptr_array(ptrs[g0 * T:g1 * T]),
                                            weights.data_ptr(), nat.ptr_array(optr[g0:g1]), addv, mask,
                                            ws.data_ptr(), ws.numel(), stream), "hck_lincomb_rescale")

    def lincomb_ptrs(self, in_ptrs, limbs: int, out_ptrs, terms: int) -> None:
        """``lincomb`` with unit weights on raw device addresses: ``in_ptrs`` holds ``terms``
        addresses per group (group-major), ``out_ptrs`` one per group, each a [>= limbs][N] uint64
        polynomial with contiguous limbs on this context's device.  The caller has checked the
        tensors behind the addresses (the KV page pool does, once per component)."""

        G = len(out_ptrs)
        if G < 1 or len(in_ptrs) != G * terms or terms < 1 or terms > 256:
            raise ValueError("lincomb_ptrs: one output per group and `terms` inputs per output (<= 256)")
        per = max(1, min(64, 256 // terms))
        lib, stream = nat.lib(), _stream_ptr(self.device)
        for g0 in range(0, G, per):
            g1 = min(G, g0 + per)
            nat.check(lib.hck_lincomb(self._h, int(limbs), g1 - g0, terms, nat.ptr_array(in_ptrs[g0 * terms:g1 * terms]),
                                      None, nat.ptr_array(out_ptrs[g0:g1]), stream), "hck_lincomb")

    def moddown(self, x: torch.Tensor, limbs: int, out: torch.Tensor | None = None) -> torch.Tensor:
        """Extended-basis polys [polys][limbs + K][N] -> [polys][limbs][N] (divide by P, round)."""

        self._check_poly(x, limbs + self.K, self.N)
        out = self.empty(x.shape[0], limbs, self.N) if out is None else out
        self._check_poly(out, limbs, self.N)
        L = nat.lib()
        ws = self.workspace(L.hck_moddown_workspace_bytes(self._h, limbs, x.shape[0]))
        nat.check(L.hck_moddown(self._h, limbs, x.shape[0], x.data_ptr(), _bstride(x), out.data_ptr(),
                                _bstride(out), ws.data_ptr(), ws.numel(), _stream_ptr(self.device)),
                  "hck_moddown")
        return out

    def modraise(self, x: torch.Tensor, to_limbs: int, out: torch.Tensor | None = None) -> torch.Tensor:
        """Lift one-limb polys x[p][0] (modulo q_0, NTT domain) to ``to_limbs`` limbs: the centered
        coefficients of limb 0 reduced modulo every q_i (the first step of a bootstrap)."""

        self._check_poly(x, 1, self.N)
        to_limbs = int(to_limbs)
        P = int(x.shape[0])
        out = self.empty(P, to_limbs, self.N) if out is None else out
        self._check_poly(out, to_limbs, self.N)
        L = nat.lib()
        ws = self.workspace(L.hck_modraise_workspace_bytes(self._h, to_limbs, P))
        nat.check(L.hck_modraise(self._h, to_limbs, P, x.data_ptr(), _bstride(x), out.data_ptr(), _bstride(out),
                                 ws.data_ptr(), ws.numel(), _stream_ptr(self.device)), "hck_modraise")
        return out

    def rescale_raw(self, x: torch.Tensor, limbs: int, out: torch.Tensor | None = None) -> torch.Tensor:
        self._check_poly(x, limbs, self.N)
        if limbs < 2:
            raise ValueError("rescale needs at least two limbs")
        if out is None:
            out = self.empty(x.shape[0], limbs - 1, self.N)
        else:
            self._check_poly(out, limbs - 1, self.N)
            if out.shape[0] != x.shape[0]:
                raise ValueError(f"out holds {out.shape[0]} polys for {x.shape[0]} inputs")
        L = nat.lib()
        ws = self.workspace(L.hck_rescale_workspace_bytes(self._h, limbs, x.shape[0]))
        nat.check(L.hck_rescale(self._h, limbs, x.shape[0], x.data_ptr(), _bstride(x), out.data_ptr(),
                                _bstride(out), ws.data_ptr(), ws.numel(), _stream_ptr(self.device)),
                  "hck_rescale")
        return out

    def bsgs_mac(self, babies_c0, babies_c1, pts: torch.Tensor, limbs: int, giants: int,
                 out: torch.Tensor | None = None, prime_idx=None) -> torch.Tensor:
        """Baby-step partial sums res[c][g][i] = sum_b pts[g*nb + b] * baby_b[i][c] (exact residues).
        babies_c0/c1: one [inputs][>=limbs][N] tensor per baby step (same batch stride); limb l
        uses prime prime_idx[l] (default: the first ``limbs`` Q primes)."""

        prime_idx = self.q_prime_idx(limbs) if prime_idx is None else list(prime_idx)
        if len(prime_idx) != limbs:
            raise ValueError("one prime index per limb")

        nb = len(babies_c0)
        if nb != len(babies_c1) or nb < 1:
            raise ValueError("one (c0, c1) pair per baby step")
        ni = int(babies_c0[0].shape[0])
        stride = babies_c0[0].stride(0)
        for t in list(babies_c0) + list(babies_c1):
            self._check_poly(t, limbs, self.N)
            if t.shape[0] != ni or _bstride(t) != stride:
                raise ValueError("baby tensors need one shape and batch stride")
        self._check_poly(pts, limbs, self.N)
        if pts.shape[0] != giants * nb:
            raise ValueError(f"expected {giants * nb} plaintext rows, got {pts.shape[0]}")
        if out is None:
            out = self.empty(2, giants, ni, limbs, self.N)
        if tuple(out.shape) != (2, giants, ni, limbs, self.N) or not out.is_contiguous():
            raise ValueError("out must be a contiguous [2][giants][inputs][limbs][N] tensor")
        nat.check(nat.lib().hck_bsgs_mac(self._h, limbs, nat.int_array(prime_idx), ni, nb, giants,
                                         nat.ptr_array([t.data_ptr() for t in babies_c0]),
                                         nat.ptr_array([t.data_ptr() for t in babies_c1]), stride,
                                         pts.data_ptr(), _bstride(pts), out.data_ptr(),
                                         _stream_ptr(self.device)), "hck_bsgs_mac")
        return out

    def pack_diagonals(self, weight: torch.Tensor, *, lanes: int, lane_shift: int, baby_steps: int,
                       giant_base: int, giant_count: int) -> torch.Tensor:
        """Diagonal rows [giant_count * baby_steps][N/2] (float64) of one BSGS chunk."""

        if weight.dtype != torch.float64 or weight.dim() != 2 or weight.shape[0] != weight.shape[1]:
            raise ValueError("weight must be a square float64 matrix")
        weight = weight.contiguous()
        out = torch.empty((giant_count * baby_steps, self.max_slots), dtype=torch.float64, device=self.device)
        nat.check(nat.lib().hck_pack_diagonals(self._h, weight.data_ptr(), int(weight.shape[0]), int(lanes),
                                               int(lane_shift), int(baby_steps), int(giant_base),
                                               int(giant_count), out.data_ptr(), _stream_ptr(self.device)),
                  "hck_pack_diagonals")
        return out

    def slot_rows(self, values, slots: int):
        """Values (one vector or [rows][slots]; numpy or torch, real or complex) -> device float64
        (re, im or None) rows of N/2 slots: a sparse vector (slots < N/2) is tiled, which is its
        encoding in the subring X^(N / 2 slots)."""

        v = values
        if isinstance(v, torch.Tensor):
            v = v.detach().to(self.device)
        else:
            v = torch.from_numpy(np.asarray(v)).to(self.device)
        if v.dim() <= 1:
            v = v.reshape(1, -1)
        else:
            v = v.reshape(v.shape[0], -1)
        n = int(v.shape[1])
        slots = int(slots)
        if n > slots or slots > self.max_slots or self.max_slots % slots or slots & (slots - 1):
            raise ValueError(f"{n} values do not fit {slots} slots (a power of two up to {self.max_slots})")
        if n < slots:
            v = torch.nn.functional.pad(v, (0, slots - n))
        reps = self.max_slots // slots
        if torch.is_complex(v):
            re = v.real.to(torch.float64).repeat(1, reps).contiguous()
            im = v.imag.to(torch.float64).repeat(1, reps).contiguous()
            return re, (im if bool(torch.any(im != 0)) else None)
        return v.to(torch.float64).repeat(1, reps).contiguous(), None

    def encode(self, values: torch.Tensor, scale: float, limbs: int, *, values_im: torch.Tensor | None = None,
               prime_idx=None, out: torch.Tensor | None = None, flags: torch.Tensor | None = None) -> torch.Tensor:
        """Encode slot rows [rows][N/2] (float64 on the device: real parts, optional imaginary parts)
        into NTT-domain residues [rows][limbs][N], limb l modulo prime prime_idx[l] (default: the
        first ``limbs`` Q primes; ``ext_prime_idx`` gives an extended-basis plaintext).

        Overflow (a coefficient reaching 2^61) sets an int32 device flag per row.  Without
        ``flags`` they are read back here (one host sync) and raise; with a caller-owned
        ``flags`` tensor ([>= rows] int32, zeroed once) the flags accumulate there for one check
        at the caller's next synchronisation point (``check_encode_flags``)."""

        for v in (values,) + ((values_im,) if values_im is not None else ()):
            if v.dtype != torch.float64 or v.dim() != 2 or v.shape[1] != self.max_slots:
                raise ValueError("values must be [rows][N/2] float64")
            if v.device.type != "cuda":
                raise ValueError("values must live on the GPU")
        values = values.contiguous()
        rows = int(values.shape[0])
        if values_im is not None:
            if values_im.shape[0] != rows:
                raise ValueError("values_im needs one row per values row")
            values_im = values_im.contiguous()
        prime_idx = self.q_prime_idx(limbs) if prime_idx is None else list(prime_idx)
        if len(prime_idx) != int(limbs):
            raise ValueError("one prime index per limb")
        if out is None:
            out = self.empty(rows, limbs, self.N)
        self._check_poly(out, limbs, self.N)
        own = flags is None
        if own:
            flags = torch.zeros(max(rows, 1), dtype=torch.int32, device=self.device)
        elif flags.dtype != torch.int32 or flags.numel() < rows or not flags.is_contiguous():
            raise ValueError("flags must be a contiguous int32 tensor with one entry per row")
        L = nat.lib()
        ws = self.workspace(L.hck_encode_workspace_bytes(self._h, rows))
        nat.check(L.hck_encode(self._h, values.data_ptr(), values_im.data_ptr() if values_im is not None else None,
                               rows, float(scale), int(limbs), nat.int_array(prime_idx), out.data_ptr(),
                               _bstride(out), ws.data_ptr(), ws.numel(), flags.data_ptr(),
                               _stream_ptr(self.device)), "hck_encode")
        if own:
            self.check_encode_flags(flags)
        return out

    @staticmethod
    def check_encode_flags(flags: torch.Tensor) -> None:
        if bool(flags.any().item()):
            raise ValueError("encoded coefficient reached 2^61: lower the scale or the value range")

    def encode_real(self, values: torch.Tensor, scale: float, limbs: int, out: torch.Tensor | None = None,
                    flags: torch.Tensor | None = None) -> torch.Tensor:
        """Real slot rows [rows][N/2] -> NTT-domain residues over the first ``limbs`` Q primes."""

        return self.encode(values, scale, limbs, out=out, flags=flags)

    def _check_key(self, k: torch.Tensor) -> None:
        shape = (2, self.beta_max, self.L + self.K, self.N)
        if k.dtype != torch.uint64 or tuple(k.shape) != shape or not k.is_contiguous():
            raise ValueError(f"key must be a contiguous uint64 tensor of shape {shape}")

    # ------------------------------------------------------------------ keys
    def make_switching_key(self, s_from: np.ndarray, s_to: np.ndarray, a: np.ndarray, e: np.ndarray) -> torch.Tensor:
        """Key switching s_from -> s_to (coefficient int64 vectors) on the GPU:
        b_j = -a_j s_to + e_j + [P]_{q_i} s_from on digit j's Q limbs, a_j as given
        (a: [beta_max][L+K][N] uniform residues, NTT domain; e: [beta_max][N] int64)."""

        np_ = self.L + self.K
        idx = list(range(np_))
        dev = self.device
        sf = self.from_signed(torch.from_numpy(np.ascontiguousarray(s_from, dtype=np.int64)).reshape(1, -1).to(dev), idx)
        st = self.from_signed(torch.from_numpy(np.ascontiguousarray(s_to, dtype=np.int64)).reshape(1, -1).to(dev), idx)
        self.ntt(sf, prime_idx=idx)
        self.ntt(st, prime_idx=idx)
        key = self.empty(2, self.beta_max, np_, self.N)
        a_t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint64)).to(dev)
        key[1].copy_(a_t)
        e_t = torch.from_numpy(np.ascontiguousarray(e, dtype=np.int64)).to(dev)
        ee = self.from_signed(e_t, idx)                      # [beta][np][N]
        self.ntt(ee, prime_idx=idx)
        pmod = []
        for i in range(np_):
            v = 1
            for pk in self.p_primes:
                v = v * pk % self.primes[i]
            pmod.append(v if i < self.L else 0)
        ps = self.empty(1, np_, self.N)
        self.poly_op(nat.HCK_OP_MUL_SCALAR, ps, sf, prime_idx=idx, scalar=pmod)
        for j in range(self.beta_max):
            b = key[0, j].unsqueeze(0)
            self.poly_op(nat.HCK_OP_MUL, b, a_t[j].unsqueeze(0), st, prime_idx=idx)
            self.poly_op(nat.HCK_OP_SUB, b, ee[j].unsqueeze(0), b, prime_idx=idx)
            lo, hi = j * self.alpha, min((j + 1) * self.alpha, self.L)
            sub = list(range(lo, hi))
            bv = key[0, j, lo:hi].unsqueeze(0)
            self.poly_op(nat.HCK_OP_ADD, bv, bv, ps[:, lo:hi], prime_idx=sub)
        return key

    def get_rotation_key_for_limbs(self, rotation: int, cur_limbs: int) -> torch.Tensor:
        g = self.galois_element(rotation) if int(rotation) != self.M - 1 else self.M - 1
        key = self.rotation_keys.get(g)
        if key is None:
            raise KeyError(f"no rotation key for rotation {rotation} (galois element {g})")
        return key

    def key_for_galois(self, g: int) -> torch.Tensor:
        key = self.rotation_keys.get(int(g))
        if key is None:
            raise KeyError(f"no key for galois element {g}")
        return key

    def clear_cuda_rotation_cache(self, keep_rotations=()) -> None:
        keep = {self.galois_element(r) for r in keep_rotations}
        for g in list(self.rotation_keys):
            if g not in keep:
                del self.rotation_keys[g]


__all__ = ["CKKSContext", "Cipher", "CipherState"]
