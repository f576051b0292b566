"""ctypes loader for the CPU oracle (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
module, and only as the checker or the timed CPU baseline: the product package ``holmes_amd``
never imports it.  The oracle library is ``oracle/_build/libckks_oracle.so`` built from
``oracle/ckks_oracle.c`` by ``oracle/Makefile``.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "_build" / "libckks_oracle.so"

_u64p = ctypes.POINTER(ctypes.c_uint64)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int)
_vp = ctypes.c_void_p
_f64p = ctypes.POINTER(ctypes.c_double)
_lib = None


def build() -> None:
    import subprocess

    subprocess.run(["make", "-B", "-C", str(_HERE)], check=True, capture_output=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    L = ctypes.CDLL(str(LIB_PATH))
    u64, i = ctypes.c_uint64, ctypes.c_int
    sig = {
        "or_is_prime": (i, [u64]),
        "or_gen_primes": (i, [i, i, i, _u64p, i, _u64p]),
        "or_find_psi": (u64, [u64, i]),
        "or_make_tables": (None, [u64, u64, i, _u64p, _u64p]),
        "or_ntt_fwd": (None, [_u64p, i, u64, _u64p]),
        "or_ntt_inv": (None, [_u64p, i, u64, _u64p]),
        "or_automorph_coeff": (None, [_u64p, _u64p, i, u64, u64]),
        "or_automorph_ntt": (None, [_u64p, _u64p, i, u64]),
        "or_ctx_new": (_vp, [i, i, i, i, _u64p]),
        "or_ctx_free": (None, [_vp]),
        "or_ctx_tables": (None, [_vp, i, _u64p, _u64p]),
        "or_ntt_fwd_limbs": (None, [_vp, _u64p, i, _i32p]),
        "or_ntt_inv_limbs": (None, [_vp, _u64p, i, _i32p]),
        "or_modup": (None, [_vp, i, i, _u64p, _u64p]),
        "or_moddown": (None, [_vp, i, _u64p, _u64p]),
        "or_keyswitch": (None, [_vp, i, _u64p, _u64p, _u64p, _u64p]),
        "or_keyswitch_batch": (None, [_vp, i, i, _u64p, ctypes.POINTER(_u64p), _u64p, _u64p]),
        "or_rotate": (None, [_vp, i, u64, _u64p, _u64p, _u64p, _u64p, _u64p]),
        "or_rescale": (None, [_vp, i, _u64p, _u64p]),
        "or_make_ksk": (None, [_vp, _i64p, _i64p, _u64p, _i64p, _u64p]),
        "or_bsgs_mac": (None, [_vp, i, i, i, _u64p, _u64p, _u64p]),
        "or_mul_limbs": (None, [_vp, i, _u64p, _u64p, _u64p]),
        "or_tensor": (None, [_vp, i, _u64p, _u64p, _u64p, _u64p, _u64p, _u64p, _u64p]),
        "or_weighted_sum": (None, [_vp, i, i, i, _u64p, _u64p, _u64p]),
        "or_modraise": (None, [_vp, i, _u64p, _u64p]),
        "or_num_threads": (i, []),
        "or_encode_twiddles": (None, [i, _f64p, _f64p]),
        "or_special_ifft": (None, [i, _f64p, _f64p, _f64p, _f64p]),
        "or_encode_real": (i, [_vp, _f64p, ctypes.c_double, i, _i32p, i, _u64p]),
        "or_encode_stage1": (None, [_vp, _f64p, _f64p]),
        "or_pack_diagonals": (None, [_f64p, i, i, i, i, i, i, i, _f64p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    if a.dtype == np.uint64:
        return a.ctypes.data_as(_u64p)
    if a.dtype == np.int64:
        return a.ctypes.data_as(_i64p)
    if a.dtype == np.int32:
        return a.ctypes.data_as(_i32p)
    if a.dtype == np.float64:
        return a.ctypes.data_as(_f64p)
    raise TypeError(a.dtype)


def is_prime(n: int) -> bool:
    return bool(lib().or_is_prime(int(n)))


def gen_primes(log_n: int, bits: int, count: int, exclude=()) -> list[int]:
    excl = np.ascontiguousarray(np.asarray(list(exclude), dtype=np.uint64).reshape(-1))
    if excl.size == 0:
        excl = np.zeros(1, dtype=np.uint64)
        n_excl = 0
    else:
        n_excl = int(excl.size)
    out = np.zeros(max(1, count), dtype=np.uint64)
    got = lib().or_gen_primes(log_n, bits, count, _p(excl), n_excl, _p(out))
    if got != count:
        raise ValueError("not enough primes")
    return [int(v) for v in out[:count]]


def find_psi(q: int, log_n: int) -> int:
    return int(lib().or_find_psi(int(q), int(log_n)))


def make_tables(q: int, psi: int, log_n: int):
    n = 1 << log_n
    a = np.zeros(n, dtype=np.uint64)
    b = np.zeros(n, dtype=np.uint64)
    lib().or_make_tables(int(q), int(psi), int(log_n), _p(a), _p(b))
    return a, b


def ntt_fwd(a: np.ndarray, log_n: int, q: int, psi_rev: np.ndarray) -> np.ndarray:
    out = np.ascontiguousarray(a, dtype=np.uint64).copy()
    lib().or_ntt_fwd(_p(out), log_n, int(q), _p(np.ascontiguousarray(psi_rev, dtype=np.uint64)))
    return out


def ntt_inv(a: np.ndarray, log_n: int, q: int, ipsi_rev: np.ndarray) -> np.ndarray:
    out = np.ascontiguousarray(a, dtype=np.uint64).copy()
    lib().or_ntt_inv(_p(out), log_n, int(q), _p(np.ascontiguousarray(ipsi_rev, dtype=np.uint64)))
    return out


def automorph_coeff(a: np.ndarray, log_n: int, g: int, q: int) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint64)
    out = np.zeros_like(a)
    lib().or_automorph_coeff(_p(out), _p(a), log_n, int(g), int(q))
    return out


def automorph_ntt(a: np.ndarray, log_n: int, g: int) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint64)
    out = np.zeros_like(a)
    lib().or_automorph_ntt(_p(out), _p(a), log_n, int(g))
    return out


class OracleContext:
    """Oracle CKKS context: primes (Q then P) and its own NTT tables."""

    def __init__(self, log_n: int, L: int, K: int, alpha: int, primes):
        self.log_n, self.L, self.K, self.alpha = int(log_n), int(L), int(K), int(alpha)
        self.n = 1 << self.log_n
        self.primes = [int(p) for p in primes]
        assert len(self.primes) == self.L + self.K
        arr = np.asarray(self.primes, dtype=np.uint64)
        self._h = lib().or_ctx_new(self.log_n, self.L, self.K, self.alpha, _p(arr))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.or_ctx_free(h)
            self._h = None

    def beta(self, ell: int) -> int:
        return (int(ell) + self.alpha - 1) // self.alpha

    def tables(self, prime_idx: int):
        a = np.zeros(self.n, dtype=np.uint64)
        b = np.zeros(self.n, dtype=np.uint64)
        lib().or_ctx_tables(self._h, int(prime_idx), _p(a), _p(b))
        return a, b

    def ntt_fwd_limbs(self, data: np.ndarray, prime_idx) -> np.ndarray:
        out = np.ascontiguousarray(data, dtype=np.uint64).copy()
        idx = np.ascontiguousarray(np.asarray(prime_idx, dtype=np.int32))
        lib().or_ntt_fwd_limbs(self._h, _p(out), int(idx.size), _p(idx))
        return out

    def ntt_inv_limbs(self, data: np.ndarray, prime_idx) -> np.ndarray:
        out = np.ascontiguousarray(data, dtype=np.uint64).copy()
        idx = np.ascontiguousarray(np.asarray(prime_idx, dtype=np.int32))
        lib().or_ntt_inv_limbs(self._h, _p(out), int(idx.size), _p(idx))
        return out

    def modup(self, ell: int, digit: int, d: np.ndarray) -> np.ndarray:
        d = np.ascontiguousarray(d, dtype=np.uint64)
        ext = np.zeros((ell + self.K, self.n), dtype=np.uint64)
        lib().or_modup(self._h, int(ell), int(digit), _p(d), _p(ext))
        return ext

    def moddown(self, ell: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.uint64)
        out = np.zeros((ell, self.n), dtype=np.uint64)
        lib().or_moddown(self._h, int(ell), _p(x), _p(out))
        return out

    def keyswitch(self, ell: int, d: np.ndarray, ksk: np.ndarray):
        d = np.ascontiguousarray(d, dtype=np.uint64)
        ksk = np.ascontiguousarray(ksk, dtype=np.uint64)
        ob = np.zeros((ell, self.n), dtype=np.uint64)
        oa = np.zeros((ell, self.n), dtype=np.uint64)
        lib().or_keyswitch(self._h, int(ell), _p(d), _p(ksk), _p(ob), _p(oa))
        return ob, oa

    def keyswitch_batch(self, ell: int, d: np.ndarray, ksks):
        d = np.ascontiguousarray(d, dtype=np.uint64)
        count = int(d.shape[0])
        ksks = [np.ascontiguousarray(k, dtype=np.uint64) for k in ksks]
        arr = (_u64p * count)(*[_p(k) for k in ksks])
        ob = np.zeros((count, ell, self.n), dtype=np.uint64)
        oa = np.zeros((count, ell, self.n), dtype=np.uint64)
        lib().or_keyswitch_batch(self._h, int(ell), count, _p(d), arr, _p(ob), _p(oa))
        return ob, oa

    def rotate(self, ell: int, g: int, c0: np.ndarray, c1: np.ndarray, ksk: np.ndarray):
        c0 = np.ascontiguousarray(c0, dtype=np.uint64)
        c1 = np.ascontiguousarray(c1, dtype=np.uint64)
        ksk = np.ascontiguousarray(ksk, dtype=np.uint64)
        o0 = np.zeros((ell, self.n), dtype=np.uint64)
        o1 = np.zeros((ell, self.n), dtype=np.uint64)
        lib().or_rotate(self._h, int(ell), int(g), _p(c0), _p(c1), _p(ksk), _p(o0), _p(o1))
        return o0, o1

    def rescale(self, ell: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.uint64)
        out = np.zeros((ell - 1, self.n), dtype=np.uint64)
        lib().or_rescale(self._h, int(ell), _p(x), _p(out))
        return out

    def make_ksk(self, s_from, s_to, a, e) -> np.ndarray:
        s_from = np.ascontiguousarray(s_from, dtype=np.int64)
        s_to = np.ascontiguousarray(s_to, dtype=np.int64)
        a = np.ascontiguousarray(a, dtype=np.uint64)
        e = np.ascontiguousarray(e, dtype=np.int64)
        beta = self.beta(self.L)
        out = np.zeros((2, beta, self.L + self.K, self.n), dtype=np.uint64)
        lib().or_make_ksk(self._h, _p(s_from), _p(s_to), _p(a), _p(e), _p(out))
        return out

    def encode_real(self, values: np.ndarray, scale: float, prime_idx, ntt: bool = True):
        """Encode one real slot vector (N/2 values): (residues [limbs][N], ok)."""

        values = np.ascontiguousarray(values, dtype=np.float64)
        idx = np.ascontiguousarray(np.asarray(prime_idx, dtype=np.int32))
        out = np.zeros((idx.size, self.n), dtype=np.uint64)
        rc = lib().or_encode_real(self._h, _p(values), float(scale), int(idx.size), _p(idx), int(bool(ntt)), _p(out))
        return out, rc == 0

    def encode_stage1(self, values: np.ndarray) -> np.ndarray:
        """The special IFFT's output w (interleaved Re, Im per slot; N doubles) that encode_real
        rounds: the encode sidecar's stage-2 input (bench/cmp/kernels/holmes_encode.cu:108-111)."""

        values = np.ascontiguousarray(values, dtype=np.float64)
        out = np.empty(1 << self.log_n, dtype=np.float64)
        lib().or_encode_stage1(self._h, _p(values), _p(out))
        return out

    def tensor(self, limbs: int, a0, a1, b0, b1):
        """(a0 b0, a0 b1 + a1 b0, a1 b1) over the first ``limbs`` Q primes ([limbs][N] each)."""

        ins = [np.ascontiguousarray(np.asarray(v)[:limbs], dtype=np.uint64) for v in (a0, a1, b0, b1)]
        outs = [np.zeros((limbs, self.n), dtype=np.uint64) for _ in range(3)]
        lib().or_tensor(self._h, int(limbs), *[_p(v) for v in ins], *[_p(v) for v in outs])
        return tuple(outs)

    def relinearize(self, limbs: int, d0, d1, d2, rlk: np.ndarray):
        """(d0, d1) + KeySwitch(d2) with the s^2 -> s key ``rlk`` (the oracle's key switch)."""

        kb, ka = self.keyswitch(limbs, d2, rlk)
        q = np.asarray(self.primes[:limbs], dtype=np.uint64)[:, None]
        return (np.asarray(d0[:limbs], dtype=np.uint64) + kb) % q, (np.asarray(d1[:limbs], dtype=np.uint64) + ka) % q

    def mul_relin(self, limbs: int, a0, a1, b0, b1, rlk: np.ndarray):
        d0, d1, d2 = self.tensor(limbs, a0, a1, b0, b1)
        return self.relinearize(limbs, d0, d1, d2, rlk)

    def modraise(self, to: int, x: np.ndarray) -> np.ndarray:
        """One NTT-domain limb modulo q_0 lifted (centered) to ``to`` limbs."""

        x = np.ascontiguousarray(np.asarray(x).reshape(-1)[: self.n], dtype=np.uint64)
        out = np.zeros((to, self.n), dtype=np.uint64)
        lib().or_modraise(self._h, int(to), _p(x), _p(out))
        return out

    def weighted_sum(self, limbs: int, x: np.ndarray, w: np.ndarray) -> np.ndarray:
        """out[g] = sum_j w[g][j][l] x[j][l]: x [n][limbs][N], w [groups][n][limbs]."""

        x = np.ascontiguousarray(np.asarray(x)[:, :limbs], dtype=np.uint64)
        w = np.ascontiguousarray(w, dtype=np.uint64)
        G, n = int(w.shape[0]), int(w.shape[1])
        out = np.zeros((G, limbs, self.n), dtype=np.uint64)
        lib().or_weighted_sum(self._h, int(limbs), n, G, _p(x), _p(w), _p(out))
        return out

    def bsgs_mac(self, limbs: int, nb: int, G: int, pt: np.ndarray, baby: np.ndarray) -> np.ndarray:
        pt = np.ascontiguousarray(pt, dtype=np.uint64)
        baby = np.ascontiguousarray(baby, dtype=np.uint64)
        res = np.zeros((2, G, limbs, self.n), dtype=np.uint64)
        lib().or_bsgs_mac(self._h, int(limbs), int(nb), int(G), _p(pt), _p(baby), _p(res))
        return res


def encode_twiddles(log_n: int):
    n = 1 << (log_n - 1)
    re = np.zeros(n, dtype=np.float64)
    im = np.zeros(n, dtype=np.float64)
    lib().or_encode_twiddles(int(log_n), _p(re), _p(im))
    return re, im


def pack_diagonals(W: np.ndarray, lanes: int, lane_shift: int, baby_steps: int, giant_base: int,
                   giant_count: int, slots: int) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.float64)
    D = int(W.shape[0])
    out = np.zeros((giant_count * baby_steps, slots), dtype=np.float64)
    lib().or_pack_diagonals(_p(W), D, int(lanes), int(lane_shift), int(baby_steps), int(giant_base),
                            int(giant_count), int(slots), _p(out))
    return out


def num_threads() -> int:
    return int(lib().or_num_threads())


def cpu_count_env() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
