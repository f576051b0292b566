"""CPU checks of the C ABI: the library builds, loads and exports every declared symbol, and the
argument validation that needs no GPU rejects bad inputs with the documented codes."""

import ctypes
import re
from pathlib import Path

import pytest

from holmes_amd import _native as nat

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "holmes_ckks.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:hck|holmes)_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = nat.lib()
    names = declared_symbols()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name
    # the binding table covers the header exactly
    assert sorted(nat.SIGNATURES) == names


def test_bindings_match_the_header_arity():
    """Every ctypes signature has as many arguments as the header's prototype: a binding that
    drifts from the header would pass shifted pointers to the kernels."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    decls = re.findall(r"\b((?:hck|holmes)_[a-z0-9_]+)\s*\(([^;{)]*)\)\s*;", text)
    assert len(decls) >= len(nat.SIGNATURES)
    for name, params in decls:
        p = params.strip()
        n = 0 if p in ("", "void") else p.count(",") + 1
        assert len(nat.SIGNATURES[name][1]) == n, f"{name}: header {n}, binding {len(nat.SIGNATURES[name][1])}"


def test_error_strings():
    lib = nat.lib()
    assert lib.hck_error_string(0) == b"ok"
    assert b"prime" in lib.hck_error_string(-3)
    assert b"workspace" in lib.hck_error_string(-5)


def test_context_create_rejects_bad_parameters_without_touching_the_gpu():
    lib = nat.lib()
    h = ctypes.c_void_p()
    primes = nat.u64_array([3, 5])
    # log_n other than 16, missing arrays, bad counts: argument errors before any HIP call
    assert lib.hck_context_create(ctypes.byref(h), 15, 1, 1, 1, primes) == -2
    assert lib.hck_context_create(None, 16, 1, 1, 1, primes) == -1
    assert lib.hck_context_create(ctypes.byref(h), 16, 0, 1, 1, primes) == -1
    # a prime >= 2^50, or not 1 mod 2N, or composite: rejected
    assert lib.hck_context_create(ctypes.byref(h), 16, 1, 1, 1, nat.u64_array([(1 << 50) + (1 << 17) + 1, 3])) == -3
    assert lib.hck_context_create(ctypes.byref(h), 16, 1, 1, 1, nat.u64_array([1125899906842597, 1125899906842597])) == -3


def test_null_context_is_an_argument_error():
    lib = nat.lib()
    idx = nat.int_array([0])
    assert lib.hck_ntt_forward(None, None, None, 1, 0, 0, 1, idx, None) == -1
    assert lib.hck_keyswitch_workspace_bytes(None, 1, 1) == 0
    assert lib.hck_automorphism(None, None, None, 1, 0, 0, 1, 5, None) == -1
    assert lib.hck_rescale(None, 2, 1, None, 0, None, 0, None, 0, None) == -1


def test_product_fails_loudly_without_gpu():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    from holmes_amd import fhe

    with pytest.raises(RuntimeError, match="GPU"):
        fhe.generate_client_context(fhe.CKKSContextSpec())


def test_holmes_mac_multi_validates_like_the_sidecar():
    """The sidecar's return codes (bench/cmp/kernels/holmes_mac.cu:363-366): checked before any
    device call, so they need no GPU."""
    lib = nat.lib()
    f = lib.holmes_mac_multi
    args = lambda inputs=1, nb=1, groups=1, ti=10108: (None, None, None, 0, nb, inputs, None, 0, groups, ti, 1,  # noqa: E731
                                                         None, None, None, None)
    assert f(*args(inputs=0)) == -1 and f(*args(inputs=33)) == -1
    assert f(*args(nb=0)) == -2
    assert f(*args(groups=0)) == -3 and f(*args(groups=17)) == -3 and f(*args(groups=9)) == -3
    assert f(*args(ti=8)) == -4 and f(*args(ti=10109)) == -4
    assert f(*args(groups=9, ti=10116)) == -1  # valid selector, null buffers: an argument error
