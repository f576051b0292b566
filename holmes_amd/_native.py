"""ctypes binding of libholmes_ckks.so (C ABI declared in include/holmes_ckks.h).

The product path has exactly one implementation: the HIP kernels behind this library.  If the
library is missing or no GPU is visible, every operation raises -- there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libholmes_ckks.so"

HCK_ERR_ARG = -1
HCK_ERR_WORKSPACE = -5
HCK_ERR_SCRATCH = -6
HCK_NOALLOC_SCRATCH_BYTES = 128 << 20   # include/holmes_ckks.h: the array behind hck_rotate_noalloc

HCK_OP_ADD = 0
HCK_OP_SUB = 1
HCK_OP_MUL = 2
HCK_OP_NEG = 3
HCK_OP_MUL_SCALAR = 4
HCK_OP_MUL_XHALF = 5
HCK_OP_MAC = 6
HCK_OP_ADD_SCALAR = 7

# Every symbol include/holmes_ckks.h declares, with (restype, argtypes).
_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_u32 = ctypes.c_uint32
_sz = ctypes.c_size_t
_ip = ctypes.POINTER(ctypes.c_int)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_u32p = ctypes.POINTER(ctypes.c_uint32)

SIGNATURES = {
    "hck_context_create": (_i, [ctypes.POINTER(_vp), _i, _i, _i, _i, _u64p]),
    "hck_context_destroy": (None, [_vp]),
    "hck_context_info": (_i, [_vp, _ip, _ip, _ip, _ip]),
    "hck_context_twiddles": (_i, [_vp, _i, _i, _u64p]),
    "hck_context_root_tables": (_i, [_vp, _vp, _vp]),
    "hck_error_string": (ctypes.c_char_p, [_i]),
    "hck_context_set_conv_engine": (_i, [_vp, _i]),
    "hck_ntt_forward": (_i, [_vp, _vp, _vp, _i, _i64, _i64, _i, _ip, _vp]),
    "hck_ntt_inverse": (_i, [_vp, _vp, _vp, _i, _i64, _i64, _i, _ip, _vp]),
    "hck_automorphism": (_i, [_vp, _vp, _vp, _i, _i64, _i64, _i, _u32, _vp]),
    "hck_keyswitch_workspace_bytes": (_sz, [_vp, _i, _i]),
    "hck_keyswitch": (_i, [_vp, _i, _i, _vp, _i64, ctypes.POINTER(_vp), _vp, _i64, _vp, _vp, _i64, _vp, _sz, _vp]),
    "hck_rotate_workspace_bytes": (_sz, [_vp, _i, _i]),
    "hck_rotate": (_i, [_vp, _i, _i, _u32, _vp, _vp, _i64, ctypes.POINTER(_vp), _vp, _vp, _i64, _vp, _vp, _i64,
                        _vp, _sz, _vp]),
    "hck_rotate_rescale_workspace_bytes": (_sz, [_vp, _i, _i]),
    "hck_rotate_rescale": (_i, [_vp, _i, _i, _u32, _vp, _vp, _i64, ctypes.POINTER(_vp), _vp, _vp, _i64, _vp, _sz,
                                _vp]),
    "hck_rescale_workspace_bytes": (_sz, [_vp, _i, _i]),
    "hck_rescale": (_i, [_vp, _i, _i, _vp, _i64, _vp, _i64, _vp, _sz, _vp]),
    "hck_poly_op": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i64, _i64, _i64, _i, _ip, _u64p, _vp]),
    "hck_poly_from_signed": (_i, [_vp, _vp, _vp, _i, _i64, _i64, _i, _ip, _vp]),
    "hck_bsgs_mac": (_i, [_vp, _i, _ip, _i, _i, _i, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _i64, _vp, _i64, _vp,
                          _vp]),
    "holmes_mac_multi": (_i, [_vp, _vp, _vp, ctypes.c_longlong, _i, _i, _vp, ctypes.c_longlong, _i, _i, _i, _vp, _vp,
                              _vp, _vp]),
    "hck_rotate_noalloc": (_i, [_vp, _i, _i, _u32, _vp, _vp, _i64, ctypes.POINTER(_vp), _vp, _vp, _i64, _vp, _vp,
                                _i64, _vp]),
    "hck_rotate_noalloc_limit": (_sz, [_vp, _i]),
    "hck_rotate_ext": (_i, [_vp, _i, _i, _u32, _vp, _vp, _i64, ctypes.POINTER(_vp), _vp, _vp, _i64, _vp, _vp, _i64,
                            _vp, _sz, _vp]),
    "hck_rotate_many": (_i, [_vp, _i, _i, _u32p, _vp, _vp, _i64, ctypes.POINTER(_vp), _vp, _vp, _i64, _vp, _vp,
                             _i64, _vp, _sz, _vp]),
    "hck_rotate_ext_many": (_i, [_vp, _i, _i, _u32p, _vp, _vp, _i64, ctypes.POINTER(_vp), _vp, _vp, _i64, _vp, _vp,
                                 _i64, _vp, _sz, _vp]),
    "hck_rotate_ext_sum": (_i, [_vp, _i, _i, _i, _u32p, _vp, _vp, _i64, ctypes.POINTER(_vp), _vp, _vp, _i64, _vp,
                                _vp, _i64, _vp, _sz, _vp]),
    "hck_rotate_hoist_digits_bytes": (_sz, [_vp, _i, _i]),
    "hck_rotate_hoist_workspace_bytes": (_sz, [_vp, _i, _i, _i]),
    "hck_rotate_hoist_prepare": (_i, [_vp, _i, _i, _vp, _i64, _vp, _vp, _sz, _vp]),
    "hck_rotate_hoisted": (_i, [_vp, _i, _i, _i, _u32p, _vp, _vp, _i64, _vp, ctypes.POINTER(_vp), _vp, _vp, _i64, _vp,
                                _sz, _vp]),
    "hck_moddown_workspace_bytes": (_sz, [_vp, _i, _i]),
    "hck_moddown": (_i, [_vp, _i, _i, _vp, _i64, _vp, _i64, _vp, _sz, _vp]),
    "hck_pack_diagonals": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp]),
    "hck_encode_workspace_bytes": (_sz, [_vp, _i]),
    "hck_encode": (_i, [_vp, _vp, _vp, _i, ctypes.c_double, _i, _ip, _vp, _i64, _vp, _sz, _vp, _vp]),
    "hck_tensor": (_i, [_vp, _i, _i, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp]),
    "hck_relinearize_workspace_bytes": (_sz, [_vp, _i, _i]),
    "hck_relinearize": (_i, [_vp, _i, _i, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _sz, _vp]),
    "hck_mul_relin_workspace_bytes": (_sz, [_vp, _i, _i]),
    "hck_mul_relin": (_i, [_vp, _i, _i, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _sz, _vp]),
    "hck_mul_relin_rescale_workspace_bytes": (_sz, [_vp, _i, _i]),
    "hck_mul_relin_rescale": (_i, [_vp, _i, _i, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _sz, _vp]),
    "hck_mul_relin_rescale_postop": (_i, [_vp, _i, _i, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _i, _vp, _vp, _i64, _u64p,
                                          _vp, _vp, _i64, _vp, _sz, _vp]),
    "hck_weighted_sum": (_i, [_vp, _i, _i, _i, _vp, _i64, _vp, _vp, _i64, _vp]),
    "hck_lincomb": (_i, [_vp, _i, _i, _i, ctypes.POINTER(_vp), _vp, ctypes.POINTER(_vp), _vp]),
    "hck_lincomb_rescale_workspace_bytes": (_sz, [_vp, _i, _i]),
    "hck_lincomb_rescale": (_i, [_vp, _i, _i, _i, ctypes.POINTER(_vp), _vp, ctypes.POINTER(_vp), _u64p,
                                 ctypes.c_uint64, _vp, _sz, _vp]),
    "hck_modraise_workspace_bytes": (_sz, [_vp, _i, _i]),
    "hck_modraise": (_i, [_vp, _i, _i, _vp, _i64, _vp, _i64, _vp, _sz, _vp]),
    # the reference sidecar's encode entry (argtypes of bench/cmp/holmes_fast_stage2.py:37)
    "holmes_encode_stage2": (_i, [_vp, _vp, ctypes.c_longlong, _i, ctypes.c_double, _i, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _vp, _i, _i, _i]),
}

_lib = None


class NativeError(RuntimeError):
    """A non-zero return code from libholmes_ckks."""


def lib():
    """Load libholmes_ckks.so; raise if it has not been built."""

    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build the HIP extension first "
            "(python -m holmes_amd.build); there is no CPU fallback"
        )
    handle = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    _lib = handle
    return handle


def check(rc: int, what: str) -> None:
    if int(rc) != 0:
        msg = lib().hck_error_string(int(rc))
        raise NativeError(f"{what} failed: {msg.decode() if msg else rc} (code {int(rc)})")


def int_array(values) -> ctypes.Array:
    values = [int(v) for v in values]
    return (ctypes.c_int * max(1, len(values)))(*values)


def u64_array(values) -> ctypes.Array:
    values = [int(v) for v in values]
    return (ctypes.c_uint64 * max(1, len(values)))(*values)


def u32_array(values) -> ctypes.Array:
    values = [int(v) for v in values]
    return (ctypes.c_uint32 * max(1, len(values)))(*values)


def ptr_array(ptrs) -> ctypes.Array:
    ptrs = [int(p) for p in ptrs]
    return (ctypes.c_void_p * max(1, len(ptrs)))(*ptrs)
