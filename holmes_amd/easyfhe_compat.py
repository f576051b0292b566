"""Expose this backend under the module names Holmes' package imports.

llama3fhe binds its CKKS engine by import: ``from easyfhe import fhe`` in every operator module
(e.g. llama3fhe/operators/linear/operator.py:9), ``import easyfhe as torch`` for the tensor shim
(operators/linear/gpu_packer.py:14), ``import easyfhe.bs.openfhe as bs`` for bootstrapping
(operators/nonlinear/bootstrap.py:18), ``from easyfhe.fhe.ops.layout import cipher_batch_item``
(operators/nonlinear/polynomial.py:294), ``from easyfhe.fhe.ciphertext import CipherState``
(operators/attention/sparse_fused.py:154) and ``easyfhe.multiprocessing``
(parallel/prefill/transport.py:79).  ``install()`` builds that module tree in ``sys.modules``:

    easyfhe                      package; unknown attributes resolve to torch (the tensor shim)
    easyfhe.cuda                 torch.cuda (HIP devices, streams and events on ROCm)
    easyfhe.multiprocessing      torch.multiprocessing
    easyfhe.fhe                  package over holmes_amd.fhe (every fhe.<op> name)
    easyfhe.fhe.ciphertext       Cipher, CipherState
    easyfhe.fhe.constants        MAX_ENCODED_BITS
    easyfhe.fhe.ops              package
    easyfhe.fhe.ops.layout       cipher_batch_item, pack_cipher_batch, unpack_cipher_batch
    easyfhe.bs                   package
    easyfhe.bs.openfhe           holmes_amd.bootstrap (BootstrapSpec, generate, bootstrap, requirements)

The modules are views, not copies: ``easyfhe.fhe.homo_rotate is holmes_amd.fhe.homo_rotate``.
Nothing is written to disk, and ``uninstall()`` removes exactly the names ``install()`` added.
"""

from __future__ import annotations

import sys
import types

_MARK = "__holmes_amd__"
_NAMES = (
    "easyfhe",
    "easyfhe.cuda",
    "easyfhe.multiprocessing",
    "easyfhe.fhe",
    "easyfhe.fhe.ciphertext",
    "easyfhe.fhe.constants",
    "easyfhe.fhe.ops",
    "easyfhe.fhe.ops.layout",
    "easyfhe.bs",
    "easyfhe.bs.openfhe",
)


def _package(name: str, doc: str, fallback=None, **attrs) -> types.ModuleType:
    """A module that imports treat as a package (it has ``__path__``); attributes it does not hold
    are looked up on ``fallback`` (PEP 562 module ``__getattr__``)."""

    mod = types.ModuleType(name, doc)
    mod.__path__ = []
    mod.__package__ = name
    setattr(mod, _MARK, True)
    for key, value in attrs.items():
        setattr(mod, key, value)
    if fallback is not None:
        def __getattr__(attr, _src=fallback, _name=name):
            try:
                return getattr(_src, attr)
            except AttributeError:
                raise AttributeError(f"module {_name!r} has no attribute {attr!r}") from None

        mod.__getattr__ = __getattr__
    return mod


def _tree() -> dict[str, types.ModuleType]:
    import torch
    import torch.multiprocessing

    from . import bootstrap, context, encoding, fhe

    ciphertext = _package("easyfhe.fhe.ciphertext", "Ciphertext types.", Cipher=context.Cipher,
                          CipherState=context.CipherState)
    constants = _package("easyfhe.fhe.constants", "Encoder limits.", MAX_ENCODED_BITS=encoding.MAX_ENCODED_BITS)
    layout = _package("easyfhe.fhe.ops.layout", "Batch layout helpers.", cipher_batch_item=fhe.cipher_batch_item,
                      pack_cipher_batch=fhe.pack_cipher_batch, unpack_cipher_batch=fhe.unpack_cipher_batch)
    ops = _package("easyfhe.fhe.ops", "Operation modules.", layout=layout)
    fhe_pkg = _package("easyfhe.fhe", fhe.__doc__, fallback=fhe, ciphertext=ciphertext, constants=constants, ops=ops)
    openfhe = _package("easyfhe.bs.openfhe", bootstrap.__doc__, fallback=bootstrap)
    bs = _package("easyfhe.bs", "Bootstrapping programs.", openfhe=openfhe)
    root = _package("easyfhe", __doc__, fallback=torch, fhe=fhe_pkg, bs=bs, cuda=torch.cuda,
                    multiprocessing=torch.multiprocessing,
                    get_device_module=lambda device=None: torch.cuda)
    return {
        "easyfhe": root,
        "easyfhe.cuda": torch.cuda,
        "easyfhe.multiprocessing": torch.multiprocessing,
        "easyfhe.fhe": fhe_pkg,
        "easyfhe.fhe.ciphertext": ciphertext,
        "easyfhe.fhe.constants": constants,
        "easyfhe.fhe.ops": ops,
        "easyfhe.fhe.ops.layout": layout,
        "easyfhe.bs": bs,
        "easyfhe.bs.openfhe": openfhe,
    }


def install(force: bool = False) -> types.ModuleType:
    """Register the alias tree and return the ``easyfhe`` package.  A different, already imported
    ``easyfhe`` (a real EasyFHE install) is kept unless ``force``."""

    present = sys.modules.get("easyfhe")
    if present is not None and not getattr(present, _MARK, False) and not force:
        raise RuntimeError("another 'easyfhe' is already imported; install(force=True) replaces it")
    if present is not None:
        uninstall(any_owner=True)
    tree = _tree()
    sys.modules.update(tree)
    return tree["easyfhe"]


def uninstall(any_owner: bool = False) -> None:
    """Remove the alias tree (only names this module registered, unless ``any_owner``)."""

    root = sys.modules.get("easyfhe")
    if root is None or (not any_owner and not getattr(root, _MARK, False)):
        return
    for name in [n for n in sys.modules if n == "easyfhe" or n.startswith("easyfhe.")]:
        sys.modules.pop(name, None)


__all__ = ["install", "uninstall"]
