"""Expose this backend under the module names Holmes' operators import.

llama3fhe imports ``from easyfhe import fhe`` (llama3fhe/operators/linear/operator.py:9) and uses
the tensor shim ``easyfhe.{from_numpy, empty, zeros, stack, cat, uint64, cuda, get_device_module}``
(llama3fhe/backend.py:1-60).  ``install()`` registers ``easyfhe``, ``easyfhe.fhe`` and
``easyfhe.cuda`` in ``sys.modules`` so that unchanged operator code binds to ``holmes_amd.fhe``
(HIP kernels) and PyTorch-ROCm tensors.  Nothing is installed on disk.
"""

from __future__ import annotations

import sys
import types


def install(force: bool = False) -> types.ModuleType:
    """Register the alias modules; returns the ``easyfhe`` module.  An existing, different
    ``easyfhe`` module is left alone unless ``force``."""

    import torch

    from . import fhe

    existing = sys.modules.get("easyfhe")
    if existing is not None and not force and getattr(existing, "__holmes_amd__", False) is False:
        raise RuntimeError("a different 'easyfhe' module is already imported; pass force=True to replace it")
    mod = types.ModuleType("easyfhe")
    mod.__holmes_amd__ = True
    mod.fhe = fhe
    mod.cuda = torch.cuda
    mod.from_numpy = torch.from_numpy
    mod.empty = torch.empty
    mod.zeros = torch.zeros
    mod.stack = torch.stack
    mod.cat = torch.cat
    mod.uint64 = torch.uint64
    mod.get_device_module = lambda device=None: torch.cuda
    sys.modules["easyfhe"] = mod
    sys.modules["easyfhe.fhe"] = fhe
    sys.modules["easyfhe.cuda"] = torch.cuda
    return mod


def uninstall() -> None:
    mod = sys.modules.get("easyfhe")
    if mod is not None and getattr(mod, "__holmes_amd__", False):
        for name in ("easyfhe", "easyfhe.fhe", "easyfhe.cuda"):
            sys.modules.pop(name, None)
