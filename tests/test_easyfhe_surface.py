"""After ``easyfhe_compat.install()`` every ``easyfhe`` import and attribute the reference package
uses resolves (the list in tests/golden/easyfhe_surface.json was built by a text search of
llama3fhe/, tests/golden/make_easyfhe_surface.py), and binds to this backend."""

import importlib
import json
from pathlib import Path

import pytest

SURFACE = json.loads((Path(__file__).parent / "golden" / "easyfhe_surface.json").read_text())


@pytest.fixture
def easyfhe():
    from holmes_amd import easyfhe_compat

    mod = easyfhe_compat.install()
    try:
        yield mod
    finally:
        easyfhe_compat.uninstall()


def _resolve(root, dotted: str):
    obj = root
    for part in dotted.split("."):
        obj = getattr(obj, part)
    return obj


def test_every_import_statement_resolves(easyfhe):
    assert SURFACE["modules"] and SURFACE["from_imports"]
    for name in SURFACE["modules"]:
        assert importlib.import_module(name) is not None, name
    for mod, name in SURFACE["from_imports"]:
        m = importlib.import_module(mod)
        assert getattr(m, name) is not None, f"from {mod} import {name}"
    # the statement forms the reference writes
    exec("import easyfhe.bs.openfhe as bs\nfrom easyfhe.fhe.ops.layout import cipher_batch_item\n"
         "from easyfhe.fhe.ciphertext import CipherState\nfrom easyfhe import fhe\nimport easyfhe as torch", {})


def test_every_dotted_attribute_resolves(easyfhe):
    for dotted in SURFACE["dotted"]:
        assert _resolve(easyfhe, dotted.split(".", 1)[1]) is not None, dotted
    for name in SURFACE["fhe_attributes"]:
        assert getattr(easyfhe.fhe, name) is not None, f"fhe.{name}"
    for name in SURFACE["bs_attributes"]:
        if name != "openfhe":
            assert getattr(easyfhe.bs.openfhe, name) is not None, f"bs.{name}"
    for name in SURFACE["shim_attributes"]:
        assert _resolve(easyfhe, name) is not None, f"torch shim {name}"


def test_aliases_are_this_backend(easyfhe):
    import torch

    from holmes_amd import bootstrap, context, fhe

    import easyfhe.bs.openfhe as bs  # noqa: E402
    from easyfhe.fhe.ciphertext import Cipher, CipherState
    from easyfhe.fhe.ops.layout import cipher_batch_item

    assert easyfhe.fhe.homo_rotate is fhe.homo_rotate and easyfhe.fhe.hoisted_mac_sum is fhe.hoisted_mac_sum
    assert bs.BootstrapSpec is bootstrap.BootstrapSpec and bs.generate is bootstrap.generate
    assert Cipher is context.Cipher and CipherState is context.CipherState
    assert cipher_batch_item is fhe.cipher_batch_item
    assert easyfhe.uint64 is torch.uint64 and easyfhe.cuda is torch.cuda
    assert easyfhe.fhe.constants.MAX_ENCODED_BITS == 61
    with pytest.raises(AttributeError):
        easyfhe.fhe.no_such_operation


def test_reference_bootstrap_call_forms(easyfhe):
    """The spec keywords and requirement call of llama3fhe/operators/nonlinear/bootstrap.py:119-160,
    296-348 (strategy "double_hoist", dim1, baby_step, output_levels, a tuple of specs)."""

    import easyfhe.bs.openfhe as bs

    spec = bs.BootstrapSpec(log_slots=15, level_budget=(3, 3), output_levels=0, strategy="double_hoist",
                            mode="modraise_first", dim1=None, baby_step=None)
    req = bs.requirements((spec,), log_n=16)
    assert req.rotations and (1 << 17) - 1 in req.rotations
    with pytest.raises(ValueError):
        bs.requirements((bs.BootstrapSpec(strategy="no_such_strategy"),), log_n=16)


def test_install_refuses_a_foreign_easyfhe_and_uninstall_is_exact():
    import sys
    import types

    from holmes_amd import easyfhe_compat

    foreign = types.ModuleType("easyfhe")
    sys.modules["easyfhe"] = foreign
    try:
        with pytest.raises(RuntimeError):
            easyfhe_compat.install()
        easyfhe_compat.uninstall()
        assert sys.modules["easyfhe"] is foreign
    finally:
        sys.modules.pop("easyfhe", None)
    easyfhe_compat.install()
    easyfhe_compat.install()  # idempotent
    easyfhe_compat.uninstall()
    assert not [n for n in sys.modules if n == "easyfhe" or n.startswith("easyfhe.")]
