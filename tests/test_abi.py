"""CPU: the C ABI library loads and exports every entry point
include/dmx_radix.h declares, with the bindings' signatures; calls that
need no GPU behave; the product path never reaches the oracle and fails
loudly when its library is missing."""

import ast
import ctypes as ct
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dmx_radix.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dmx_\w+)\s*\(", text)))


def test_header_declares_the_bound_entry_points():
    from drinkme_amd import _native

    assert _declared() == sorted(_native.SIGNATURES)


def test_library_exports_every_declared_symbol():
    from drinkme_amd import _native

    L = ct.CDLL(_native.LIB)
    for name in _declared():
        assert hasattr(L, name), name
    assert _native.lib().dmx_abi_version() == 1


def test_oracle_library_exports():
    from oracle import radix_oracle as O

    L = O.lib()
    for name in ("orc_palette", "orc_plan", "orc_encode", "orc_decode", "orc_padded_decode", "orc_schedule",
                 "orc_gemv_f64", "orc_gemv_f32"):
        assert hasattr(L, name)


def test_calls_that_need_no_gpu():
    from drinkme_amd import _native

    L = _native.lib()
    assert L.dmx_radix_set_policy(1) in (0, 1)
    assert L.dmx_radix_set_policy(2) == 1
    assert L.dmx_radix_set_policy(0) == 2
    assert L.dmx_radix_set_policy(7) < 0
    err = _native.error_buffer()
    w = np.array([3, 8], np.uint32)
    # a bad op code is refused by name, as radix_native refuses one
    st = L.dmx_radix_native(9, None, 1, 1, 1, 1, 7, 8, w.ctypes.data, 2, None, None, None, 0, 0, 0, None, err,
                            len(err))
    assert st != 0 and err.value
    # a NULL tensor descriptor is refused before any device call
    st = L.dmx_radix_gemv(None, None, 0, 1, None, 0, None, 0, None, err, len(err))
    assert st != 0 and b"tensor" in err.value


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from drinkme_amd import _native

    monkeypatch.setattr(_native, "LIB", str(tmp_path / "missing.so"))
    monkeypatch.setattr(_native, "_lib", None)
    with pytest.raises(ImportError, match="not built"):
        _native.lib()


def test_product_modules_never_import_the_oracle():
    pkg = os.path.join(ROOT, "drinkme_amd")
    for name in os.listdir(pkg):
        if not name.endswith(".py"):
            continue
        tree = ast.parse(open(os.path.join(pkg, name)).read())
        for node in ast.walk(tree):
            if isinstance(node, ast.Import):
                assert not any(a.name.split(".")[0] == "oracle" for a in node.names), name
            if isinstance(node, ast.ImportFrom):
                assert (node.module or "").split(".")[0] != "oracle", name
    for name in os.listdir(os.path.join(pkg, "csrc")):
        assert "radix_oracle" not in open(os.path.join(pkg, "csrc", name)).read(), name
