"""CPU checks of the C ABI: the library loads and exports every entry point
declared in include/walsh.h, with the ctypes table in sync (no GPU calls)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "walsh.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(walsh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "walsh_hadamard_linear_fwd" in names and "walsh_last_error" in names


def test_library_exports_every_declared_symbol():
    from src.model import _hip
    if not os.path.exists(_hip.LIB_PATH):
        pytest.skip("libwalsh_hip.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_hip.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_table_matches_header():
    from src.model import _hip
    assert sorted(_hip.SIGNATURES) == declared_functions()


def test_identity_calls_need_no_gpu():
    from src.model import _hip
    if not os.path.exists(_hip.LIB_PATH):
        pytest.skip("libwalsh_hip.so not built")
    L = _hip.lib()
    assert L.walsh_abi_version() == 1
    assert L.walsh_device_arch() == b"gfx950"


def declared_arities():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(walsh_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_ctypes_arity_matches_header():
    from src.model import _hip
    ar = declared_arities()
    bad = {n: (ar[n], len(a)) for n, (_, a) in _hip.SIGNATURES.items() if ar.get(n) != len(a)}
    assert not bad, bad
