"""The C-ABI library loads and exports every entry point ``include/t2w.h`` declares (no GPU calls)."""

import os
import re

import t2w_amd  # noqa: F401
from t2w_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "t2w.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(t2w_\w+)\s*\(", text)))


def test_header_declares_the_bound_symbols():
    assert set(declared()) == set(_lib.exported_symbols())


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    missing = [n for n in declared() if not hasattr(L, n)]
    assert not missing, missing
    assert L.t2w_abi_version() == 1
