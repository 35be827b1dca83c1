"""The C-ABI library loads without a GPU and exports every symbol include/*.h declares.

No compute calls here: only loading, symbol lookup and the calls that need no device.
"""
import re
from pathlib import Path

import pytest

from pufferlean_amd import _lib as L

ROOT = Path(__file__).resolve().parent.parent
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_ \*]*?\b(ph_[A-Za-z0-9_]+)\s*\(", re.M)


def declared_symbols():
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(DECL.findall(text))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "ph_vtrace" in names and "ph_gemm" in names
    assert len(names) >= 10


@pytest.mark.parametrize("name", declared_symbols())
def test_library_exports_symbol(name):
    lib = L.lib()
    assert hasattr(lib, name), f"{name} declared in include/ but not exported"


def test_signatures_cover_exports():
    for name in L.SIGNATURES:
        assert name in declared_symbols(), f"{name} bound in _lib but not declared"


def test_no_device_calls_fail_cleanly():
    lib = L.lib()
    assert lib.ph_version() == 100
    n = lib.ph_device_count()
    assert n >= 0
