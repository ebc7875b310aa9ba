"""The C-ABI library loads without a GPU and exports every entry point include/*.h declares;
its host-side tables equal the reference's ROM text and table image.  CPU only."""
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols(prefix="cm_", header=None):
    names = set()
    inc = os.path.join(ROOT, "include")
    for f in os.listdir(inc):
        if f.endswith(".h") and (header is None or f == header):
            text = open(os.path.join(inc, f)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(" + prefix + r"\w+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    from cormorant_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libcormo_hip.so is not built (run __graft_entry__.build())")
    return _lib.lib()


def test_every_declared_symbol_is_exported(lib):
    from cormorant_amd import _lib
    syms = declared_symbols()
    assert len(syms) >= 10
    for s in syms:
        assert hasattr(lib, s), s
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"


def test_abi_version(lib):
    assert lib.cm_abi_version() == 100


def test_host_act_tables_equal_the_oracle_and_rom(lib, oracle_lib):
    from cormorant_amd import units
    for act in (4, 5, 6):
        np.testing.assert_array_equal(units.host_act_table(act), oracle_lib.act_table(act))


def test_host_rowops_image_equals_tables_hex(lib):
    from cormorant_amd import units
    from golden_io import load
    np.testing.assert_array_equal(units.host_rowops_table_image(), load("rowops")["tables"])


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from cormorant_amd import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(_lib.HipLibraryMissing):
        _lib.lib()


def test_every_declared_host_symbol_is_exported():
    """libcormo_host.so exports every cmh_ entry point include/cormorant_host.h declares."""
    from cormorant_amd import host_ops
    syms = declared_symbols("cmh_", "cormorant_host.h")
    assert len(syms) >= 9
    lib = host_ops.host_lib()
    for s in syms:
        assert hasattr(lib, s), s
        assert s in host_ops.HOST_SIGNATURES, f"{s} has no ctypes signature"
    assert lib.cmh_abi_version() == 100
