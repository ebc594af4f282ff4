"""CPU checks of the drop-in boundary: the native libraries load and export
every entry point the public headers declare (no GPU calls)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = {
    "einsum_ir_hip.h": os.path.join(ROOT, "einsum_ir_amd", "libeinsum_ir_hip.so"),
    "einsum_ir.h": os.path.join(ROOT, "einsum_ir_amd", "libeinsum_ir.so"),
}


def declared_functions(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(etir_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header", sorted(HEADERS))
def test_library_exports_every_declared_symbol(header):
    lib = ctypes.CDLL(HEADERS[header])
    names = declared_functions(header)
    assert len(names) >= 10, f"only {len(names)} declarations found in {header}"
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"{HEADERS[header]} lacks {missing}"


def test_package_loads_native_library():
    import einsum_ir_amd as eir
    lib = eir.hip_lib()
    assert lib.etir_hip_last_error() is not None


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    import einsum_ir_amd._lib as L
    monkeypatch.setattr(L, "LIB_HIP_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(L, "_lib_hip", None)
    with pytest.raises(ImportError):
        L.hip_lib()
