"""The C-ABI library loads and exports every symbol declared in include/*.h (CPU only)."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "bytes_amd", "libbytes_amd.so")


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?\w+\**\s+\**(bytes_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_header_declares_entry_points():
    names = _declared()
    assert "bytes_decode_attn_bf16" in names and "bytes_error_string" in names


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} not built (run python -m bytes_amd.build)")
    h = ctypes.CDLL(LIB)
    missing = [n for n in sorted(_declared()) if not hasattr(h, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_signatures_cover_header():
    from bytes_amd._lib import SIGNATURES
    missing = sorted(_declared() - set(SIGNATURES))
    assert not missing, f"no ctypes signature for {missing}"


def test_abi_version_and_error_string():
    h = ctypes.CDLL(LIB)
    assert h.bytes_abi_version() == 1
    h.bytes_error_string.restype = ctypes.c_char_p
    assert h.bytes_error_string(0)


def test_no_gpu_fallback_when_library_missing(monkeypatch):
    import bytes_amd._lib as L
    monkeypatch.setattr(L, "_lib", None)
    monkeypatch.setattr(L, "LIB_PATH", "/nonexistent/libbytes_amd.so")
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        L.lib()
