"""The C-ABI library loads and exports every symbol include/*.h declares
(no compute calls: this runs without a GPU)."""
import ctypes
import os
import re

import pytest

from oxionnx_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    inc = os.path.join(ROOT, "include")
    for fn in os.listdir(inc):
        if fn.endswith(".h"):
            text = open(os.path.join(inc, fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(ohip_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "ohip_gemm" in names and "ohip_qconv2d" in names and len(names) >= 30


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert set(declared_symbols()) == set(L.SIGNATURES)


def test_device_free_entry_points():
    lib = L.lib()
    assert lib.ohip_version().startswith(b"oxionnx-hip")
    assert lib.ohip_conv_out_dim(128, 1, 1, 3, 1, 1) == 128
    assert lib.ohip_conv_out_dim(2, 0, 0, 5, 1, 1) == -1
    n = ctypes.c_int(-1)
    assert lib.ohip_device_count(ctypes.byref(n)) == 0 and n.value >= 0
    h = ctypes.c_void_p()
    if n.value == 0:
        assert lib.ohip_ctx_create(0, ctypes.byref(h)) == L.E_NODEVICE
        assert b"no HIP device" in lib.ohip_last_error()


def test_env_flag_truthiness(monkeypatch):
    lib = L.lib()
    for v, want in [("1", 1), ("true", 1), ("please", 1), ("", 0), ("0", 0), (" FALSE ", 0), ("no", 0),
                    ("Off", 0)]:
        monkeypatch.setenv("OHIP_TEST_FLAG", v)
        assert lib.ohip_env_flag(b"OHIP_TEST_FLAG") == want, v
    monkeypatch.delenv("OHIP_TEST_FLAG")
    assert lib.ohip_env_flag(b"OHIP_TEST_FLAG") == 0
