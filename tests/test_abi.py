"""The C-ABI library loads and exports exactly what include/aihost_hip.h
declares; argument checking that needs no GPU."""
import ctypes
import os
import re
import subprocess

import pytest

from aihost_amd import _native as nat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "aihost_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aih_[a-z0-9_]+)\s*\(", text)))


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", nat.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    return sorted({ln.split()[-1] for ln in out.splitlines() if " T aih_" in ln})


def test_every_declared_symbol_is_exported():
    d, e = declared(), exported()
    assert len(d) >= 20
    assert set(d) <= set(e), set(d) - set(e)


def test_no_undeclared_exports():
    assert set(exported()) <= set(declared())


def test_binding_covers_header():
    assert set(nat.SIGNATURES) == set(declared())
    L = nat.lib()
    for name in declared():
        assert getattr(L, name) is not None


def test_abi_version_and_strerror():
    L = nat.lib()
    assert L.aih_abi_version() == 1
    for code in (0, -1, -2, -3, -4, -5, -6, 2, -99):
        s = nat.strerror(code)
        assert isinstance(s, str) and s
    assert "double free" in nat.strerror(nat.AIH_E_NOT_ALLOCATED)


def test_row_bytes():
    L = nat.lib()
    assert L.aih_row_bytes(nat.Q4_K, 4096) == 2304
    assert L.aih_row_bytes(nat.Q6_K, 14336) == 11760
    assert L.aih_row_bytes(nat.Q8_0, 4096) == 4352
    assert L.aih_row_bytes(nat.Q4_0, 14336) == 8064
    assert L.aih_row_bytes(nat.Q4_K, 100) == nat.AIH_E_INVALID
    assert L.aih_row_bytes(3, 4096) == nat.AIH_E_UNSUPPORTED  # Q4_1: not on this path


def test_null_context_is_rejected():
    L = nat.lib()
    assert L.aih_qmatvec(None, nat.Q4_K, None, 1, 256, None, 256, None, 1, 1) == nat.AIH_E_INVALID
    assert L.aih_qgemm(None, nat.Q4_K, None, 1, 256, None, 16, None) == nat.AIH_E_INVALID
    assert L.aih_dequantize(None, nat.Q4_K, None, None, 256, 0) == nat.AIH_E_INVALID
    assert L.aih_malloc(None, 16, ctypes.byref(ctypes.c_void_p())) == nat.AIH_E_INVALID
    assert L.aih_free(None, None) == nat.AIH_E_INVALID
    assert L.aih_sync(None) == nat.AIH_E_INVALID
    assert L.aih_destroy(None) == nat.AIH_E_INVALID
    assert L.aih_stream(None) is None
    assert L.aih_init(0, None) == nat.AIH_E_INVALID


def test_host_utils_reject_bad_arguments():
    L = nat.lib()
    assert L.aih_host_quantize(nat.Q4_K, None, None, 1, 256) == nat.AIH_E_INVALID
    assert L.aih_host_quantize(nat.F32, None, None, 1, 256) == nat.AIH_E_UNSUPPORTED
    assert L.aih_host_quantize(nat.Q4_K, None, None, 0, 256) == nat.AIH_OK
    assert L.aih_host_fill_normal(1, 0.0, 1.0, None, 4) == nat.AIH_E_INVALID


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(nat, "_lib", None)
    monkeypatch.setattr(nat, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(OSError):
        nat.lib()
