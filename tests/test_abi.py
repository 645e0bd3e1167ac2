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
    for code in (0, -1, -2, -3, -4, -5, -6, -7, 2, -99):
        s = nat.strerror(code)
        assert isinstance(s, str) and s
    assert "double free" in nat.strerror(nat.AIH_E_NOT_ALLOCATED)
    assert "AIH_NOALLOC_SCRATCH_BYTES" in nat.strerror(nat.AIH_E_SCRATCH)
    assert nat.strerror(-99) == "unknown aihost_hip status"


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
    assert L.aih_matmul_weights_q_noalloc(None, nat.Q4_K, None, 1, 256, None, 16, None) == nat.AIH_E_INVALID
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


# TransformerBase.MapType (TransformerBase.cs:558-575), written out by name:
# GGUFTensorType ids (GGUFValueType.cs:26-56) and the DataType members
# (IComputeBuffer.cs:57-75) in their declaration order.
DATATYPE_ORDER = ["F32", "F16", "Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0", "Q8_1", "Q2_K", "Q3_K", "Q4_K", "Q5_K",
                  "Q6_K", "Q8_K", "I8", "I16", "I32"]
GGUF_IDS = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q8_1": 9, "Q2_K": 10,
            "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "Q8_K": 15}


def test_datatype_mapping_is_maptype():
    L = nat.lib()
    for name, gid in GGUF_IDS.items():
        dt = DATATYPE_ORDER.index(name)
        assert L.aih_datatype_from_type(gid) == dt, name
        assert L.aih_type_from_datatype(dt) == gid, name
    # MapType throws for every other GGUF type; DataType I8/I16/I32 have no GGUF tensor type here
    for gid in [4, 5] + list(range(16, 40)) + [-1]:
        assert L.aih_datatype_from_type(gid) == nat.AIH_E_UNSUPPORTED, gid
    for dt in (14, 15, 16, 17, -1):
        assert L.aih_type_from_datatype(dt) == nat.AIH_E_UNSUPPORTED, dt


def test_reference_datatypes_reach_the_right_format():
    # The ordinals a reference Tensor carries for this path's formats are
    # ggml ids of other formats (8 = Q8_0 but DataType Q2_K; 12 = Q4_K but
    # DataType Q6_K).  Through the mapping they select the right block
    # geometry: a Q6_K row is never sized (and so never read) as Q4_K.
    from aihost_amd import compute as C
    L = nat.lib()
    assert [C.DataType.Q4_0, C.DataType.Q8_0, C.DataType.Q4_K, C.DataType.Q6_K] == [2, 6, 10, 12]
    for dt, gid, rb in ((C.DataType.Q8_0, nat.Q8_0, 272), (C.DataType.Q4_K, nat.Q4_K, 144),
                        (C.DataType.Q6_K, nat.Q6_K, 210), (C.DataType.Q4_0, nat.Q4_0, 144)):
        assert L.aih_type_from_datatype(int(dt)) == gid
        assert C.row_bytes(dt, 256) == rb
        assert C.gguf_type(dt) == gid
        assert C.map_type(gid) == dt
    assert L.aih_row_bytes(int(C.DataType.Q6_K), 256) == 144   # the raw ordinal would be read as Q4_K
    with pytest.raises(NotImplementedError):
        C.gguf_type(C.DataType.I8)
    with pytest.raises(NotImplementedError):
        C.map_type(23)   # IQ4_XS
