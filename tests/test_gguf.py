"""GGUF upload path: header / metadata / tensor-table parsing, alignment of
the data section, zero-copy tensor views, and (on the GPU) verbatim upload of
packed blocks through aih_upload_tensor with a matvec on the uploaded weight.

The files are synthetic GGUF v3 files written by aihost_amd.gguf.write_gguf;
the reference holds no GGUF fixture for the formats on this path (its model
test needs an absent TinyLlama file).
"""
import os
import struct

import numpy as np
import pytest

from aihost_amd import _native as nat
from aihost_amd import compute as C
from aihost_amd import gguf


def _tensors():
    rng = np.random.default_rng(3)
    q4k = C.quantize(nat.Q4_K, C.fill_normal(1, 64 * 512, 0.0, 0.02), 64, 512)
    q6k = C.quantize(nat.Q6_K, C.fill_normal(2, 16 * 256, 0.0, 0.02), 16, 256)
    q80 = C.quantize(nat.Q8_0, C.fill_normal(3, 5 * 96, 0.0, 0.02), 5, 96)
    q40 = C.quantize(nat.Q4_0, C.fill_normal(4, 3 * 64, 0.0, 0.02), 3, 64)
    f32 = rng.standard_normal(4096).astype(np.float32)
    return [
        ("blk.0.ffn_up.weight", (512, 64), nat.Q4_K, q4k.tobytes()),
        ("output.weight", (256, 16), nat.Q6_K, q6k.tobytes()),
        ("blk.0.attn_q.weight", (96, 5), nat.Q8_0, q80.tobytes()),
        ("token_embd.weight", (64, 3), nat.Q4_0, q40.tobytes()),
        ("output_norm.weight", (4096,), 0, f32.tobytes()),
    ]


META = {
    "general.architecture": (gguf.STRING, "llama"),
    "llama.context_length": (gguf.U32, 4096),
    "llama.rope.freq_base": (gguf.F32V, 10000.0),
    "llama.attention.layer_norm_rms_epsilon": (gguf.F32V, 1e-5),
    "general.file_type": (gguf.U32, 15),
    "tokenizer.ggml.tokens": (gguf.ARRAY, (gguf.STRING, ["<s>", "</s>", "a"])),
    "tokenizer.ggml.scores": (gguf.ARRAY, (gguf.F32V, [0.0, -1.5, 2.25])),
    "test.flag": (gguf.BOOL, True),
    "test.i64": (gguf.I64, -(1 << 40)),
}


@pytest.mark.parametrize("alignment", [None, 64, 4096])
def test_round_trip(tmp_path, alignment):
    tens = _tensors()
    path = str(tmp_path / "m.gguf")
    gguf.write_gguf(path, tens, META, alignment=alignment)
    with gguf.GGUFReader(path) as r:
        assert r.version == 3
        assert r.alignment == (alignment or 32)
        assert r.data_offset % r.alignment == 0
        assert r.metadata["general.architecture"] == "llama"
        assert r.metadata["llama.context_length"] == 4096
        assert r.metadata["tokenizer.ggml.tokens"] == ["<s>", "</s>", "a"]
        assert r.metadata["tokenizer.ggml.scores"] == [0.0, -1.5, 2.25]
        assert r.metadata["test.flag"] is True and r.metadata["test.i64"] == -(1 << 40)
        assert [t.name for t in r.tensors] == [t[0] for t in tens]
        for (name, dims, ttype, data), info in zip(tens, r.tensors):
            assert info.dims == dims and info.type == ttype
            assert info.offset % r.alignment == 0
            assert info.nbytes == len(data)
            assert r.tensor_bytes(name).tobytes() == data


def test_header_layout_is_little_endian_gguf_v3(tmp_path):
    path = str(tmp_path / "h.gguf")
    gguf.write_gguf(path, _tensors()[:1], {"general.architecture": (gguf.STRING, "llama")})
    raw = open(path, "rb").read(24)
    magic, version, nt, nkv = struct.unpack("<IIQQ", raw)
    assert raw[:4] == b"GGUF" and magic == gguf.MAGIC
    assert (version, nt, nkv) == (3, 1, 1)


def test_sizes_follow_the_ggml_block_table():
    assert gguf.tensor_nbytes(nat.Q4_K, (4096, 14336)) == 14336 * 2304
    assert gguf.tensor_nbytes(nat.Q6_K, (14336, 4096)) == 4096 * 11760
    assert gguf.tensor_nbytes(nat.Q8_0, (4096, 4096)) == 4096 * 4352
    assert gguf.tensor_nbytes(nat.Q4_0, (4096, 14336)) == 14336 * 2304
    assert gguf.tensor_nbytes(10, (256,)) == 84   # Q2_K (the reference's table says 82)
    for t in (nat.Q4_0, nat.Q8_0, nat.Q4_K, nat.Q6_K):
        assert gguf.tensor_nbytes(t, (1024, 3)) == 3 * C.row_bytes(t, 1024)
    with pytest.raises(ValueError):
        gguf.tensor_nbytes(nat.Q4_K, (100, 2))


def test_rejects_bad_files(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGML" + b"\0" * 60)
    with pytest.raises(ValueError):
        gguf.GGUFReader(str(p))
    good = str(tmp_path / "g.gguf")
    gguf.write_gguf(good, _tensors())
    raw = open(good, "rb").read()
    (tmp_path / "t.gguf").write_bytes(raw[:len(raw) // 2])      # truncated data section
    with pytest.raises(ValueError):
        gguf.GGUFReader(str(tmp_path / "t.gguf"))
    with pytest.raises(ValueError):
        gguf.write_gguf(str(tmp_path / "x.gguf"), [("w", (256, 2), nat.Q4_K, b"\0" * 10)])


@pytest.mark.gpu
def test_upload_verbatim_and_matvec(device, orc, tmp_path):
    tens = _tensors()
    path = str(tmp_path / "m.gguf")
    gguf.write_gguf(path, tens, META, alignment=64)
    with gguf.GGUFReader(path) as r:
        bufs = {}
        try:
            for name, dims, ttype, data in tens:
                bufs[name] = gguf.load_tensor(device, r, name)
                got = bufs[name].read_range(0, len(data), np.uint8)
                assert got.tobytes() == data, name
            # the uploaded Q4_K weight feeds the fused matvec directly
            name, (k, n), ttype, data = tens[0]
            x = C.fill_normal(5, 2 * k, 0.0, 1.0).reshape(2, k)
            xb = device.create_buffer(x.nbytes)
            yb = device.create_buffer(2 * n * 4)
            xb.write(x)
            nat.check(nat.lib().aih_qmatvec(device.handle, ttype, bufs[name].get_pointer(), n, k,
                                            xb.get_pointer(), k, yb.get_pointer(), n, 2), "qmatvec")
            y = yb.read_range(0, 2 * n, np.float32).reshape(2, n)
            ref = orc.matvec(ttype, np.frombuffer(data, np.uint8), n, k, x)
            assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-3
            xb.dispose()
            yb.dispose()
        finally:
            for b in bufs.values():
                b.dispose()
