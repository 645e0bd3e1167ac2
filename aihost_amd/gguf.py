"""GGUF files: read the header, metadata and tensor table, and upload packed
tensors verbatim into device memory.

Mirrors the reference's reader and loader for the upload path:
  - GGUFReader.Load / ReadHeader / ReadMetadata / ReadTensorInfo
    (AIHost/AIHost/GGUF/GGUFReader.cs:31-99): little-endian header
    (magic "GGUF", version, tensor count, metadata count), typed key/value
    metadata, then per tensor (name, n_dims, dims[], ggml type, offset);
  - the data section starts at the end of the tensor table rounded up to the
    alignment.  The reference always rounds to 32 (GGUFReader.cs:49); here
    the file's `general.alignment` is honoured, 32 when absent;
  - LazyGGUFModel.LoadTensor (AIHost/AIHost/GGUF/LazyGGUFModel.cs:140-177)
    reads a tensor's bytes into a host array and copies them into the buffer's
    pointer with a host memcpy, which is wrong for device memory.  Here the
    file is memory-mapped and the packed blocks go to HBM through
    aih_upload_tensor (pinned, double-buffered staging), byte for byte in
    their on-disk layout: the kernels read that layout directly.

write_gguf() produces files in the same format for tests and benchmarks.
"""
import mmap
import os
import struct

import numpy as np

from . import _native as nat

MAGIC = 0x46554747   # "GGUF" little endian
DEFAULT_ALIGNMENT = 32

# metadata value types (GGUFValueType.cs:6-20)
U8, I8, U16, I16, U32, I32, F32V, BOOL, STRING, ARRAY, U64, I64, F64V = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32V: "<f", BOOL: "<B",
           U64: "<Q", I64: "<q", F64V: "<d"}

# ggml tensor types: (elements per block, bytes per block) (GGUF definition;
# the reference's GGUFTensorInfo.SizeInBytes, GGUFTensorInfo.cs:51-78, has the
# same values except Q2_K, which it lists as 82 bytes instead of 84)
TYPE_SIZES = {
    0: (1, 4),       # F32
    1: (1, 2),       # F16
    2: (32, 18),     # Q4_0
    3: (32, 20),     # Q4_1
    6: (32, 22),     # Q5_0
    7: (32, 24),     # Q5_1
    8: (32, 34),     # Q8_0
    9: (32, 36),     # Q8_1
    10: (256, 84),   # Q2_K
    11: (256, 110),  # Q3_K
    12: (256, 144),  # Q4_K
    13: (256, 176),  # Q5_K
    14: (256, 210),  # Q6_K
    15: (256, 292),  # Q8_K
    24: (1, 1),      # I8
    25: (1, 2),      # I16
    26: (1, 4),      # I32
    27: (1, 8),      # I64
    28: (1, 8),      # F64
    30: (1, 2),      # BF16
}


def tensor_nbytes(ggml_type, dims):
    """Bytes of a tensor of `ggml_type` with GGUF dims (ne0 innermost)."""
    if ggml_type not in TYPE_SIZES:
        raise NotImplementedError("ggml type %d has no size entry" % ggml_type)
    qk, bb = TYPE_SIZES[ggml_type]
    n = 1
    for d in dims:
        n *= int(d)
    if dims and int(dims[0]) % qk:
        raise ValueError("ne0 = %d is not a whole number of %d-element blocks" % (dims[0], qk))
    return n // qk * bb


class TensorInfo:
    __slots__ = ("name", "dims", "type", "offset", "nbytes")

    def __init__(self, name, dims, ggml_type, offset):
        self.name, self.dims, self.type, self.offset = name, tuple(dims), ggml_type, offset
        self.nbytes = tensor_nbytes(ggml_type, dims)

    def __repr__(self):
        return "TensorInfo(%r, dims=%s, type=%d, offset=%d, nbytes=%d)" % (
            self.name, self.dims, self.type, self.offset, self.nbytes)


class GGUFReader:
    """Parsed GGUF file with the data section memory-mapped (read only)."""

    def __init__(self, path):
        self.path = path
        self._f = open(path, "rb")
        try:
            self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        except ValueError:          # empty file
            self._f.close()
            raise
        self._pos = 0
        magic, self.version = self._unpack("<II")
        if magic != MAGIC:
            self.close()
            raise ValueError("not a GGUF file: magic 0x%08X" % magic)
        if self.version not in (2, 3):
            self.close()
            raise ValueError("unsupported GGUF version %d" % self.version)
        n_tensors, n_kv = self._unpack("<QQ")
        self.metadata = {}
        for _ in range(n_kv):
            key = self._string()
            (vtype,) = self._unpack("<I")
            self.metadata[key] = self._value(vtype)
        self.tensors = []
        for _ in range(n_tensors):
            name = self._string()
            (nd,) = self._unpack("<I")
            dims = self._unpack("<%dQ" % nd) if nd else ()
            ttype, offset = self._unpack("<IQ")
            self.tensors.append(TensorInfo(name, dims, ttype, offset))
        self.alignment = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            self.close()
            raise ValueError("general.alignment %d is not a power of two" % self.alignment)
        self.data_offset = (self._pos + self.alignment - 1) // self.alignment * self.alignment
        for t in self.tensors:
            if self.data_offset + t.offset + t.nbytes > len(self._mm):
                self.close()
                raise ValueError("tensor %r runs past the end of the file" % t.name)
        self._by_name = {t.name: t for t in self.tensors}

    # -- parsing helpers
    def _unpack(self, fmt):
        size = struct.calcsize(fmt)
        if self._pos + size > len(self._mm):
            raise ValueError("truncated GGUF file")
        vals = struct.unpack_from(fmt, self._mm, self._pos)
        self._pos += size
        return vals

    def _string(self):
        (n,) = self._unpack("<Q")
        if self._pos + n > len(self._mm):
            raise ValueError("truncated GGUF file")
        s = bytes(self._mm[self._pos:self._pos + n]).decode("utf-8")
        self._pos += n
        return s

    def _value(self, vtype):
        if vtype in _SCALAR:
            (v,) = self._unpack(_SCALAR[vtype])
            return bool(v) if vtype == BOOL else v
        if vtype == STRING:
            return self._string()
        if vtype == ARRAY:
            etype, n = self._unpack("<IQ")
            return [self._value(etype) for _ in range(n)]
        raise ValueError("unknown metadata value type %d" % vtype)

    # -- access
    def tensor(self, name):
        try:
            return self._by_name[name]
        except KeyError:
            raise KeyError("tensor %r not found in %s" % (name, self.path)) from None

    def tensor_bytes(self, name):
        """Zero-copy uint8 view of a tensor's packed bytes in the mapped file."""
        t = self.tensor(name)
        return np.frombuffer(self._mm, dtype=np.uint8, count=t.nbytes, offset=self.data_offset + t.offset)

    def close(self):
        if getattr(self, "_mm", None) is not None:
            try:
                self._mm.close()
            except BufferError:      # a view is still alive; the mapping goes with it
                pass
            self._mm = None
        if getattr(self, "_f", None) is not None:
            self._f.close()
            self._f = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def load_tensor(device, reader, name):
    """Upload one tensor's packed blocks verbatim into a new device buffer.

    The source is the memory-mapped file itself; aih_upload_tensor stages it
    through pinned memory.  Returns a HipComputeBuffer of exactly nbytes."""
    from .compute import HipComputeBuffer  # noqa: F401  (type of the result)
    t = reader.tensor(name)
    buf = device.create_buffer(max(t.nbytes, 16))
    if t.nbytes:
        view = reader.tensor_bytes(name)
        st = nat.lib().aih_upload_tensor(device.handle, buf.get_pointer(), view.ctypes.data, t.nbytes)
        del view
        nat.check(st, "aih_upload_tensor(%s)" % name)
    return buf


def write_gguf(path, tensors, metadata=None, alignment=None, version=3):
    """Write a GGUF file.

    tensors: list of (name, dims, ggml_type, data) with dims in GGUF order
    (ne0 first) and data a bytes-like object of tensor_nbytes(type, dims).
    metadata: dict key -> (value_type, value); arrays as (ARRAY, (elem_type, list)).
    alignment: written as general.alignment when given (default layout: 32)."""
    meta = dict(metadata or {})
    if alignment is not None:
        meta["general.alignment"] = (U32, int(alignment))
    align = int(alignment or DEFAULT_ALIGNMENT)

    def enc_string(s):
        b = s.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    def enc_value(vtype, v):
        if vtype in _SCALAR:
            return struct.pack(_SCALAR[vtype], int(v) if vtype == BOOL else v)
        if vtype == STRING:
            return enc_string(v)
        if vtype == ARRAY:
            etype, items = v
            return struct.pack("<IQ", etype, len(items)) + b"".join(enc_value(etype, x) for x in items)
        raise ValueError("unknown metadata value type %d" % vtype)

    out = bytearray(struct.pack("<IIQQ", MAGIC, version, len(tensors), len(meta)))
    for k, (vt, v) in meta.items():
        out += enc_string(k) + struct.pack("<I", vt) + enc_value(vt, v)
    offsets, off = [], 0
    for name, dims, ttype, data in tensors:
        nb = tensor_nbytes(ttype, dims)
        if len(data) != nb:
            raise ValueError("tensor %r: %d bytes given, %d expected" % (name, len(data), nb))
        offsets.append(off)
        off = (off + nb + align - 1) // align * align
    for (name, dims, ttype, _), o in zip(tensors, offsets):
        out += enc_string(name) + struct.pack("<I", len(dims)) + struct.pack("<%dQ" % len(dims), *dims)
        out += struct.pack("<IQ", ttype, o)
    pad = (-len(out)) % align
    out += b"\0" * pad
    base = len(out)
    with open(path, "wb") as f:
        f.write(out)
        for (name, dims, ttype, data), o in zip(tensors, offsets):
            f.seek(base + o)
            f.write(bytes(data))
        end = base + off
        if f.tell() < end:
            f.seek(end - 1)
            f.write(b"\0")
    return path


if os.name != "posix":  # pragma: no cover
    raise ImportError("aihost_amd.gguf needs POSIX mmap")
