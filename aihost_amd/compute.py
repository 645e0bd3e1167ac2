"""Host-side mirror of AIHost's compute interfaces for the quantized-matmul path.

Names, argument meaning and error behaviour follow the reference so that code
(and tests) written against it read the same:

  HipComputeDevice   IComputeDevice   AIHost/AIHost/ICompute/IComputeDevice.cs:27-72
  HipComputeBuffer   IComputeBuffer   AIHost/AIHost/ICompute/IComputeBuffer.cs:6-42
  Tensor             Tensor           AIHost/AIHost/Compute/Tensor.cs:8-150
  DataType           DataType         AIHost/AIHost/ICompute/IComputeBuffer.cs:57-75
  map_type           MapType          AIHost/AIHost/Compute/TransformerBase.cs:558-575
  ComputeOps         ComputeOps       AIHost/AIHost/Compute/ComputeOps.cs
      dequantize        Dequantize      :733-745
      dequantize_into   DequantizeInto  :761-861
      matmul_weights    MatMulWeights   :275-309 (quantized weight: fused kernels)
      clone, concat, layer_norm, apply_rope_full, fused_mha_generate,
      multi_head_attention, add, multiply, silu, embedding_lookup,
      embedding_lookup_from_quantized, feed_forward, transformer_layer
                        the reference's operators of the same names, over
                        LibraryKernel (the device's kernel objects)
  KVCache            KVCache          AIHost/AIHost/Inference/InferenceEngine.cs:585-622
  InsufficientVramException  AIHost/AIHost/ICompute/InsufficientVramException.cs:10-29

Type arguments are a DataType (the reference Tensor's numbering) or a ggml /
GGUFTensorType id; a bare int is read as a ggml id, the numbering of the
library's operators (DataType.Q6_K is 12, the ggml id of Q4_K).

Everything runs through libaihost_hip.so; there is no CPU path.
"""
import ctypes
import enum
from dataclasses import dataclass

import numpy as np

from . import _native as nat


class GGUFTensorType(enum.IntEnum):
    """ggml tensor type ids of the GGUF file (GGUFTensorType,
    AIHost/AIHost/GGUF/GGUFValueType.cs:26-56): the type argument of the
    library's operators.  The four block types of this path and F32."""
    F32 = nat.F32
    Q4_0 = nat.Q4_0
    Q8_0 = nat.Q8_0
    Q4_K = nat.Q4_K
    Q6_K = nat.Q6_K


class DataType(enum.IntEnum):
    """The reference Tensor's type (DataType, AIHost/AIHost/ICompute/
    IComputeBuffer.cs:57-75), numbered as its declaration order.  Not the
    ggml numbering: DataType.Q6_K (12) is the ggml id of Q4_K."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 4
    Q5_1 = 5
    Q8_0 = 6
    Q8_1 = 7
    Q2_K = 8
    Q3_K = 9
    Q4_K = 10
    Q5_K = 11
    Q6_K = 12
    Q8_K = 13
    I8 = 14
    I16 = 15
    I32 = 16


def map_type(ggml_type):
    """TransformerBase.MapType (TransformerBase.cs:558-575): GGUF tensor type ->
    DataType, through the library; NotImplementedError where MapType throws
    NotSupportedException."""
    dt = nat.lib().aih_datatype_from_type(int(ggml_type))
    if dt < 0:
        raise NotImplementedError("Unsupported tensor type: %d" % int(ggml_type))
    return DataType(dt)


def gguf_type(dtype):
    """The ggml id the operators take for a type: a DataType is translated
    by the library (aih_type_from_datatype); a GGUFTensorType or a plain int
    is already one."""
    if isinstance(dtype, DataType):
        t = nat.lib().aih_type_from_datatype(int(dtype))
        if t < 0:
            raise NotImplementedError("DataType %s has no GGUF tensor type" % dtype.name)
        return t
    return int(dtype)


def data_type(dtype):
    """A DataType for a DataType or a ggml id (GGUFTensorType or int)."""
    return dtype if isinstance(dtype, DataType) else map_type(dtype)


class InsufficientVramException(MemoryError):
    """Raised when a device allocation fails for lack of memory."""


def row_bytes(dtype, k):
    """GGUFTensorInfo.SizeInBytes of one row of k elements (dtype: a DataType
    or a ggml id)."""
    rb = int(nat.lib().aih_row_bytes(gguf_type(dtype), int(k)))
    if rb < 0:
        raise ValueError("K=%d is not a whole number of %s blocks" % (k, data_type(dtype).name))
    return rb


@dataclass
class DeviceMemoryInfo:
    """IComputeDevice.GetMemoryInfo result (IComputeDevice.cs:6-22)."""
    total_bytes: int
    available_bytes: int
    used_bytes: int
    tracked_allocated_bytes: int
    supports_native_query: bool = True


class HipComputeBuffer:
    """Device memory owned by this object; freed by dispose()."""

    def __init__(self, device, size, element_type=DataType.F32):
        self.device = device
        self.size = int(size)
        self.element_type = data_type(element_type)
        ptr = ctypes.c_void_p()
        st = nat.lib().aih_malloc(device.handle, ctypes.c_size_t(self.size), ctypes.byref(ptr))
        if st == nat.HIP_ERROR_OUT_OF_MEMORY:
            raise InsufficientVramException("cannot allocate %d bytes on %s" % (self.size, device.name))
        nat.check(st, "aih_malloc")
        self._ptr = ptr.value

    def get_pointer(self):
        return self._ptr

    # writes of at most this many bytes keep a host copy: the params structs
    # of the reference's kernels, read back on the host by LibraryKernel
    HOST_COPY_BYTES = 256

    def write(self, data, byte_offset=0):
        a = np.ascontiguousarray(data)
        if byte_offset + a.nbytes > self.size:
            raise ValueError("write of %d bytes at %d exceeds buffer of %d" % (a.nbytes, byte_offset, self.size))
        nat.check(nat.lib().aih_memcpy_h2d(self.device.handle, self._ptr + byte_offset,
                                           a.ctypes.data, a.nbytes), "aih_memcpy_h2d")
        if byte_offset == 0 and a.nbytes <= self.HOST_COPY_BYTES:
            self.host_copy = a.tobytes()

    def read(self, dtype=np.float32):
        return self.read_range(0, self.size // np.dtype(dtype).itemsize, dtype)

    def read_range(self, byte_offset, element_count, dtype=np.float32):
        out = np.empty(int(element_count), dtype=dtype)
        if byte_offset + out.nbytes > self.size:
            raise ValueError("read past the end of the buffer")
        nat.check(nat.lib().aih_memcpy_d2h(self.device.handle, out.ctypes.data,
                                           self._ptr + byte_offset, out.nbytes), "aih_memcpy_d2h")
        return out

    def dispose(self):
        if self._ptr:
            nat.lib().aih_free(self.device.handle, self._ptr)  # Dispose never throws
            self._ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()


class HipComputeDevice:
    """One gfx950 device with one in-order stream."""

    provider_name = "HIP"

    def __init__(self, device_index=0):
        h = ctypes.c_void_p()
        nat.check(nat.lib().aih_init(int(device_index), ctypes.byref(h)), "aih_init")
        self.handle = h.value
        info = self.info()
        self.name = info.name.decode()
        self.arch = info.arch.decode()
        self.api_version = "aihost_hip ABI %d" % nat.lib().aih_abi_version()

    def info(self):
        info = nat.DeviceInfo()
        nat.check(nat.lib().aih_device_info_get(self.handle, ctypes.byref(info)), "aih_device_info_get")
        return info

    def create_buffer(self, size, element_type=DataType.F32, require_device_local=True):
        # HIP allocations are always device-local; require_device_local is accepted for parity.
        return HipComputeBuffer(self, size, element_type)

    def create_kernel(self, source_name, entry_point="main"):
        """IComputeDevice.CreateKernel (IComputeDevice.cs:52) for one of the
        reference's ComputeShaders sources, named by its field: the library
        operation that computes what the shader computes (LibraryKernel).
        NotImplementedError for a source without one."""
        if source_name not in LibraryKernel.OPS:
            raise NotImplementedError("ComputeShaders.%s has no library operation on the HIP device" % source_name)
        return LibraryKernel(self, source_name)

    def rope_table(self, head_dim, theta, rows):
        """A device RoPE table (aih_rope_table) of at least `rows` positions
        for (head_dim, theta), kept and grown by the device; returns
        (pointer, rows held).  A replaced table stays allocated until
        dispose(): work already queued may still read it."""
        key = (int(head_dim), float(np.float32(theta)))
        cur = self._tables.get(key) if hasattr(self, "_tables") else None
        if cur is None or cur[1] < rows:
            n = max(int(rows), 4096, 2 * cur[1] if cur else 0)
            buf = self.create_buffer(n * head_dim * 4)
            nat.check(nat.lib().aih_rope_table(self.handle, buf.get_pointer(), n, int(head_dim), float(theta)),
                      "aih_rope_table")
            self._tables = getattr(self, "_tables", {})
            self._kept = getattr(self, "_kept", []) + [buf]
            self._tables[key] = cur = (buf.get_pointer(), n)
        return cur

    def attention_scratch(self, n_heads, max_len):
        """(pointer, floats) of the device's attention scratch, grown to what
        aih_attention needs for n_heads and max_len (replaced buffers kept
        until dispose())."""
        need = int(nat.lib().aih_attention_scratch_floats(int(n_heads), int(max_len)))
        if need < 0:
            nat.check(need, "aih_attention_scratch_floats")
        cur = getattr(self, "_scratch", None)
        if cur is None or cur[1] < need:
            buf = self.create_buffer(max(16, need * 4))
            self._kept = getattr(self, "_kept", []) + [buf]
            self._scratch = cur = (buf.get_pointer(), need)
        return cur

    def synchronize(self):
        nat.check(nat.lib().aih_sync(self.handle), "aih_sync")

    def get_memory_info(self):
        i = self.info()
        return DeviceMemoryInfo(i.total_bytes, i.free_bytes, i.total_bytes - i.free_bytes, i.tracked_bytes)

    def dispose(self):
        if self.handle:
            for b in getattr(self, "_kept", []):
                b.dispose()
            self._kept, self._tables, self._scratch = [], {}, None
            nat.lib().aih_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()


class LibraryKernel:
    """The kernel object a HIP device returns for one of the reference's GLSL
    sources (IComputeKernel, AIHost/AIHost/ICompute/IComputeKernel.cs:6-34).
    ComputeOps binds buffers by binding index and a params struct in a small
    buffer (read here from that buffer's host copy), exactly as for the
    shader; dispatch runs the library operation over the same buffers:

      Copy              (src, dst, {size})                   aih_memcpy_d2d
      ConcatAxis0       (a, b, out, {rows_a, rows_b, cols})  two aih_memcpy_d2d
      LayerNorm         (x in place, w, {rows, cols, eps})   aih_rmsnorm
      RoPEFull          (x in place, {seqLen, numHeads,      aih_rope over a device
                         headDim, startPosition, theta})     table of (headDim, theta)
      FusedMHAGenerate  (Q, K, V, out, {numQHeads,           aih_attention, one row at
                         numKvHeads, headDim, kvSeqLen,      position kvSeqLen - 1
                         scale})
      ElementWiseAdd    (a, b, c, {size})                    aih_add
      ElementWiseMul    (a, b, c, {size})                    aih_mul
      SiLU              (x in place, {size})                 aih_silu
      EmbeddingLookup   (ids, table, out, {seqLen, dModel})  aih_embed_q (F32 rows)
      DequantizeQ4K/Q6K (q, out, {elementOffset});           aih_dequantize of
                         groups of 256 elements              groups * 256 elements

    Sources (ComputeShaders.cs:12-73) and params layouts: ComputeOps.cs
    :360-416 (element-wise), 419-452 (concat), 493-542 (SiLU, LayerNorm),
    658-677 / 761-861 (dequantization), 959-979 (RoPE), 1015-1043 (attention),
    1780-1800 (embedding), 1893-1915 (copy)."""

    OPS = ("Copy", "ConcatAxis0", "LayerNorm", "RoPEFull", "FusedMHAGenerate", "ElementWiseAdd", "ElementWiseMul",
           "SiLU", "EmbeddingLookup", "DequantizeQ4K", "DequantizeQ6K")

    def __init__(self, device, name):
        self.device, self.name = device, name
        self.args = {}

    def set_argument(self, index, value):
        self.args[int(index)] = value

    def compile(self):
        """Compiled ahead of time into libaihost_hip.so: nothing to do."""

    def _ptr(self, i):
        return self.args[i].get_pointer()

    def _params(self, i, fmt):
        import struct
        return struct.unpack_from("<" + fmt, self.args[i].host_copy)

    def dispatch(self, global_work_size, local_work_size=None):
        L, h, n = nat.lib(), self.device.handle, self.name
        if n == "Copy":
            (size,) = self._params(2, "I")
            nat.check(L.aih_memcpy_d2d(h, self._ptr(1), self._ptr(0), 4 * size), "Copy")
        elif n == "ConcatAxis0":
            ra, rb, cols = self._params(3, "III")
            nat.check(L.aih_memcpy_d2d(h, self._ptr(2), self._ptr(0), 4 * ra * cols), "ConcatAxis0")
            nat.check(L.aih_memcpy_d2d(h, self._ptr(2) + 4 * ra * cols, self._ptr(1), 4 * rb * cols), "ConcatAxis0")
        elif n == "LayerNorm":
            rows, cols, eps = self._params(2, "IIf")
            nat.check(L.aih_rmsnorm(h, self._ptr(0), self._ptr(1), self._ptr(0), rows, cols, eps), "LayerNorm")
        elif n == "RoPEFull":
            seq, heads, hd, start, theta = self._params(1, "IIIIf")
            table, rows = self.device.rope_table(hd, theta, start + seq)
            nat.check(L.aih_rope(h, self._ptr(0), heads * hd, self._ptr(0), heads * hd, seq, heads, hd, start, None,
                                 table, rows, 0, seq), "RoPEFull")
        elif n == "FusedMHAGenerate":
            nh, nkv, hd, kv_len, scale = self._params(4, "IIIIf")
            scratch, floats = self.device.attention_scratch(nh, kv_len)
            nat.check(L.aih_attention(h, self._ptr(0), self._ptr(1), self._ptr(2), self._ptr(3), 1, nh, nkv, hd,
                                      kv_len - 1, None, kv_len, scale, scratch, floats), "FusedMHAGenerate")
        elif n in ("ElementWiseAdd", "ElementWiseMul"):
            (size,) = self._params(3, "I")
            fn = L.aih_add if n == "ElementWiseAdd" else L.aih_mul
            nat.check(fn(h, self._ptr(0), self._ptr(1), self._ptr(2), size), n)
        elif n == "SiLU":
            (size,) = self._params(1, "I")
            nat.check(L.aih_silu(h, self._ptr(0), self._ptr(0), size), "SiLU")
        elif n == "EmbeddingLookup":
            seq, dim = self._params(3, "II")
            vocab = self.args[1].size // (4 * dim)
            nat.check(L.aih_embed_q(h, nat.F32, self._ptr(1), vocab, dim, self._ptr(0), seq, self._ptr(2)),
                      "EmbeddingLookup")
        else:   # DequantizeQ4K / DequantizeQ6K
            qt, bb = (nat.Q4_K, 144) if n == "DequantizeQ4K" else (nat.Q6_K, 210)
            (off,) = self._params(2, "I")
            count = min(256 * int(global_work_size[0]), self.args[1].size // 4 - off)
            nat.check(L.aih_dequantize(h, qt, self._ptr(0) + off // 256 * bb, self._ptr(1) + 4 * off,
                                       ctypes.c_uint64(count), nat.F16_IEEE), n)

    def dispose(self):
        pass


class Tensor:
    """Buffer + shape + DataType (the reference's numbering; a ggml id given
    here is mapped as TransformerBase.MapType does).  Quantized weights use
    GGUF dims [K, N]."""

    def __init__(self, buffer, shape, dtype, name=None):
        self.buffer, self.shape, self.name = buffer, tuple(int(s) for s in shape), name
        self.dtype = data_type(dtype)

    @property
    def total_elements(self):
        n = 1
        for s in self.shape:
            n *= s
        return n

    @staticmethod
    def create(device, shape, dtype=DataType.F32, name=None):
        n = 1
        for s in shape:
            n *= int(s)
        dtype = data_type(dtype)
        if dtype != DataType.F32:
            # Tensor.GetDataTypeSize throws for block types (Tensor.cs:138-149)
            raise NotImplementedError("Tensor.create supports F32 only; wrap quantized buffers instead")
        return Tensor(device.create_buffer(max(4, n * 4), dtype), shape, dtype, name)

    @staticmethod
    def from_data(device, data, shape=None, name=None):
        a = np.ascontiguousarray(data, dtype=np.float32)
        t = Tensor.create(device, shape or a.shape, DataType.F32, name)
        t.buffer.write(a)
        return t

    @staticmethod
    def from_quantized(device, packed, k, n, dtype, name=None):
        """Upload packed GGUF blocks verbatim as a [K, N] weight (row n = K/QK
        blocks); dtype is a DataType or a ggml id."""
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        dtype = data_type(dtype)
        if packed.nbytes != n * row_bytes(dtype, k):
            raise ValueError("packed size %d != N*row_bytes = %d" % (packed.nbytes, n * row_bytes(dtype, k)))
        buf = device.create_buffer(packed.nbytes, dtype)
        nat.check(nat.lib().aih_upload_tensor(device.handle, buf.get_pointer(), packed.ctypes.data,
                                              packed.nbytes), "aih_upload_tensor")
        return Tensor(buf, (k, n), dtype, name)

    def read(self):
        return self.buffer.read_range(0, self.total_elements, np.float32).reshape(self.shape)

    def dispose(self):
        self.buffer.dispose()


class ComputeOps:
    """AIHost's ComputeOps on the HIP device: the quantized-weight operators
    (the fused kernels), and the reference's other operators written as it
    writes them -- params structs, bindings and dispatch sizes of
    ComputeOps.cs -- over the device's kernel objects (LibraryKernel), so that
    a layer runs in the reference's operator order with no GLSL kernel."""

    def __init__(self, device):
        self.device = device
        self._deferred = []     # buffers queued work may still read (the reference's Defer)

    # the params struct of a kernel, as ComputeOps writes it into a small buffer
    def _params(self, fmt, *values):
        import struct
        raw = np.frombuffer(struct.pack("<" + fmt, *values), np.uint8)
        buf = self.device.create_buffer(raw.nbytes, DataType.I32)
        buf.write(raw)
        self._deferred.append(buf)
        return buf

    def _run(self, name, args, groups):
        k = self.device.create_kernel(name)
        for i, a in enumerate(args):
            k.set_argument(i, a)
        k.dispatch([int(groups)])

    def flush(self):
        """Wait for the device, then free the deferred buffers (ComputeOps.Flush)."""
        self.device.synchronize()
        for b in self._deferred:
            b.dispose()
        self._deferred = []

    # ComputeOps.Clone (ComputeOps.cs:1893-1915)
    def clone(self, x, name=None):
        r = Tensor.create(self.device, x.shape, DataType.F32, name)
        n = x.total_elements
        self._run("Copy", [x.buffer, r.buffer, self._params("I", n)], (n + 255) // 256)
        return r

    # ComputeOps.Concat, axis 0 (ComputeOps.cs:419-452): the KV cache append of KVCache.Add
    def concat(self, a, b, axis=1, name=None):
        if axis != 0:
            raise NotImplementedError("only axis 0 (rows) is on the HIP path")
        if a.shape[1] != b.shape[1]:
            raise ValueError("Columns must match for axis=0 concat: %d != %d" % (a.shape[1], b.shape[1]))
        r = Tensor.create(self.device, (a.shape[0] + b.shape[0], a.shape[1]), DataType.F32, name)
        self._run("ConcatAxis0", [a.buffer, b.buffer, r.buffer, self._params("III", a.shape[0], b.shape[0],
                                                                             a.shape[1])],
                  (r.total_elements + 255) // 256)
        return r

    # ComputeOps.LayerNorm (ComputeOps.cs:517-542): RMSNorm of each row, in place
    def layer_norm(self, x, weight, eps=1e-5):
        rows, cols = (x.shape[0], x.shape[1]) if len(x.shape) >= 2 else (1, x.shape[0])
        self._run("LayerNorm", [x.buffer, weight.buffer, self._params("IIf", rows, cols, eps)], rows)

    # ComputeOps.ApplyRoPEFull (ComputeOps.cs:959-979), in place
    def apply_rope_full(self, x, start, n_heads, head_dim, theta=10000.0):
        seq = x.shape[0]
        self._run("RoPEFull", [x.buffer, self._params("IIIIf", seq, n_heads, head_dim, start, theta)],
                  (seq * n_heads * head_dim // 2 + 255) // 256)

    # ComputeOps.FusedMHAGenerate (ComputeOps.cs:1015-1043)
    def fused_mha_generate(self, q, k, v, n_heads, n_kv_heads, head_dim, scale, name=None):
        r = Tensor.create(self.device, (1, n_heads * head_dim), DataType.F32, name)
        self._run("FusedMHAGenerate", [q.buffer, k.buffer, v.buffer, r.buffer,
                                       self._params("IIIIf", n_heads, n_kv_heads, head_dim, k.shape[0], scale)],
                  n_heads)
        return r

    # ComputeOps.MultiHeadAttention (ComputeOps.cs:1055-1102): one row through
    # FusedMHAGenerate; more rows, where the reference loops over heads with
    # SliceCols / Transpose / MatMul / Scale / CausalMask / RowwiseSoftmax /
    # ScatterCols, through one aih_attention call (same causal rule: row i
    # sees keys 0 .. start + i)
    def multi_head_attention(self, q, k, v, n_heads, start=0, name=None):
        seq, dq = q.shape
        head_dim = dq // n_heads
        n_kv = k.shape[1] // head_dim
        scale = float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))
        if seq == 1:
            return self.fused_mha_generate(q, k, v, n_heads, n_kv, head_dim, scale, name)
        r = Tensor.create(self.device, (seq, dq), DataType.F32, name)
        scratch, floats = self.device.attention_scratch(n_heads, k.shape[0])
        nat.check(nat.lib().aih_attention(self.device.handle, q.buffer.get_pointer(), k.buffer.get_pointer(),
                                          v.buffer.get_pointer(), r.buffer.get_pointer(), seq, n_heads, n_kv,
                                          head_dim, int(start), None, k.shape[0], scale, scratch, floats),
                  "MultiHeadAttention")
        return r

    def _elementwise(self, kernel, a, b, name):
        if a.total_elements != b.total_elements:
            raise ValueError("Tensors must have same total elements for element-wise ops")
        r = Tensor.create(self.device, a.shape, DataType.F32, name)
        n = a.total_elements
        self._run(kernel, [a.buffer, b.buffer, r.buffer, self._params("I", n)], (n + 255) // 256)
        return r

    # ComputeOps.Add / Multiply (ComputeOps.cs:389-416, 360-387)
    def add(self, a, b, name=None):
        return self._elementwise("ElementWiseAdd", a, b, name)

    def multiply(self, a, b, name=None):
        return self._elementwise("ElementWiseMul", a, b, name)

    # ComputeOps.SiLU (ComputeOps.cs:493-510), in place
    def silu(self, x):
        n = x.total_elements
        self._run("SiLU", [x.buffer, self._params("I", n)], (n + 255) // 256)

    # ComputeOps.EmbeddingLookup (ComputeOps.cs:1780-1800): table [vocab, dModel] F32
    # (GGUF dims [dModel, vocab])
    def embedding_lookup(self, token_ids, table, name=None):
        ids = np.ascontiguousarray(token_ids, dtype=np.int32)
        d_model = table.shape[0]
        r = Tensor.create(self.device, (ids.size, d_model), DataType.F32, name)
        tok = self.device.create_buffer(max(4, ids.nbytes), DataType.I32)
        tok.write(ids)
        self._deferred.append(tok)
        self._run("EmbeddingLookup", [tok, table.buffer, r.buffer, self._params("II", ids.size, d_model)],
                  (ids.size * d_model + 255) // 256)
        return r

    # ComputeOps.EmbeddingLookupFromQuantized (ComputeOps.cs:1399-1454): below
    # 512 MiB of F32 the whole table is dequantized and looked up; above it
    # only the rows are (the reference on the CPU, here aih_embed_q)
    def embedding_lookup_from_quantized(self, token_ids, qtable, name=None):
        d_model, vocab = qtable.shape
        if d_model * vocab * 4 <= 512 * 1024 * 1024:
            full = self.dequantize(qtable)
            r = self.embedding_lookup(token_ids, full, name)
            self._deferred.append(full.buffer)
            return r
        ids = np.ascontiguousarray(token_ids, dtype=np.int32)
        r = Tensor.create(self.device, (ids.size, d_model), DataType.F32, name)
        tok = self.device.create_buffer(max(4, ids.nbytes), DataType.I32)
        tok.write(ids)
        self._deferred.append(tok)
        nat.check(nat.lib().aih_embed_q(self.device.handle, gguf_type(qtable.dtype), qtable.buffer.get_pointer(),
                                        vocab, d_model, tok.get_pointer(), ids.size, r.buffer.get_pointer()),
                  "EmbeddingLookupFromQuantized")
        return r

    # ComputeOps.FeedForward (ComputeOps.cs:1218-1241)
    def feed_forward(self, x, w_gate, w_up, w_down, name=None):
        gate = self.matmul_weights(x, w_gate, "ffn_gate")
        self.silu(gate)
        up = self.matmul_weights(x, w_up, "ffn_up")
        gu = self.multiply(gate, up, "ffn_gate_up")
        out = self.matmul_weights(gu, w_down, name or "ffn_output")
        self._deferred += [gate.buffer, up.buffer, gu.buffer]
        return out

    # ComputeOps.TransformerLayer (ComputeOps.cs:1250-1356), with the KV cache
    # of InferenceEngine (KVCache below)
    def transformer_layer(self, x, attn_norm, wq, wk, wv, wo, ffn_norm, w_gate, w_up, w_down, n_heads, position,
                          kv_cache=None, layer=0, eps=1e-5, name=None):
        head_dim = x.shape[1] // n_heads
        xn = self.clone(x, "attn_norm_input")
        self.layer_norm(xn, attn_norm, eps)
        q = self.matmul_weights(xn, wq, "Q")
        k = self.matmul_weights(xn, wk, "K")
        v = self.matmul_weights(xn, wv, "V")
        n_kv = k.shape[1] // head_dim
        self.apply_rope_full(q, position, n_heads, head_dim)
        self.apply_rope_full(k, position, n_kv, head_dim)
        if kv_cache is not None:
            kv_cache.add(layer, k, v)
            kc, vc = kv_cache.get(layer)
            att = self.multi_head_attention(q, kc, vc, n_heads, position, "attn_out")
        else:
            att = self.multi_head_attention(q, k, v, n_heads, position, "attn_out")
            self._deferred += [k.buffer, v.buffer]
        proj = self.matmul_weights(att, wo, "attn_proj")
        x1 = self.add(x, proj, "x_after_attn")
        x1n = self.clone(x1, "ffn_norm_input")
        self.layer_norm(x1n, ffn_norm, eps)
        ffn = self.feed_forward(x1n, w_gate, w_up, w_down, "ffn_out")
        out = self.add(x1, ffn, name or "layer_output")
        self._deferred += [xn.buffer, q.buffer, att.buffer, proj.buffer, x1.buffer, x1n.buffer, ffn.buffer]
        return out

    # ComputeOps.Dequantize (ComputeOps.cs:733-745)
    def dequantize(self, quantized, f16_mode=nat.F16_IEEE, name=None):
        if quantized.dtype == DataType.F32:
            return quantized
        result = Tensor.create(self.device, quantized.shape, DataType.F32, name)
        self.dequantize_into(quantized, result, f16_mode)
        return result

    # ComputeOps.DequantizeInto (ComputeOps.cs:761-861)
    def dequantize_into(self, quantized, target, f16_mode=nat.F16_IEEE):
        if target.dtype != DataType.F32:
            raise ValueError("Target must be F32")
        if quantized.dtype == DataType.F32:
            raise NotImplementedError("DequantizeInto not supported for F32")
        if target.total_elements < quantized.total_elements:
            raise ValueError("target too small")
        nat.check(nat.lib().aih_dequantize(self.device.handle, gguf_type(quantized.dtype),
                                           quantized.buffer.get_pointer(), target.buffer.get_pointer(),
                                           ctypes.c_uint64(quantized.total_elements), int(f16_mode)),
                  "aih_dequantize")

    # ComputeOps.MatMulWeights (ComputeOps.cs:275-309): A [M, K] x W (GGUF [K, N]) -> C [M, N]
    def matmul_weights(self, a, b, name=None):
        if len(a.shape) != 2 or len(b.shape) != 2:
            raise ValueError("MatMulWeights requires 2D tensors")
        m, k = a.shape
        kb, n = b.shape
        if k != kb:
            raise ValueError("Incompatible shapes for MatMulWeights: [%dx%d] x [%dx%d]" % (m, k, kb, n))
        if b.dtype == DataType.F32:
            raise NotImplementedError("F32 weights are not on the HIP quantized path")
        result = Tensor.create(self.device, (m, n), DataType.F32, name)
        nat.check(nat.lib().aih_matmul_weights_q(self.device.handle, gguf_type(b.dtype), b.buffer.get_pointer(),
                                                 n, k, a.buffer.get_pointer(), m, result.buffer.get_pointer()),
                  "aih_matmul_weights_q")
        return result


class KVCache:
    """InferenceEngine's KV cache (InferenceEngine.cs:585-622): the first add
    of a layer takes the K and V tensors, later ones concatenate rows
    (ComputeOps.Concat, axis 0)."""

    def __init__(self, ops):
        self.ops = ops
        self.cache = {}
        self.sequence_length = 0

    def add(self, layer, key, value):
        if layer not in self.cache:
            self.cache[layer] = (key, value)
        else:
            k0, v0 = self.cache[layer]
            nk = self.ops.concat(k0, key, 0, "kv_cache_k_layer%d" % layer)
            nv = self.ops.concat(v0, value, 0, "kv_cache_v_layer%d" % layer)
            self.ops._deferred += [k0.buffer, v0.buffer, key.buffer, value.buffer]
            self.cache[layer] = (nk, nv)
        self.sequence_length = self.cache[layer][0].shape[0]

    def get(self, layer):
        return self.cache.get(layer, (None, None))

    def dispose(self):
        for k, v in self.cache.values():
            k.dispose()
            v.dispose()
        self.cache = {}


def fill_normal(seed, n, mean=0.0, std=1.0):
    """Deterministic N(mean, std) float32 samples (splitmix64 + Box-Muller)."""
    out = np.empty(int(n), dtype=np.float32)
    nat.check(nat.lib().aih_host_fill_normal(ctypes.c_uint64(seed), float(mean), float(std),
                                             out.ctypes.data, ctypes.c_uint64(out.size)), "aih_host_fill_normal")
    return out


def quantize(dtype, values, n_rows, k):
    """Quantize n_rows x k float32 values into packed GGUF blocks (uint8);
    dtype is a DataType or a ggml id."""
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    if v.size != n_rows * k:
        raise ValueError("expected %d values" % (n_rows * k))
    out = np.empty(int(n_rows) * row_bytes(dtype, k), dtype=np.uint8)
    nat.check(nat.lib().aih_host_quantize(gguf_type(dtype), v.ctypes.data, out.ctypes.data, int(n_rows), int(k)),
              "aih_host_quantize")
    return out
