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
  InsufficientVramException  AIHost/AIHost/ICompute/InsufficientVramException.cs:10-29

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

    def write(self, data, byte_offset=0):
        a = np.ascontiguousarray(data)
        if byte_offset + a.nbytes > self.size:
            raise ValueError("write of %d bytes at %d exceeds buffer of %d" % (a.nbytes, byte_offset, self.size))
        nat.check(nat.lib().aih_memcpy_h2d(self.device.handle, self._ptr + byte_offset,
                                           a.ctypes.data, a.nbytes), "aih_memcpy_h2d")

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

    def synchronize(self):
        nat.check(nat.lib().aih_sync(self.handle), "aih_sync")

    def get_memory_info(self):
        i = self.info()
        return DeviceMemoryInfo(i.total_bytes, i.free_bytes, i.total_bytes - i.free_bytes, i.tracked_bytes)

    def dispose(self):
        if self.handle:
            nat.lib().aih_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()


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
    """The quantized-weight operators of AIHost's ComputeOps on the HIP device."""

    def __init__(self, device):
        self.device = device

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
