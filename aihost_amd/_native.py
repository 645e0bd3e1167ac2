"""ctypes binding of libaihost_hip.so (include/aihost_hip.h).

This module plays the part of the reference's P/Invoke declarations
(AIHost/AIHost/ICompute/ROCm/HipApi.cs:9-188): every exported C function is
declared here with its exact signature.  There is no fallback: if the shared
library has not been built, loading raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_lib", "libaihost_hip.so")

AIH_OK = 0
AIH_E_INVALID = -1
AIH_E_UNSUPPORTED = -2
AIH_E_NOT_GFX950 = -3
AIH_E_NOT_ALLOCATED = -4
AIH_E_LIMIT = -5
AIH_E_NO_DEVICE = -6
AIH_E_SCRATCH = -7
NOALLOC_SCRATCH_BYTES = (16 << 20) + (64 << 10)   # AIH_NOALLOC_SCRATCH_BYTES
HIP_ERROR_OUT_OF_MEMORY = 2

F32, Q4_0, Q8_0, Q4_K, Q6_K = 0, 2, 8, 12, 14
F16_IEEE, F16_REFCPU = 0, 1
PRE_NONE, PRE_RMSNORM, PRE_SILU_MUL, PRE_SILU_PAIRS, PRE_F16_OPERAND = 0, 1, 2, 3, 4
POST_STORE, POST_ACCUMULATE, POST_SILU_PAIRS, POST_SILU_PAIRS_F16 = 0, 1, 2, 3


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
        ("device_index", ctypes.c_int32),
        ("compute_units", ctypes.c_int32),
        ("wavefront_size", ctypes.c_int32),
        ("clock_khz", ctypes.c_int32),
        ("memory_clock_khz", ctypes.c_int32),
        ("memory_bus_width", ctypes.c_int32),
        ("total_bytes", ctypes.c_uint64),
        ("free_bytes", ctypes.c_uint64),
        ("tracked_bytes", ctypes.c_uint64),
        ("tracked_buffers", ctypes.c_int64),
    ]


_vp, _i, _i64, _u64, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_size_t
_f, _fp = ctypes.c_float, ctypes.POINTER(ctypes.c_float)

# name -> (restype, argtypes); the full exported surface of the header
SIGNATURES = {
    "aih_abi_version": (_i, []),
    "aih_init": (_i, [_i, ctypes.POINTER(_vp)]),
    "aih_destroy": (_i, [_vp]),
    "aih_device_info_get": (_i, [_vp, ctypes.POINTER(DeviceInfo)]),
    "aih_malloc": (_i, [_vp, _sz, ctypes.POINTER(_vp)]),
    "aih_free": (_i, [_vp, _vp]),
    "aih_memset": (_i, [_vp, _vp, _i, _sz]),
    "aih_memcpy_h2d": (_i, [_vp, _vp, _vp, _sz]),
    "aih_memcpy_d2h": (_i, [_vp, _vp, _vp, _sz]),
    "aih_memcpy_d2d": (_i, [_vp, _vp, _vp, _sz]),
    "aih_upload_tensor": (_i, [_vp, _vp, _vp, _sz]),
    "aih_row_bytes": (_i64, [_i, _i64]),
    "aih_datatype_from_type": (_i, [_i]),
    "aih_type_from_datatype": (_i, [_i]),
    "aih_dequantize": (_i, [_vp, _i, _vp, _vp, _u64, _i]),
    "aih_qmatvec": (_i, [_vp, _i, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i]),
    "aih_qmatvec_fused": (_i, [_vp, _i, _vp, _i64, _i64, _vp, _vp, _f, _i, _i, _vp]),
    "aih_qgemm": (_i, [_vp, _i, _vp, _i64, _i64, _vp, _i64, _vp]),
    "aih_qgemm_fused": (_i, [_vp, _i, _vp, _i64, _i64, _vp, _vp, _f, _i64, _i, _i, _vp]),
    "aih_matmul_weights_q": (_i, [_vp, _i, _vp, _i64, _i64, _vp, _i64, _vp]),
    "aih_qgemm_qkv_rope": (_i, [_vp, _i, _vp, _i64, _vp, _vp, _f, _i64, _i, _vp, _vp, _vp, ctypes.c_int32,
                                ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _vp, _vp, ctypes.c_int32, _i64]),
    "aih_operand_bytes": (_i64, [_i64, _i64]),
    "aih_qgemm_plan": (_i, [_vp, _i64, _i64, _i64, _i, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)]),
    "aih_matmul_weights_q_noalloc": (_i, [_vp, _i, _vp, _i64, _i64, _vp, _i64, _vp]),
    "aih_probe_stream_read": (_i, [_vp, _vp, _u64, _i, _vp]),
    "aih_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _i64, _i64, _f]),
    "aih_rope_table": (_i, [_vp, _vp, ctypes.c_int32, ctypes.c_int32, _f]),
    "aih_rope": (_i, [_vp, _vp, _i64, _vp, _i64, _i64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _vp, _vp,
                      ctypes.c_int32, _i, _i64]),
    "aih_rope_qkv": (_i, [_vp, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, ctypes.c_int32, ctypes.c_int32,
                          ctypes.c_int32, ctypes.c_int32, _vp, _vp, ctypes.c_int32, _i64]),
    "aih_store_rows": (_i, [_vp, _vp, _i64, _i64, _vp, _i64, ctypes.c_int32, _vp]),
    "aih_silu_mul": (_i, [_vp, _vp, _vp, _vp, _i64]),
    "aih_silu_mul_pairs": (_i, [_vp, _vp, _vp, _i64, _i64]),
    "aih_silu": (_i, [_vp, _vp, _vp, _i64]),
    "aih_mul": (_i, [_vp, _vp, _vp, _vp, _i64]),
    "aih_add": (_i, [_vp, _vp, _vp, _vp, _i64]),
    "aih_attention_scratch_floats": (_i64, [ctypes.c_int32, ctypes.c_int32]),
    "aih_attention": (_i, [_vp, _vp, _vp, _vp, _vp, _i64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                           ctypes.c_int32, _vp, ctypes.c_int32, _f, _vp, _i64]),
    "aih_attention_strided": (_i, [_vp, _vp, _i64, _vp, _vp, _vp, _i64, ctypes.c_int32, ctypes.c_int32,
                                   ctypes.c_int32, ctypes.c_int32, _vp, ctypes.c_int32, _f, _vp, _i64]),
    "aih_attention_operand": (_i, [_vp, _vp, _i64, _vp, _vp, _vp, _i64, ctypes.c_int32, ctypes.c_int32,
                                   ctypes.c_int32, ctypes.c_int32, _vp, ctypes.c_int32, _f]),
    "aih_attention_decode_qkv": (_i, [_vp, _vp, _vp, _vp, _vp, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                      ctypes.c_int32, _vp, _vp, ctypes.c_int32, ctypes.c_int32, _f, _vp, _i64]),
    "aih_embed_q": (_i, [_vp, _i, _vp, _i64, _i64, _vp, _i64, _vp]),
    "aih_argmax": (_i, [_vp, _vp, _i64, _vp, _vp, _vp, _i64, ctypes.c_int32]),
    "aih_sync": (_i, [_vp]),
    "aih_stream": (_vp, [_vp]),
    "aih_capture_begin": (_i, [_vp]),
    "aih_capture_end": (_i, [_vp, ctypes.POINTER(_vp)]),
    "aih_graph_launch": (_i, [_vp, _vp]),
    "aih_graph_destroy": (_i, [_vp]),
    "aih_event_record": (_i, [_vp, _i]),
    "aih_event_elapsed": (_i, [_vp, _i, _i, _fp]),
    "aih_strerror": (ctypes.c_char_p, [_i]),
    "aih_host_fill_normal": (_i, [_u64, _f, _f, _vp, _u64]),
    "aih_host_quantize": (_i, [_i, _vp, _vp, _i64, _i64]),
}

_lib = None


class AihError(RuntimeError):
    """A non-zero status from the library (status code in .status)."""

    def __init__(self, status, what):
        self.status = status
        super().__init__("%s failed: %s (status %d)" % (what, strerror(status), status))


def lib():
    """Load libaihost_hip.so; raises OSError when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError("libaihost_hip.so not built (expected at %s); run aihost_amd/build.py" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def strerror(status):
    return lib().aih_strerror(int(status)).decode()


def operand_bytes(m, k):
    """Bytes of the fp16 GEMM operand image of an m x k activation matrix
    (aih_operand_bytes): what AIH_POST_SILU_PAIRS_F16 and
    aih_attention_operand write and AIH_PRE_F16_OPERAND reads."""
    n = lib().aih_operand_bytes(int(m), int(k))
    if n < 0:
        raise AihError(int(n), "aih_operand_bytes")
    return n


def qgemm_plan(handle, n, k, m, may_split=True):
    """(tile rows, K splits) that the GEMM takes for an m x k by n product on
    the context's device (aih_qgemm_plan)."""
    t, s = ctypes.c_int32(), ctypes.c_int32()
    check(lib().aih_qgemm_plan(handle, int(n), int(k), int(m), int(bool(may_split)), ctypes.byref(t),
                               ctypes.byref(s)), "aih_qgemm_plan")
    return t.value, s.value


def check(status, what):
    if status != AIH_OK:
        raise AihError(status, what)
    return status
