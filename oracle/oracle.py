"""ctypes wrapper over the CPU oracle (oracle/oracle.c).

TEST INFRASTRUCTURE ONLY.  The oracle is the checker for the HIP library: it is
imported by tests/, by the smoke check and by the CPU-baseline leg of bench.py,
never by the library itself.  See oracle.h for the reference file:line each
function restates.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

F32, Q4_0, Q8_0, Q4_K, Q6_K = 0, 2, 8, 12, 14
F16_IEEE, F16_REFCPU = 0, 1
BLOCK_ELEMS = {Q8_0: 32, Q4_0: 32, Q4_K: 256, Q6_K: 256}
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, Q4_K: 144, Q6_K: 210}

_lib = None


def build():
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        i64, vp, fp, dp = ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p
        L.orc_f16_refcpu.restype = ctypes.c_float
        L.orc_f16_refcpu.argtypes = [ctypes.c_uint16]
        L.orc_f16_glsl.restype = ctypes.c_float
        L.orc_f16_glsl.argtypes = [ctypes.c_uint16]
        L.orc_f16_decode_array.argtypes = [vp, fp, i64, ctypes.c_int]
        L.orc_get_scale_min_k4.argtypes = [ctypes.c_int, vp, vp, vp]
        L.orc_row_bytes.restype = i64
        L.orc_row_bytes.argtypes = [ctypes.c_int, i64]
        L.orc_dequantize.argtypes = [ctypes.c_int, vp, fp, i64, ctypes.c_int]
        L.orc_matvec.argtypes = [ctypes.c_int, vp, i64, i64, fp, i64, i64, fp, i64,
                                 ctypes.c_int, ctypes.c_int]
        L.orc_matvec_f64.argtypes = [ctypes.c_int, vp, i64, i64, fp, i64, i64, dp, i64,
                                     ctypes.c_int, ctypes.c_int]
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def f16_decode(h, mode):
    """Decode an array of fp16 bit patterns (uint16) to float32 with the oracle."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_decode_array(_ptr(h), _ptr(out), int(h.size), int(mode))
    return out


def get_scale_min_k4(j, scales12):
    s = np.ascontiguousarray(scales12, dtype=np.uint8)
    sc, mn = ctypes.c_uint8(), ctypes.c_uint8()
    lib().orc_get_scale_min_k4(int(j), _ptr(s), ctypes.byref(sc), ctypes.byref(mn))
    return sc.value, mn.value


def row_bytes(qtype, k):
    return int(lib().orc_row_bytes(int(qtype), int(k)))


def dequantize(qtype, data, n, mode=F16_IEEE):
    data = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty(int(n), dtype=np.float32)
    rc = lib().orc_dequantize(int(qtype), _ptr(data), _ptr(out), int(n), int(mode))
    if rc != 0:
        raise ValueError("oracle dequantize rejected type=%d n=%d" % (qtype, n))
    return out


def matvec(qtype, w, n_rows, k, x, mode=F16_IEEE, nthreads=1, f64=False):
    """Y[b, n] = sum_k X[b, k] * W[n, k] for X of shape [batch, k]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    batch = x.shape[0]
    assert x.shape[1] == k
    y = np.empty((batch, int(n_rows)), dtype=np.float64 if f64 else np.float32)
    fn = lib().orc_matvec_f64 if f64 else lib().orc_matvec
    rc = fn(int(qtype), _ptr(w), int(n_rows), int(k), _ptr(x), int(k), int(batch),
            _ptr(y), int(n_rows), int(mode), int(nthreads))
    if rc != 0:
        raise ValueError("oracle matvec rejected the arguments")
    return y
