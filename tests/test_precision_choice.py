"""Why the GEMM tiles hold fp16 and not bf16 (CPU-only numerics check).

The product Y = X W^T at K = 4096 is computed in fp64 from operands rounded
to each 16-bit format, and compared with the fp64 product of the fp32
operands.  The normwise error with bf16 operands (8-bit significand) exceeds
the 1e-3 bound the path is held to; with fp16 operands (11-bit significand)
it is well inside.  The weights are the oracle's dequantization of Q4_K
blocks from N(0, 0.02) values, as in the prefill workload.
"""
import numpy as np

from aihost_amd import _native as nat
from aihost_amd import compute as C

TOL = 1e-3


def round_bf16(a):
    """Round float32 to the nearest bfloat16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def normwise(y, ref):
    return float(np.linalg.norm(y - ref) / np.linalg.norm(ref))


def test_bf16_operands_exceed_tolerance_fp16_do_not(orc):
    n, k, m = 256, 4096, 8
    wq = C.quantize(nat.Q4_K, C.fill_normal(42, n * k, 0.0, 0.02), n, k)
    w = orc.dequantize(nat.Q4_K, wq, n * k).reshape(n, k).astype(np.float64)
    x = C.fill_normal(43, m * k, 0.0, 1.0).reshape(m, k).astype(np.float64)
    ref = x @ w.T

    bf = round_bf16(x.astype(np.float32)).astype(np.float64) @ round_bf16(w.astype(np.float32)).astype(np.float64).T
    hf = x.astype(np.float16).astype(np.float64) @ w.astype(np.float16).astype(np.float64).T
    e_bf, e_hf = normwise(bf, ref), normwise(hf, ref)
    print("normwise error: bf16 operands %.3g, fp16 operands %.3g" % (e_bf, e_hf))
    assert e_bf > TOL
    assert e_hf < TOL / 2


def test_bf16_rounding_helper():
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: ties to even -> 1
    v = np.array([1.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -2.5], dtype=np.float32)
    assert np.array_equal(round_bf16(v), np.array([1.0, 1.0, 1.0 + 2.0 ** -6, -2.5], dtype=np.float32))
