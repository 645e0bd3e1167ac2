"""Pins the oracle's weight matmul (ComputeShaders.cs:93-129 semantics,
sequential fp32 accumulation as TransformerBase.cs:454-456).

* orientation: an integer Q8_0 weight W[n, k] = f(n, k) with d = 1 gives
  exactly sum_k x[k] * f(n, k) (small integers: every sum is exact), and basis
  vectors pick out columns -- a transposed operand or wrong row stride fails;
* accuracy: fp32 result within 1e-6 normwise of an fp64 brute force over the
  independently dequantized weights;
* order: equals a left-to-right fp32 running sum (np.cumsum in float32).
"""
import numpy as np

import ggml_ref as G


def q8_from_ints(ints):
    """Pack an integer matrix (|v| <= 127) as Q8_0 with d = 1.0."""
    n, k = ints.shape
    blocks = np.zeros((n, k // 32, 34), dtype=np.uint8)
    blocks[:, :, 0], blocks[:, :, 1] = 0x00, 0x3C
    blocks[:, :, 2:] = ints.reshape(n, k // 32, 32).astype(np.int8).view(np.uint8)
    return blocks.reshape(-1)


def test_orientation_integer_weights(orc):
    n, k = 48, 96
    nn, kk = np.meshgrid(np.arange(n), np.arange(k), indexing="ij")
    ints = ((nn * 7 + kk * 3) % 11) - 5
    w = q8_from_ints(ints)
    x = np.arange(k, dtype=np.float32) % 5 - 2
    y = orc.matvec(orc.Q8_0, w, n, k, x)
    assert np.array_equal(y[0], (ints @ x.astype(np.int64)).astype(np.float32))
    for col in (0, 1, 37, k - 1):
        e = np.zeros(k, dtype=np.float32)
        e[col] = 1
        assert np.array_equal(orc.matvec(orc.Q8_0, w, n, k, e)[0], ints[:, col].astype(np.float32))
    # batch rows are independent products
    xb = np.stack([x, -x, np.ones(k, np.float32)])
    yb = orc.matvec(orc.Q8_0, w, n, k, xb)
    assert np.array_equal(yb[1], -y[0]) and np.array_equal(yb[2], ints.sum(1).astype(np.float32))


def test_fp32_close_to_fp64_brute_force(orc):
    rng = np.random.default_rng(7)
    n, k = 64, 512
    data = rng.integers(0, 256, n * (k // 256) * 144).astype(np.uint8).reshape(-1, 144)
    data[:, 0:2] = np.array([0x2000], np.uint16).view(np.uint8)   # d = 2^-7
    data[:, 2:4] = np.array([0x1C00], np.uint16).view(np.uint8)   # dmin = 2^-8
    data = data.reshape(-1)
    x = rng.standard_normal((3, k)).astype(np.float32)
    w = G.dequantize(G.Q4_K, data).reshape(n, k).astype(np.float64)
    ref = x.astype(np.float64) @ w.T
    y = orc.matvec(orc.Q4_K, data, n, k, x)
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-6
    y64 = orc.matvec(orc.Q4_K, data, n, k, x, f64=True)
    assert np.linalg.norm(y64 - ref) / np.linalg.norm(ref) < 1e-13


def test_sequential_accumulation_order(orc):
    rng = np.random.default_rng(11)
    n, k = 8, 256
    data = rng.integers(0, 256, n * 210).astype(np.uint8).reshape(n, 210)
    data[:, 208:210] = np.array([0x1400], np.uint16).view(np.uint8)
    data = data.reshape(-1)
    x = rng.standard_normal(k).astype(np.float32)
    w = G.dequantize(G.Q6_K, data).reshape(n, k)
    y = orc.matvec(orc.Q6_K, data, n, k, x)[0]
    run = np.cumsum(x[None, :] * w, axis=1, dtype=np.float32)[:, -1]
    assert np.array_equal(y, run)


def test_threads_do_not_change_results(orc):
    rng = np.random.default_rng(3)
    n, k = 96, 256
    data = rng.integers(0, 256, n * 144).astype(np.uint8).reshape(n, 144)
    data[:, 0:4] = np.array([0x2000, 0x1C00], np.uint16).view(np.uint8)
    data = data.reshape(-1)
    x = rng.standard_normal((2, k)).astype(np.float32)
    a = orc.matvec(orc.Q4_K, data, n, k, x, nthreads=1)
    b = orc.matvec(orc.Q4_K, data, n, k, x, nthreads=4)
    assert np.array_equal(a, b)
