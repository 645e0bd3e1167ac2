"""Host utilities of libaihost_hip.so (no GPU needed): the synthetic normal
generator and the GGUF quantizers used to build benchmark/test weights.

The quantizers have no reference counterpart (AIHost only reads GGUF files);
they are checked for producing valid blocks whose dequantization (by the
oracle) is close to the input, and for the fp16 rounding of their scales.
"""
import numpy as np
import pytest

from aihost_amd import compute as C


def splitmix_normal(seed, n):
    """numpy restatement of the generator: splitmix64 counter + Box-Muller."""
    i = np.arange(2 * ((n + 1) // 2), dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (i + np.uint64(1)) * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    u = ((z >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    th = 2.0 * np.pi * u2
    out = np.empty(u.size, dtype=np.float64)
    out[0::2], out[1::2] = r * np.cos(th), r * np.sin(th)
    return out[:n]


def test_fill_normal_definition_and_stats():
    a = C.fill_normal(42, 100001, 0.0, 1.0)
    b = C.fill_normal(42, 100001, 0.0, 1.0)
    assert np.array_equal(a, b)
    ref = splitmix_normal(42, 100001)
    assert np.max(np.abs(a.astype(np.float64) - ref)) < 1e-6
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    w = C.fill_normal(43, 200000, 0.0, 0.02)
    assert abs(w.std() - 0.02) < 3e-4
    assert not np.array_equal(C.fill_normal(1, 16), C.fill_normal(2, 16))


@pytest.mark.parametrize("dtype,rel_rms", [(C.GGUFTensorType.Q8_0, 0.01), (C.GGUFTensorType.Q4_0, 0.15),
                                           (C.GGUFTensorType.Q4_K, 0.12), (C.GGUFTensorType.Q6_K, 0.03)])
def test_quantize_round_trip(orc, dtype, rel_rms):
    n, k = 32, 512
    x = C.fill_normal(5, n * k, 0.0, 0.02)
    q = C.quantize(dtype, x, n, k)
    assert q.size == n * C.row_bytes(dtype, k)
    y = orc.dequantize(int(dtype), q, n * k)
    err = np.sqrt(np.mean((y - x) ** 2)) / np.sqrt(np.mean(x ** 2))
    assert err < rel_rms, err


def test_q8_0_error_bound_and_scale_rounding(orc):
    n, k = 16, 256
    x = C.fill_normal(9, n * k, 0.0, 1.0)
    q = C.quantize(C.GGUFTensorType.Q8_0, x, n, k).reshape(-1, 34)
    xb = x.reshape(-1, 32)
    d_expect = (np.abs(xb).max(1) / np.float32(127)).astype(np.float32).astype(np.float16)
    assert np.array_equal(q[:, 0:2].copy().view(np.uint16)[:, 0], d_expect.view(np.uint16))
    y = orc.dequantize(orc.Q8_0, q.reshape(-1), n * k).reshape(-1, 32)
    d = d_expect.astype(np.float32)[:, None]
    # rounding to the nearest code plus the fp16 rounding of d itself
    assert np.all(np.abs(y - xb) <= 0.5 * d + 127 * d * 2.0 ** -11 + 1e-7)


def test_q6_k_scales_are_subnormal_at_small_sigma():
    # N(0, 0.02) weights give Q6_K super-scales below 2^-14 (fp16 subnormal)
    x = C.fill_normal(42, 64 * 256, 0.0, 0.02)
    q = C.quantize(C.GGUFTensorType.Q6_K, x, 64, 256).reshape(-1, 210)
    d = q[:, 208:210].copy().view(np.uint16)[:, 0]
    assert np.all((d & 0x7C00) == 0) and np.all((d & 0x3FF) != 0)


def test_quantize_rejects_bad_shapes():
    with pytest.raises(ValueError):
        C.quantize(C.GGUFTensorType.Q4_K, np.zeros(100, np.float32), 1, 100)
    with pytest.raises(ValueError):
        C.row_bytes(C.GGUFTensorType.Q6_K, 300)
    assert C.row_bytes(C.GGUFTensorType.Q4_K, 4096) == 2304
