"""Pins the oracle's two fp16 decoders over all 65536 bit patterns.

ieee (QuantizationFormats.cs:147-152): must equal IEEE binary16 -> binary32
(numpy's float16) for every finite value except -0 (the GLSL decoder returns
+0), and map every NaN to 0x7FC00000.

refcpu (ComputeOps.cs:1497-1522): equal to IEEE for normals, zeros and
infinities; NaN payload and sign kept; for a subnormal with mantissa m whose
leading bit is at position p it yields m * 2^(1 - 2p) (exponent 1 - p + 127 on
the normalised mantissa m / 2^p) instead of the correct m * 2^-24.
"""
import numpy as np
import pytest


@pytest.fixture(scope="module")
def table(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ieee = orc.f16_decode(h, orc.F16_IEEE)
    ref = orc.f16_decode(h, orc.F16_REFCPU)
    true = h.view(np.float16).astype(np.float32)
    return h, ieee, ref, true


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_ieee_matches_binary16(table):
    h, ieee, _, true = table
    exp = (h >> 10) & 31
    man = h & 1023
    nan = (exp == 31) & (man != 0)
    negzero = h == 0x8000
    ok = ~nan & ~negzero
    assert np.array_equal(bits(ieee)[ok], bits(true)[ok])
    assert np.all(bits(ieee)[nan] == 0x7FC00000)
    assert bits(ieee)[negzero][0] == 0x00000000


def test_refcpu_normals_zeros_inf(table):
    h, _, ref, true = table
    exp = (h >> 10) & 31
    man = h & 1023
    sel = ((exp > 0) & (exp < 31)) | (man == 0)
    assert np.array_equal(bits(ref)[sel], bits(true)[sel])


def test_refcpu_subnormal_closed_form(table):
    h, _, ref, true = table
    exp = (h >> 10) & 31
    man = (h & 1023).astype(np.int64)
    sub = (exp == 0) & (man != 0)
    assert sub.sum() == 2046
    p = np.floor(np.log2(man[sub])).astype(np.int64)
    sign = np.where(h[sub] >> 15, -1.0, 1.0)
    expect = sign * man[sub].astype(np.float64) * np.power(2.0, (1 - 2 * p).astype(np.float64))
    assert np.array_equal(ref[sub].astype(np.float64), expect)
    # and every one of them differs from the correct value
    assert np.all(ref[sub] != true[sub])
    # the survey's example: 0x00E6 -> 0.0281 instead of 1.371e-5
    i = int(np.where(h == 0x00E6)[0][0])
    assert abs(ref[i] - 0.028076171875) < 1e-9 and abs(true[i] - 1.3709068e-05) < 1e-10


def test_refcpu_nan_payload(table):
    h, _, ref, _ = table
    exp = (h >> 10) & 31
    man = (h & 1023).astype(np.uint32)
    nan = (exp == 31) & (man != 0)
    expect = ((h[nan].astype(np.uint32) >> 15) << 31) | (0xFF << 23) | (man[nan] << 13)
    assert np.array_equal(bits(ref)[nan], expect)
