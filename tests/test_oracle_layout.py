"""Pins the oracle's block decoders: scale packing, element order, arithmetic.

* get_scale_min_k4: every (scale, min) value at every sub-block index, packed by
  an independent statement of the K-quant 12-byte layout.
* element order: single-bit known-answer blocks -- with unit scales each quant
  bit moves exactly one output, at the index ggml's loop structure puts it.
* arithmetic: hand-computed blocks with literal expected values.
* random blocks: oracle == ggml-loop numpy restatement, bit for bit.
"""
import numpy as np
import pytest

import ggml_ref as G

RNG = np.random.default_rng(1234)


def f16bits(v):
    return np.array([v], dtype=np.float16).view(np.uint16)[0]


def put16(b, off, v):
    h = int(f16bits(v))
    b[off], b[off + 1] = h & 0xFF, h >> 8


# ------------------------------------------------------------ scale packing
def test_get_scale_min_k4_all_values(orc):
    for j in range(8):
        for sc in range(64):
            for mn in range(0, 64, 1 if j in (0, 7) else 7):
                scv = RNG.integers(0, 64, 8)
                mnv = RNG.integers(0, 64, 8)
                scv[j], mnv[j] = sc, mn
                packed = G.pack_scales_k4(scv, mnv)
                assert orc.get_scale_min_k4(j, packed) == (sc, mn)


# ------------------------------------------------------------ Q4_K
def q4k_unit_block(scales=None, mins=None, d=1.0, dmin=0.0):
    b = np.zeros(144, dtype=np.uint8)
    put16(b, 0, d)
    put16(b, 2, dmin)
    b[4:16] = G.pack_scales_k4(np.ones(8, int) if scales is None else scales,
                               np.zeros(8, int) if mins is None else mins)
    return b


def test_q4_k_single_bit_positions(orc):
    sc = np.arange(1, 9)
    base = q4k_unit_block(scales=sc)
    assert np.all(orc.dequantize(orc.Q4_K, base, 256) == 0)
    for i in range(128):
        for bit in range(8):
            b = base.copy()
            b[16 + i] = 1 << bit
            y = orc.dequantize(orc.Q4_K, b, 256)
            group, l = divmod(i, 32)
            e = 64 * group + l + (32 if bit >= 4 else 0)
            expect = np.zeros(256, dtype=np.float32)
            expect[e] = sc[e // 32] * (1 << (bit % 4))
            assert np.array_equal(y, expect), (i, bit)


def test_q4_k_mins_per_sub_block(orc):
    b = q4k_unit_block(scales=np.zeros(8, int), mins=np.arange(1, 9), dmin=1.0)
    y = orc.dequantize(orc.Q4_K, b, 256)
    assert np.array_equal(y, -np.repeat(np.arange(1, 9), 32).astype(np.float32))


def test_q4_k_arithmetic_literal(orc):
    # d = 0.5, dmin = 0.25, sub-block 0: sc = 3, mn = 5, q = 7 -> 0.5*3*7 - 0.25*5 = 9.25
    sc = np.array([3, 1, 1, 1, 1, 1, 1, 1])
    mn = np.array([5, 0, 0, 0, 0, 0, 0, 0])
    b = q4k_unit_block(sc, mn, d=0.5, dmin=0.25)
    b[16] = 7
    y = orc.dequantize(orc.Q4_K, b, 256)
    assert y[0] == np.float32(9.25)
    assert y[1] == np.float32(-1.25)
    assert y[32] == 0.0


# ------------------------------------------------------------ Q6_K
def q6k_unit_block(scales, d=1.0):
    b = np.zeros(210, dtype=np.uint8)
    b[192:208] = np.asarray(scales, dtype=np.int8).view(np.uint8)
    put16(b, 208, d)
    return b


def test_q6_k_single_bit_positions(orc):
    sc = np.arange(1, 17)
    base = q6k_unit_block(sc)
    y0 = orc.dequantize(orc.Q6_K, base, 256)
    assert np.array_equal(y0, (-32 * np.repeat(sc, 16)).astype(np.float32))
    for i in range(128):          # ql
        half, r = divmod(i, 64)
        for bit in range(8):
            b = base.copy()
            b[i] = 1 << bit
            y = orc.dequantize(orc.Q6_K, b, 256)
            if r < 32:
                e = 128 * half + r + (64 if bit >= 4 else 0)
            else:
                e = 128 * half + 32 + (r - 32) + (64 if bit >= 4 else 0)
            expect = y0.copy()
            expect[e] = sc[e // 16] * ((1 << (bit % 4)) - 32)
            assert np.array_equal(y, expect), ("ql", i, bit)
    for i in range(64):           # qh
        half, l = divmod(i, 32)
        for bit in range(8):
            b = base.copy()
            b[128 + i] = 1 << bit
            y = orc.dequantize(orc.Q6_K, b, 256)
            e = 128 * half + l + 32 * (bit // 2)
            expect = y0.copy()
            expect[e] = sc[e // 16] * (16 * (1 << (bit % 2)) - 32)
            assert np.array_equal(y, expect), ("qh", i, bit)


def test_q6_k_scale_sign_and_literal(orc):
    sc = np.ones(16, int)
    sc[0] = -128
    sc[1] = -3
    b = q6k_unit_block(sc, d=2.0)
    # element 16 is in sub-block 1: q = 5 -> 2 * (-3) * (5 - 32) = 162
    b[16] = 5
    y = orc.dequantize(orc.Q6_K, b, 256)
    assert y[16] == np.float32(162.0)
    assert y[0] == np.float32(2.0 * -128 * -32)
    # q = 63 (all bits) -> (63 - 32) = 31
    b2 = q6k_unit_block(np.ones(16, int), d=1.0)
    b2[0] = 0x0F
    b2[128] = 0x03
    assert orc.dequantize(orc.Q6_K, b2, 256)[0] == np.float32(31.0)


# ------------------------------------------------------------ Q8_0 / Q4_0
def test_q8_0_single_bits_and_literal(orc):
    base = np.zeros(34, dtype=np.uint8)
    put16(base, 0, 1.0)
    for j in range(32):
        for bit in range(8):
            b = base.copy()
            b[2 + j] = 1 << bit
            y = orc.dequantize(orc.Q8_0, b, 32)
            expect = np.zeros(32, dtype=np.float32)
            expect[j] = np.int8(np.uint8(1 << bit).view(np.int8))
            assert np.array_equal(y, expect)
    b = base.copy()
    put16(b, 0, 0.5)
    b[2] = np.uint8(np.int8(-7).view(np.uint8))
    assert orc.dequantize(orc.Q8_0, b, 32)[0] == np.float32(-3.5)


def test_q4_0_single_bits_and_literal(orc):
    base = np.zeros(18, dtype=np.uint8)
    put16(base, 0, 1.0)
    assert np.all(orc.dequantize(orc.Q4_0, base, 32) == -8)
    for j in range(16):
        for bit in range(8):
            b = base.copy()
            b[2 + j] = 1 << bit
            y = orc.dequantize(orc.Q4_0, b, 32)
            expect = np.full(32, -8, dtype=np.float32)
            expect[j + (16 if bit >= 4 else 0)] = (1 << (bit % 4)) - 8
            assert np.array_equal(y, expect)
    b = base.copy()
    put16(b, 0, 0.25)
    b[2] = 3
    assert orc.dequantize(orc.Q4_0, b, 32)[0] == np.float32(-1.25)


# ------------------------------------------------------------ random blocks
def finite_f16_bits(n):
    h = RNG.integers(0, 0x7C00, n).astype(np.uint16)          # finite, non-negative
    h |= (RNG.integers(0, 2, n).astype(np.uint16) << 15)
    h[h == 0x8000] = 0x0001                                  # no -0 (GLSL maps it to +0)
    return h


@pytest.mark.parametrize("qtype", [G.Q4_K, G.Q6_K, G.Q8_0, G.Q4_0])
def test_random_blocks_match_ggml_statement(orc, qtype):
    nb = 64
    bb = G.BB[qtype]
    data = RNG.integers(0, 256, nb * bb).astype(np.uint8).reshape(nb, bb)
    # keep the fp16 fields finite; include subnormal scales
    if qtype == G.Q4_K:
        data[:, 0:2] = finite_f16_bits(nb).view(np.uint8).reshape(nb, 2)
        data[:, 2:4] = finite_f16_bits(nb).view(np.uint8).reshape(nb, 2)
    elif qtype == G.Q6_K:
        data[:, 208:210] = finite_f16_bits(nb).view(np.uint8).reshape(nb, 2)
    else:
        data[:, 0:2] = finite_f16_bits(nb).view(np.uint8).reshape(nb, 2)
    data = data.reshape(-1)
    n = nb * G.QK[qtype]
    got = orc.dequantize(qtype, data, n, orc.F16_IEEE)
    ref = G.dequantize(qtype, data)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_rejects_partial_blocks(orc):
    with pytest.raises(ValueError):
        orc.dequantize(orc.Q4_K, np.zeros(144, np.uint8), 100)
    assert orc.row_bytes(orc.Q4_K, 4096) == 16 * 144
    assert orc.row_bytes(orc.Q6_K, 14336) == 11760
    assert orc.row_bytes(orc.Q8_0, 4096) == 4352
    assert orc.row_bytes(orc.Q4_0, 4096) == 2304
    assert orc.row_bytes(orc.Q4_K, 100) == -1
