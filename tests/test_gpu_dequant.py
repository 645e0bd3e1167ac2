"""GPU dequantization is bit-exact to the oracle in both fp16 modes.

Modes: IEEE = the reference GPU decoder (QuantizationFormats.cs:147-152),
REFCPU = the reference CPU decoder with its subnormal defect
(ComputeOps.cs:1497-1522).  Inputs cover random bytes with crafted fp16 scale
fields (normal, subnormal, +-0, +-inf, NaN) and real quantized N(0, 0.02)
weights at the benchmark shapes (where every Q6_K scale is subnormal).
NaN outputs are compared by position: IEEE arithmetic on a NaN operand does
not fix the payload of the result.
"""
import numpy as np
import pytest

from aihost_amd import _native as nat
from gpu_util import dequant, synth_weight

pytestmark = pytest.mark.gpu

BB = {nat.Q4_K: 144, nat.Q6_K: 210, nat.Q8_0: 34, nat.Q4_0: 18}
QK = {nat.Q4_K: 256, nat.Q6_K: 256, nat.Q8_0: 32, nat.Q4_0: 32}
SCALE_OFFS = {nat.Q4_K: (0, 2), nat.Q6_K: (208,), nat.Q8_0: (0,), nat.Q4_0: (0,)}
TYPES = [nat.Q4_K, nat.Q6_K, nat.Q8_0, nat.Q4_0]


def crafted_blocks(qtype, nb, seed):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (nb, BB[qtype])).astype(np.uint8)
    specials = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x8200, 0x0400, 0x3C00, 0xBC00,
                         0x7BFF, 0x7C00, 0xFC00, 0x7C01, 0x7E00, 0xFE55, 0x00E6, 0x1400], dtype=np.uint16)
    for off in SCALE_OFFS[qtype]:
        h = rng.integers(0, 65536, nb).astype(np.uint16)
        pick = rng.random(nb) < 0.3
        h[pick] = specials[rng.integers(0, specials.size, pick.sum())]
        sub = rng.random(nb) < 0.2
        h[sub] = rng.integers(1, 1024, sub.sum()).astype(np.uint16)   # subnormals
        b[:, off:off + 2] = h.view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def compare(got, ref):
    gn, rn = np.isnan(got), np.isnan(ref)
    assert np.array_equal(gn, rn)
    ok = ~rn
    bad = np.nonzero(got[ok].view(np.uint32) != ref[ok].view(np.uint32))[0]
    assert bad.size == 0, "first mismatch at %d: %r vs %r" % (bad[0], got[ok][bad[0]], ref[ok][bad[0]])


@pytest.mark.parametrize("mode", [nat.F16_IEEE, nat.F16_REFCPU])
@pytest.mark.parametrize("qtype", TYPES)
def test_crafted_blocks_bit_exact(device, orc, qtype, mode):
    nb = 3001
    data = crafted_blocks(qtype, nb, seed=100 + qtype)
    n = nb * QK[qtype]
    compare(dequant(device, qtype, data, n, mode), orc.dequantize(qtype, data, n, mode))


@pytest.mark.parametrize("mode", [nat.F16_IEEE, nat.F16_REFCPU])
@pytest.mark.parametrize("qtype,n,k", [(nat.Q4_K, 14336, 4096), (nat.Q6_K, 4096, 14336),
                                       (nat.Q8_0, 4096, 4096), (nat.Q4_0, 14336, 4096)])
def test_benchmark_shapes_bit_exact(device, orc, qtype, n, k, mode):
    data = synth_weight(qtype, n, k)
    got = dequant(device, qtype, data, n * k, mode)
    ref = orc.dequantize(qtype, data, n * k, mode)
    compare(got, ref)
    assert not np.isnan(got).any()


def test_refcpu_differs_only_where_q6k_scales_are_subnormal(device):
    data = synth_weight(nat.Q6_K, 64, 4096)
    a = dequant(device, nat.Q6_K, data, 64 * 4096, nat.F16_IEEE)
    b = dequant(device, nat.Q6_K, data, 64 * 4096, nat.F16_REFCPU)
    # N(0, 0.02) Q6_K super-scales are fp16 subnormals: the two decoders disagree
    assert np.mean(a != b) > 0.9
    q4 = synth_weight(nat.Q4_K, 64, 4096)
    assert np.array_equal(dequant(device, nat.Q4_K, q4, 64 * 4096, nat.F16_IEEE),
                          dequant(device, nat.Q4_K, q4, 64 * 4096, nat.F16_REFCPU))


def test_argument_errors(device):
    L = nat.lib()
    assert L.aih_dequantize(device.handle, nat.Q4_K, None, None, 0, 0) == nat.AIH_OK
    assert L.aih_dequantize(device.handle, nat.Q4_K, 16, 16, 100, 0) == nat.AIH_E_INVALID
    assert L.aih_dequantize(device.handle, 3, 16, 16, 32, 0) == nat.AIH_E_UNSUPPORTED
    assert L.aih_dequantize(device.handle, nat.Q8_0, 16, 16, 32, 7) == nat.AIH_E_INVALID
