"""aih_qmatvec_fused: the decode matvec with RMSNorm or SiLU*up fused into its
activation prologue and the residual add into its epilogue, against the
separate operators run through the C ABI.

The SiLU-pairs epilogue (gate/up rows interleaved, Y = SiLU(gate)*up) is
bit-exact to aih_qmatvec + aih_silu_mul_pairs without a prologue, within
1e-5 of them behind the RMSNorm prologue, and within 2e-5 of the oracle.

Bars: SiLU*up and the accumulate are bit-exact to aih_silu_mul + aih_qmatvec
and to y0 + aih_qmatvec (the same fp32 formulas ahead of the same product);
RMSNorm within 1e-5 normwise of aih_rmsnorm + aih_qmatvec (its sum of squares
is reduced in another order, which moves the rms by an ulp or so) and within
2e-5 of the oracle (the matvec's own bound; see test_gpu_matvec.py).  Shapes cover the
single-wave-team kernel (K 4096), multi-wave teams (K 14336), the
single-team kernel (K 65536) and a ragged row count (remainder launch).
"""
import numpy as np
import pytest

from aihost_amd import _native as nat
from aihost_amd import compute as C
from gpu_util import synth_weight, upload
from oracle import llama as ol

pytestmark = pytest.mark.gpu


def _run(device, qtype, w, n, k, x, x2, pre, post, y0):
    L = nat.lib()
    bufs = [upload(device, w), upload(device, x), upload(device, x2 if x2 is not None else np.zeros(4, np.float32)),
            upload(device, y0)]
    W, X, X2, Y = (b.get_pointer() for b in bufs)
    try:
        nat.check(L.aih_qmatvec_fused(device.handle, qtype, W, n, k, X, X2 if x2 is not None else None, 1e-5, pre,
                                      post, Y), "fused")
        return bufs[3].read_range(0, y0.size, np.float32)
    finally:
        for b in bufs:
            b.dispose()


def _plain(device, qtype, w, n, k, x):
    from gpu_util import qmatvec
    return qmatvec(device, qtype, w, n, k, x.reshape(1, k))[0, :n]


def _gpu_op(device, fn, *arrays, n):
    L = nat.lib()
    bufs = [upload(device, a) for a in arrays]
    out = device.create_buffer(n * 4)
    try:
        fn(L, device.handle, *[b.get_pointer() for b in bufs], out.get_pointer())
        return out.read_range(0, n, np.float32)
    finally:
        for b in bufs + [out]:
            b.dispose()


# the last shape is taller than one launch covers (131072 rows of eight-team
# workgroups on 256 CUs), with five odd rows for the single-team launch
SHAPES = [(nat.Q4_K, 6144, 4096), (nat.Q4_K, 4096, 14336), (nat.Q6_K, 32000, 4096), (nat.Q4_K, 8, 65536),
          (nat.Q4_K, 4101, 4096), (nat.Q8_0, 1030, 4096), (nat.Q4_0, 131101, 256)]


@pytest.mark.parametrize("qtype,n,k", SHAPES)
def test_silu_mul_prologue_and_accumulate_exact(device, orc, qtype, n, k):
    w = synth_weight(qtype, n, k, seed=n + k)
    g = C.fill_normal(n + 1, k, 0.0, 2.0)
    u = C.fill_normal(n + 2, k, 0.0, 1.0)
    y0 = C.fill_normal(n + 3, n, 0.0, 1.0)
    h = _gpu_op(device, lambda L, hd, G, U, O: nat.check(L.aih_silu_mul(hd, G, U, O, k), "silu"), g, u, n=k)
    plain = _plain(device, qtype, w, n, k, h)
    got = _run(device, qtype, w, n, k, g, u, nat.PRE_SILU_MUL, 0, np.zeros(n, np.float32))
    assert np.array_equal(got, plain)
    got = _run(device, qtype, w, n, k, g, u, nat.PRE_SILU_MUL, 1, y0)
    assert np.array_equal(got, y0 + plain)
    ref = orc.matvec(qtype, w, n, k, ol.silu_mul(g, u).reshape(1, k))[0]
    assert np.linalg.norm(plain - ref) / np.linalg.norm(ref) < 2e-5


@pytest.mark.parametrize("qtype,n,k", SHAPES)
def test_rmsnorm_prologue(device, orc, qtype, n, k):
    w = synth_weight(qtype, n, k, seed=n * 3 + k)
    x = C.fill_normal(n + 5, k, 0.0, 3.0)
    gw = 1.0 + C.fill_normal(n + 6, k, 0.0, 0.02)
    xn = _gpu_op(device, lambda L, hd, X, G, O: nat.check(L.aih_rmsnorm(hd, X, G, O, 1, k, 1e-5), "norm"), x, gw,
                 n=k)
    plain = _plain(device, qtype, w, n, k, xn)
    got = _run(device, qtype, w, n, k, x, gw, nat.PRE_RMSNORM, 0, np.zeros(n, np.float32))
    assert np.linalg.norm(got - plain) / np.linalg.norm(plain) < 1e-5
    ref = orc.matvec(qtype, w, n, k, ol.rmsnorm(x.reshape(1, k), gw).reshape(1, k))[0]
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 2e-5


def test_plain_and_accumulate_without_prologue(device):
    n, k = 4096, 4096
    w = synth_weight(nat.Q4_K, n, k, seed=9)
    x = C.fill_normal(10, k, 0.0, 1.0)
    y0 = C.fill_normal(11, n, 0.0, 1.0)
    plain = _plain(device, nat.Q4_K, w, n, k, x)
    assert np.array_equal(_run(device, nat.Q4_K, w, n, k, x, None, nat.PRE_NONE, 0, y0), plain)
    assert np.array_equal(_run(device, nat.Q4_K, w, n, k, x, None, nat.PRE_NONE, 1, y0), y0 + plain)


def _interleave(qtype, gate, up, n, k):
    rb = C.row_bytes(qtype, k)
    return np.stack([gate.reshape(n, rb), up.reshape(n, rb)], axis=1).reshape(-1)


# (qtype, ffn, k): 8 single-wave teams (k 4096), 4 two-wave teams (k 8192),
# 2 four-wave teams (k 16384), a launch split by the 64-row-group cap
PAIR_SHAPES = [(nat.Q4_K, 14336, 4096), (nat.Q4_K, 4096, 8192), (nat.Q6_K, 1000, 16384), (nat.Q8_0, 1028, 4096),
               (nat.Q4_K, 65536 + 8, 256)]


@pytest.mark.parametrize("qtype,f,k", PAIR_SHAPES)
@pytest.mark.parametrize("pre", [nat.PRE_NONE, nat.PRE_RMSNORM])
def test_silu_pairs_epilogue(device, orc, qtype, f, k, pre):
    gate = synth_weight(qtype, f, k, seed=f + k)
    up = synth_weight(qtype, f, k, seed=f + k + 1)
    w = _interleave(qtype, gate, up, f, k)
    x = C.fill_normal(f + 5, k, 0.0, 1.0 if pre == nat.PRE_NONE else 3.0)
    gw = 1.0 + C.fill_normal(f + 6, k, 0.0, 0.02)
    got = _run(device, qtype, w, 2 * f, k, x, gw if pre else None, pre, nat.POST_SILU_PAIRS,
               np.zeros(f, np.float32))
    xin = x
    if pre == nat.PRE_RMSNORM:
        xin = _gpu_op(device, lambda L, hd, X, G, O: nat.check(L.aih_rmsnorm(hd, X, G, O, 1, k, 1e-5), "norm"),
                      x, gw, n=k)
    y = _plain(device, qtype, w, 2 * f, k, xin)
    two_step = _gpu_op(device, lambda L, hd, Y, O: nat.check(L.aih_silu_mul_pairs(hd, Y, O, 1, f), "pairs"),
                       y, n=f)
    if pre == nat.PRE_NONE:
        assert np.array_equal(got, two_step)
    else:
        assert np.linalg.norm(got - two_step) / np.linalg.norm(two_step) < 1e-5
    xr = x.reshape(1, k) if pre == nat.PRE_NONE else ol.rmsnorm(x.reshape(1, k), gw).reshape(1, k)
    ref = ol.silu_mul(orc.matvec(qtype, gate, f, k, xr)[0], orc.matvec(qtype, up, f, k, xr)[0])
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 2e-5


def test_fused_argument_errors(device):
    L = nat.lib()
    b = upload(device, np.zeros(2304 * 4, np.uint8))
    X = upload(device, np.zeros(4096, np.float32))
    h = device.handle
    try:
        P, XP = b.get_pointer(), X.get_pointer()
        assert L.aih_qmatvec_fused(h, nat.Q4_K, P, 4, 4096, XP, None, 1e-5, 3, 0, XP) == nat.AIH_E_INVALID
        assert L.aih_qmatvec_fused(h, nat.Q4_K, P, 4, 4096, XP, None, 1e-5, nat.PRE_RMSNORM, 0, XP) == nat.AIH_E_INVALID
        assert L.aih_qmatvec_fused(h, nat.Q4_K, P, 4, 4096, XP, XP + 4, 1e-5, nat.PRE_SILU_MUL, 0, XP) \
            == nat.AIH_E_INVALID
        assert L.aih_qmatvec_fused(h, nat.F32, P, 4, 4096, XP, None, 1e-5, 0, 0, XP) == nat.AIH_E_UNSUPPORTED
        assert L.aih_qmatvec_fused(h, nat.Q4_K, P, 4, 4096, XP, None, 1e-5, 0, 3, XP) == nat.AIH_E_INVALID
        # pairs: an odd height, a height that is not a multiple of the team
        # count (8 for K 4096), a width past 16384 (single-team kernel)
        pairs = nat.POST_SILU_PAIRS
        assert L.aih_qmatvec_fused(h, nat.Q4_K, P, 3, 4096, XP, None, 1e-5, 0, pairs, XP) == nat.AIH_E_INVALID
        assert L.aih_qmatvec_fused(h, nat.Q4_K, P, 4, 4096, XP, None, 1e-5, 0, pairs, XP) == nat.AIH_E_LIMIT
        assert L.aih_qmatvec_fused(h, nat.Q4_K, P, 2, 16640, XP, None, 1e-5, 0, pairs, XP) == nat.AIH_E_LIMIT
        device.synchronize()
    finally:
        b.dispose()
        X.dispose()
