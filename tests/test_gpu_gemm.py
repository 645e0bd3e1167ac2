"""Fused prefill GEMM (MFMA) vs the oracle (fp32 sequential accumulation over
the reference-decoded weights): normwise and max relative error <= 1e-3.

Covers the prefill workload (Q4_K W 4096x4096, X 512x4096), every format,
partial tiles in M and N, K of one step, the ComputeOps-style routing
(M <= 8 -> matvec, larger -> GEMM) and argument errors.
"""
import numpy as np
import pytest

from aihost_amd import _native as nat
from aihost_amd import compute as C
from gpu_util import assert_close, qgemm, synth_weight, upload

pytestmark = pytest.mark.gpu

TOL = 1e-3  # relative 1e-3 with fp32 accumulation


def x_of(m, k, seed=43):
    return C.fill_normal(seed, m * k, 0.0, 1.0).reshape(m, k)


def test_prefill_workload(device, orc):
    n, k, m = 4096, 4096, 512
    w = synth_weight(nat.Q4_K, n, k)
    x = x_of(m, k)
    y = qgemm(device, nat.Q4_K, w, n, k, x)
    ref = orc.matvec(nat.Q4_K, w, n, k, x, nthreads=16)
    nrm, mx = assert_close(y, ref, TOL, "Q4_K 4096x4096 M=512")
    print("Q4_K prefill normwise=%.3g max=%.3g" % (nrm, mx))


@pytest.mark.parametrize("qtype,n,k,m", [
    (nat.Q4_K, 64, 256, 128), (nat.Q4_K, 65, 512, 129), (nat.Q4_K, 1, 256, 9), (nat.Q4_K, 200, 1024, 300),
    (nat.Q6_K, 64, 256, 128), (nat.Q6_K, 100, 768, 77), (nat.Q6_K, 130, 4096, 40),
    (nat.Q8_0, 64, 64, 128), (nat.Q8_0, 63, 320, 200), (nat.Q8_0, 257, 128, 17),
    (nat.Q4_0, 64, 64, 128), (nat.Q4_0, 99, 2048, 65), (nat.Q4_0, 5, 192, 130),
    # 25 64-k chunks: full super-steps in the producers' main loop, a partial
    # last one (one chunk) staged after it
    (nat.Q8_0, 70, 1600, 40), (nat.Q4_0, 33, 1600, 100),
])
def test_shapes(device, orc, qtype, n, k, m):
    w = synth_weight(qtype, n, k, seed=n * 7 + k)
    x = x_of(m, k, seed=m + k)
    y = qgemm(device, qtype, w, n, k, x)
    assert_close(y, orc.matvec(qtype, w, n, k, x, nthreads=8), TOL, "type %d %dx%d M=%d" % (qtype, n, k, m))


# Grids large enough for the 256-row tiles on a 256-CU device (fewer rounds of
# workgroups than the 128-row tiles), and the 512-row tiles of the largest
# grids: partial tiles in M and N, and for Q8_0 a partial last super-step.
@pytest.mark.parametrize("qtype,n,k,m", [
    (nat.Q4_K, 6377, 1536, 300), (nat.Q6_K, 6400, 1024, 384),
    (nat.Q8_0, 6377, 1600, 300), (nat.Q4_0, 6400, 1600, 257),
    # 512-row tiles (more than 256 rows over 447-448 column tiles)
    (nat.Q4_K, 28600, 512, 300), (nat.Q6_K, 28672, 768, 512),
    (nat.Q8_0, 28000, 832, 450), (nat.Q4_0, 28672, 576, 257),
])
def test_wide_tiles(device, orc, qtype, n, k, m):
    tile, splits = nat.qgemm_plan(device.handle, n, k, m)
    want = 512 if n > 20000 else 256
    if (tile, splits) != (want, 1):
        pytest.skip("on this device's CU count the shape takes %d-row tiles, %d splits" % (tile, splits))
    w = synth_weight(qtype, n, k, seed=n + k)
    x = x_of(m, k, seed=m * 3 + k)
    y = qgemm(device, qtype, w, n, k, x)
    assert_close(y, orc.matvec(qtype, w, n, k, x, nthreads=16), TOL, "type %d %dx%d M=%d" % (qtype, n, k, m))


# Products of more than 256 rows whose 512-row tiles leave CUs idle split K
# over workgroups (aih_qgemm;
# aih_matmul_weights_q never splits): the oracle's bound, and the unsplit
# result to summation-order rounding; Q8_0 at K = 4160 and Q4_0 at K = 2112
# end on a partial super-step inside the last split.
@pytest.mark.parametrize("qtype,n,k,m", [
    (nat.Q4_K, 1024, 14336, 300), (nat.Q6_K, 1000, 14336, 512),
    (nat.Q8_0, 512, 4160, 300), (nat.Q4_0, 256, 2112, 290),
])
def test_split_k(device, orc, qtype, n, k, m):
    tile, splits = nat.qgemm_plan(device.handle, n, k, m)
    if splits < 2:
        pytest.skip("on this device's CU count the shape does not split K (%d-row tiles)" % tile)
    assert nat.qgemm_plan(device.handle, n, k, m, may_split=False)[1] == 1
    w = synth_weight(qtype, n, k, seed=n + k + 1)
    x = x_of(m, k, seed=m + 5)
    y = qgemm(device, qtype, w, n, k, x)
    assert_close(y, orc.matvec(qtype, w, n, k, x, nthreads=16), TOL, "type %d %dx%d M=%d" % (qtype, n, k, m))
    wb, xb, yb = upload(device, w), upload(device, x), device.create_buffer(m * n * 4)
    try:
        nat.check(nat.lib().aih_matmul_weights_q(device.handle, int(qtype), wb.get_pointer(), n, k, xb.get_pointer(),
                                                 m, yb.get_pointer()), "aih_matmul_weights_q")
        ref = yb.read_range(0, m * n, np.float32).reshape(m, n)
    finally:
        for b in (wb, xb, yb):
            b.dispose()
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-6


def test_subnormal_scales(device, orc):
    rng = np.random.default_rng(9)
    n, k, m = 70, 512, 33
    for qtype, bb, offs in ((nat.Q4_K, 144, (0, 2)), (nat.Q6_K, 210, (208,)), (nat.Q8_0, 34, (0,)),
                            (nat.Q4_0, 18, (0,))):
        nb = n * k // (256 if bb in (144, 210) else 32)
        data = rng.integers(0, 256, (nb, bb)).astype(np.uint8)
        for off in offs:
            h = rng.integers(0x0001, 0x2400, nb).astype(np.uint16)
            data[:, off:off + 2] = h.view(np.uint8).reshape(nb, 2)
        data = data.reshape(-1)
        x = x_of(m, k, seed=qtype)
        assert_close(qgemm(device, qtype, data, n, k, x), orc.matvec(qtype, data, n, k, x), TOL,
                     "type %d" % qtype)


def test_matmul_weights_routing(device, orc):
    n, k = 96, 512
    w = synth_weight(nat.Q4_K, n, k)
    ops = C.ComputeOps(device)
    wt = C.Tensor.from_quantized(device, w, k, n, C.DataType.Q4_K)
    for m in (1, 8, 9, 40):
        x = x_of(m, k, seed=m)
        a = C.Tensor.from_data(device, x)
        y = ops.matmul_weights(a, wt)
        assert y.shape == (m, n)
        assert_close(y.read(), orc.matvec(nat.Q4_K, w, n, k, x), TOL, "M=%d" % m)
        a.dispose()
        y.dispose()
    wt.dispose()


def test_gemm_rows_match_matvec(device):
    # The GEMM rounds x (times a power of two per row) and each dequantized
    # weight to fp16; the matvec multiplies the codes exactly by a 22-bit
    # fixed-point x and applies the scales in fp32.  The GEMM's two roundings
    # move the result by about 2e-4 normwise; the two paths agree within that.
    from gpu_util import qmatvec
    n, k, m = 256, 4096, 16
    w = synth_weight(nat.Q6_K, n, k)
    x = x_of(m, k)
    yg = qgemm(device, nat.Q6_K, w, n, k, x)
    ym = np.vstack([qmatvec(device, nat.Q6_K, w, n, k, x[i:i + 1]) for i in range(m)])
    assert_close(yg, ym, 5e-4)


def test_argument_errors(device):
    L = nat.lib()
    h = device.handle
    wb = upload(device, np.zeros(4352 * 4, np.uint8))
    xb = upload(device, np.zeros(64 * 4096, np.float32))
    yb = upload(device, np.zeros(64 * 64, np.float32))
    W, X, Y = wb.get_pointer(), xb.get_pointer(), yb.get_pointer()
    try:
        assert L.aih_qgemm(h, nat.Q8_0, W, 4, 4096, X, 16, Y) == nat.AIH_OK
        assert L.aih_qgemm(h, nat.Q8_0, W, 0, 4096, X, 16, Y) == nat.AIH_OK
        assert L.aih_qgemm(h, nat.Q8_0, W, 4, 4096, X, 0, Y) == nat.AIH_OK
        assert L.aih_qgemm(h, nat.Q8_0, W, 4, 100, X, 16, Y) == nat.AIH_E_INVALID
        assert L.aih_qgemm(h, nat.Q8_0, W, 4, 96, X, 16, Y) == nat.AIH_E_LIMIT
        assert L.aih_qgemm(h, nat.F32, W, 4, 4096, X, 16, Y) == nat.AIH_E_UNSUPPORTED
        assert L.aih_qgemm(h, nat.Q8_0, None, 4, 4096, X, 16, Y) == nat.AIH_E_INVALID
        device.synchronize()
    finally:
        for b in (wb, xb, yb):
            b.dispose()


def test_split_shape_same_bits_eager_and_replayed(device):
    """A shape that splits K gives the same bits eagerly and from a replayed
    graph (on a context that ran it once before the capture, so both
    workspaces are sized); a fresh context cannot record it (AIH_E_LIMIT,
    the workspaces cannot grow during a capture) rather than recording an
    unsplit product."""
    import ctypes
    n, k, m = 1024, 14336, 300
    if nat.qgemm_plan(device.handle, n, k, m)[1] < 2:
        pytest.skip("on this device's CU count the shape does not split K")
    L = nat.lib()
    w = synth_weight(nat.Q4_K, n, k, seed=7)
    x = x_of(m, k, seed=8)
    fresh = C.HipComputeDevice(0)
    bufs = []
    try:
        for dev in (device, fresh):
            wb, xb, yb = upload(dev, w), upload(dev, x), dev.create_buffer(m * n * 4)
            bufs.append((dev, wb, xb, yb))
        dev, wb, xb, yb = bufs[0]
        h = dev.handle
        args = (nat.Q4_K, wb.get_pointer(), n, k, xb.get_pointer(), m, yb.get_pointer())
        nat.check(L.aih_qgemm(h, *args), "eager")
        eager = yb.read_range(0, m * n, np.float32).copy()
        nat.check(L.aih_capture_begin(h), "capture")
        st = L.aih_qgemm(h, *args)
        g = ctypes.c_void_p()
        nat.check(L.aih_capture_end(h, ctypes.byref(g)), "capture end")
        nat.check(st, "captured")
        try:
            for _ in range(3):
                nat.check(L.aih_memset(h, yb.get_pointer(), 0xFF, m * n * 4), "memset")
                nat.check(L.aih_graph_launch(h, g.value), "replay")
                dev.synchronize()
                assert np.array_equal(yb.read_range(0, m * n, np.float32).view(np.uint32), eager.view(np.uint32))
        finally:
            L.aih_graph_destroy(g.value)
        dev, wb, xb, yb = bufs[1]
        h = dev.handle
        nat.check(L.aih_capture_begin(h), "capture")
        st = L.aih_qgemm(h, nat.Q4_K, wb.get_pointer(), n, k, xb.get_pointer(), m, yb.get_pointer())
        g = ctypes.c_void_p()
        nat.check(L.aih_capture_end(h, ctypes.byref(g)), "capture end")
        if g.value:
            L.aih_graph_destroy(g.value)
        assert st == nat.AIH_E_LIMIT, nat.strerror(st)
    finally:
        for dev, wb, xb, yb in bufs:
            for b in (wb, xb, yb):
                b.dispose()
        fresh.dispose()
