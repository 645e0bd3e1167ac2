"""Fused decode matvec vs the oracle (fp32 sequential accumulation over the
reference-decoded weights): normwise and max relative error <= 2e-5.

Both matvec kernels compute with fp32-equivalent precision (exact integer
or fp16 x fp16 products of the codes and a power-of-two-scaled fixed-point
or hi/lo split of x; fp32 sums; the reference's scale formulas in fp32).
Measured against an fp64 product over the same dequantized weights they
are within 2e-6; the oracle's own sequential fp32 sum is 1e-6 (K = 4096) to
5e-6 (K = 65536) away from that, so 2e-5 leaves a margin of about 4 over
the largest combined error.

Covers the benchmark shapes (Q8_0 4096x4096; Q4_0 and Q4_K 14336x4096; Q6_K
4096x14336 at batch 1, 2, 4, 8), odd row counts (partial row groups), small K,
multi-wave K (14336), K beyond 256 units (1024-thread variant), odd batch,
matrices taller than one launch, padded strides, and argument errors.
"""
import ctypes

import numpy as np
import pytest

from aihost_amd import _native as nat
from aihost_amd import compute as C
from gpu_util import assert_close, qmatvec, synth_weight, upload

pytestmark = pytest.mark.gpu

TOL = 2e-5  # fp32-equivalent: see the module docstring


def x_of(k, batch, seed=43):
    return C.fill_normal(seed, batch * k, 0.0, 1.0).reshape(batch, k)


@pytest.mark.parametrize("qtype,n,k,batch", [
    (nat.Q8_0, 4096, 4096, 1),
    (nat.Q4_0, 14336, 4096, 1),
    (nat.Q4_K, 14336, 4096, 1),
    (nat.Q6_K, 4096, 14336, 1),
    (nat.Q6_K, 4096, 14336, 2),
    (nat.Q6_K, 4096, 14336, 4),
    (nat.Q6_K, 4096, 14336, 8),
])
def test_benchmark_shapes(device, orc, qtype, n, k, batch):
    w = synth_weight(qtype, n, k)
    x = x_of(k, batch)
    y = qmatvec(device, qtype, w, n, k, x)
    ref = orc.matvec(qtype, w, n, k, x, nthreads=8)
    nrm, mx = assert_close(y, ref, TOL, "type %d %dx%d b%d" % (qtype, n, k, batch))
    print("type=%d N=%d K=%d batch=%d normwise=%.3g max=%.3g" % (qtype, n, k, batch, nrm, mx))


@pytest.mark.parametrize("qtype,n,k,batch", [
    (nat.Q4_K, 1, 256, 1), (nat.Q4_K, 37, 256, 1), (nat.Q4_K, 101, 1024, 3), (nat.Q4_K, 64, 14336, 2),
    (nat.Q6_K, 33, 512, 2), (nat.Q6_K, 7, 256, 5), (nat.Q6_K, 130, 4096, 1),
    (nat.Q8_0, 19, 128, 1), (nat.Q8_0, 9, 64, 2), (nat.Q8_0, 8, 20480, 1), (nat.Q8_0, 5, 4160, 3),
    (nat.Q4_0, 5, 64, 1), (nat.Q4_0, 66, 2048, 2), (nat.Q4_0, 3, 32768, 1),
    (nat.Q4_K, 3, 65536, 1),
    # batch 1-2, several teams of several waves sharing x through LDS (the
    # first weight row is loaded after the conversion): four teams of two
    # waves (K 4160..8192), two teams of three waves (K 12288), and an odd N
    # whose last row goes to the single-team launch
    (nat.Q4_K, 70, 8192, 1), (nat.Q6_K, 41, 6144, 2), (nat.Q4_0, 9, 5120, 1), (nat.Q8_0, 23, 12288, 2),
    (nat.Q6_K, 51, 14336, 1),
    # taller than one launch covers (at most 64 row groups per workgroup, one
    # workgroup per CU: 131072 rows of eight-team workgroups on 256 CUs): a
    # second launch at a row offset, then the odd rows' single-team launch
    (nat.Q4_0, 131101, 256, 1), (nat.Q4_K, 131101, 256, 2),
    # batch 3..8 (matrix-core kernel): chunks per wave around the ring depth
    # (8 sets; 6 for Q6_K) -- tail only, one loop pass, exact multiples, a
    # shorter last wave
    (nat.Q4_K, 40, 8192, 3), (nat.Q4_K, 40, 8704, 4), (nat.Q4_K, 33, 7680, 8), (nat.Q4_K, 24, 8960, 3),
    (nat.Q6_K, 48, 6144, 3), (nat.Q6_K, 48, 6656, 8), (nat.Q6_K, 17, 5632, 5),
    (nat.Q8_0, 20, 8192, 6), (nat.Q4_0, 20, 8704, 7),
    # a partial last unit (Q8_0: 130 blocks = 16 units + 2 blocks; Q4_0: 34
    # blocks), a unit of two blocks, a single unit
    (nat.Q8_0, 9, 4160, 3), (nat.Q4_0, 30, 1088, 6), (nat.Q8_0, 40, 64, 4), (nat.Q4_K, 16, 512, 8),
    # batch 3..8 with K split over workgroups (sizes for 256 CUs): splits of
    # several rounds with a partial last unit (Q4_0, 17 units of which the
    # last holds 2 blocks, 3 splits of 6/6/5 units); rounds of 2 + 1 units
    # (Q6_K); one split per row tile, Y stored directly (Q8_0, 1032 tiles)
    (nat.Q4_0, 21888, 4160, 4), (nat.Q6_K, 21888, 2048, 8), (nat.Q8_0, 66000, 256, 5),
])
def test_edge_shapes(device, orc, qtype, n, k, batch):
    w = synth_weight(qtype, n, k, seed=n * 1000 + k)
    x = x_of(k, batch, seed=k + batch)
    y = qmatvec(device, qtype, w, n, k, x)
    ref = orc.matvec(qtype, w, n, k, x, nthreads=8)
    assert_close(y, ref, TOL, "type %d %dx%d b%d" % (qtype, n, k, batch))


@pytest.mark.parametrize("qtype,n,k,batch", [
    (nat.Q8_0, 140001, 64, 2),     # more rows than one launch holds (64 row groups per workgroup)
    (nat.Q4_K, 140001, 256, 1),
    (nat.Q6_K, 32000, 4096, 1),    # output-projection shape: many rows per team
])
def test_tall_matrices(device, orc, qtype, n, k, batch):
    w = synth_weight(qtype, n, k, seed=7)
    x = x_of(k, batch, seed=11)
    y = qmatvec(device, qtype, w, n, k, x)
    ref = orc.matvec(qtype, w, n, k, x, nthreads=8)
    assert_close(y, ref, TOL, "type %d %dx%d b%d" % (qtype, n, k, batch))


def test_small_batch_in_graphs(orc):
    """Batch 3..8 captured into a graph: before the workspace is sized the
    call runs with one split (no workspace); after it, with the split path,
    whose replays equal the eager call bit for bit (the splits are added in a
    fixed order).  Replays alternate with eager work."""
    from aihost_amd.compute import HipComputeDevice
    L = nat.lib()
    n, k, batch = 4096, 7168, 4
    w = synth_weight(nat.Q6_K, n, k, seed=3)
    x = x_of(k, batch, seed=4)
    ref = orc.matvec(nat.Q6_K, w, n, k, x, nthreads=8)
    dev = HipComputeDevice(0)   # a fresh context: empty workspace
    bufs = []
    try:
        wb, xb = upload(dev, w), upload(dev, x)
        ya, yb = dev.create_buffer(batch * n * 4), dev.create_buffer(batch * n * 4)
        bufs = [wb, xb, ya, yb]

        def call(y):
            nat.check(L.aih_qmatvec(dev.handle, nat.Q6_K, wb.get_pointer(), n, k, xb.get_pointer(), k,
                                    y.get_pointer(), n, batch), "aih_qmatvec")

        def capture(y):
            nat.check(L.aih_capture_begin(dev.handle), "capture_begin")
            call(y)
            g = ctypes.c_void_p()
            nat.check(L.aih_capture_end(dev.handle, ctypes.byref(g)), "capture_end")
            return g.value

        def read(y):
            return y.read_range(0, batch * n, np.float32).reshape(batch, n)

        g1 = capture(ya)                      # workspace empty: one split
        outs = []
        for _ in range(3):
            nat.check(L.aih_memset(dev.handle, ya.get_pointer(), 0xFF, batch * n * 4), "memset")
            nat.check(L.aih_graph_launch(dev.handle, g1), "graph_launch")
            outs.append(read(ya))
            call(yb)                          # eager work between replays (sizes the workspace)
            dev.synchronize()
        for o in outs:
            assert_close(o, ref, TOL, "one-split graph")
            assert np.array_equal(o, outs[0])
        eager = read(yb)
        assert_close(eager, ref, TOL, "split path")
        g2 = capture(ya)                      # workspace sized: split path in the graph
        for _ in range(3):
            nat.check(L.aih_memset(dev.handle, ya.get_pointer(), 0xFF, batch * n * 4), "memset")
            nat.check(L.aih_graph_launch(dev.handle, g2), "graph_launch")
            assert np.array_equal(read(ya), eager)
            call(yb)
            dev.synchronize()
        # the first graph still runs after the workspace grew
        nat.check(L.aih_graph_launch(dev.handle, g1), "graph_launch")
        assert np.array_equal(read(ya), outs[0])
        L.aih_graph_destroy(g1)
        L.aih_graph_destroy(g2)
    finally:
        for b in bufs:
            b.dispose()
        dev.dispose()


def test_padded_strides_leave_gaps_untouched(device, orc):
    n, k, batch = 50, 512, 3
    w = synth_weight(nat.Q4_K, n, k)
    x = x_of(k, batch)
    y = qmatvec(device, nat.Q4_K, w, n, k, x, ldx=k + 64, ldy=n + 14)
    assert_close(y[:, :n], orc.matvec(nat.Q4_K, w, n, k, x), TOL)
    assert np.all(np.isnan(y[:, n:]))  # memset 0xFF pattern untouched


@pytest.mark.parametrize("batch", [2, 5])   # integer-dot kernel (batch 1-2), matrix-core kernel (3-8)
def test_subnormal_and_extreme_scales(device, orc, batch):
    # random bytes with small finite scales: exercises every code value
    rng = np.random.default_rng(5)
    n, k = 64, 1024
    for qtype, bb, offs in ((nat.Q4_K, 144, (0, 2)), (nat.Q6_K, 210, (208,)), (nat.Q8_0, 34, (0,)),
                            (nat.Q4_0, 18, (0,))):
        nb = n * k // (256 if bb in (144, 210) else 32)
        data = rng.integers(0, 256, (nb, bb)).astype(np.uint8)
        for off in offs:
            h = rng.integers(0x0001, 0x2400, nb).astype(np.uint16)   # subnormal .. 2^-6
            data[:, off:off + 2] = h.view(np.uint8).reshape(nb, 2)
        data = data.reshape(-1)
        x = x_of(k, batch, seed=qtype)
        assert_close(qmatvec(device, qtype, data, n, k, x), orc.matvec(qtype, data, n, k, x), TOL,
                     "type %d batch %d" % (qtype, batch))


@pytest.mark.parametrize("batch_path", [2, 3])   # dot2 kernel (1-2 columns), MFMA kernel (3-8)
def test_linearity_at_full_size(device, batch_path):
    n, k = 14336, 4096
    w = synth_weight(nat.Q4_K, n, k)
    x1, x2 = x_of(k, 1, 1), x_of(k, 1, 2)
    extra = [x_of(k, 1, 3)] * (batch_path - 2)
    ya = qmatvec(device, nat.Q4_K, w, n, k, np.vstack([x1, x2] + extra))
    yb = qmatvec(device, nat.Q4_K, w, n, k, np.vstack([x2, x1] + extra))
    # columns are computed independently of each other: swapping them swaps
    # the results bit for bit
    assert np.array_equal(ya[0], yb[1]) and np.array_equal(ya[1], yb[0])
    y12 = qmatvec(device, nat.Q4_K, w, n, k, np.vstack([x1 + x2, x1] + extra))
    assert_close(y12[0], ya[0] + ya[1], TOL)         # linearity
    y1 = qmatvec(device, nat.Q4_K, w, n, k, x1)      # single-column kernel
    if batch_path == 2:
        # one column of the two-column pass is the single-column result, bit for bit
        assert np.array_equal(ya[0], y1[0])
    else:
        assert_close(ya[0], y1[0], 1e-5)             # matrix-core and dot-product kernels agree


@pytest.mark.parametrize("dt", ["Q4_0", "Q8_0", "Q4_K", "Q6_K"])
def test_compute_ops_mirror(device, orc, dt):
    # Tensors carry the reference's DataType numbering (Q8_0 = 6, Q4_K = 10,
    # Q6_K = 12); ComputeOps translates it through aih_type_from_datatype, so
    # every format reaches its own kernels (a raw DataType.Q6_K would be read
    # as Q4_K blocks).
    ops = C.ComputeOps(device)
    dtype = C.DataType[dt]
    qtype = C.gguf_type(dtype)
    n, k = 300, 2048
    wq = synth_weight(qtype, n, k)
    w = C.Tensor.from_quantized(device, wq, k, n, dtype)
    assert w.dtype == dtype
    for m in (2, 12):     # the matvec (M <= 8) and the GEMM (M > 8)
        x = x_of(k, m)
        a = C.Tensor.from_data(device, x)
        y = ops.matmul_weights(a, w)
        assert y.shape == (m, n)
        assert_close(y.read(), orc.matvec(qtype, wq, n, k, x), TOL if m <= 8 else 1e-3)
        for t in (a, y):
            t.dispose()
    f = ops.dequantize(w)
    assert np.array_equal(f.read().reshape(-1), orc.dequantize(qtype, wq, n * k))
    with pytest.raises(ValueError):
        ops.matmul_weights(C.Tensor.from_data(device, x_of(k // 2, 1)), w)
    for t in (w, f):
        t.dispose()


def test_argument_errors(device):
    L = nat.lib()
    h = device.handle
    wb = upload(device, np.zeros(2304 * 4, np.uint8))
    xb = upload(device, np.zeros(4096, np.float32))
    yb = upload(device, np.zeros(64, np.float32))
    W, X, Y = wb.get_pointer(), xb.get_pointer(), yb.get_pointer()
    try:
        assert L.aih_qmatvec(h, nat.Q4_K, W, 4, 4096, X, 4096, Y, 4, 1) == nat.AIH_OK
        assert L.aih_qmatvec(h, nat.Q4_K, W, 0, 4096, X, 4096, Y, 4, 1) == nat.AIH_OK
        assert L.aih_qmatvec(h, nat.Q4_K, W, 4, 100, X, 4096, Y, 4, 1) == nat.AIH_E_INVALID
        assert L.aih_qmatvec(h, nat.Q4_K, W, 4, 4096, X, 4096, Y, 4, 9) == nat.AIH_E_INVALID
        assert L.aih_qmatvec(h, nat.Q4_K, W, 4, 4096, X, 100, Y, 4, 1) == nat.AIH_E_INVALID
        assert L.aih_qmatvec(h, nat.Q4_K, W + 8, 4, 4096, X, 4096, Y, 4, 1) == nat.AIH_E_INVALID
        assert L.aih_qmatvec(h, nat.F32, W, 4, 4096, X, 4096, Y, 4, 1) == nat.AIH_E_UNSUPPORTED
        assert L.aih_qmatvec(h, nat.Q4_K, W, 4, 256 * 260, X, 256 * 260, Y, 4, 1) == nat.AIH_E_LIMIT
        assert L.aih_qmatvec(h, nat.Q8_0, W, 4, 96, X, 96, Y, 4, 1) == nat.AIH_E_LIMIT
        device.synchronize()
    finally:
        for b in (wb, xb, yb):
            b.dispose()
