"""aih_matmul_weights_q_noalloc, the allocation-free variant of
aih_matmul_weights_q: the same kernels with their staging memory (the
3..8-column matvec's partial sums, the GEMM's fp16 copy of X) in one static
device buffer instead of the context workspace.

Bar: bit-identical to aih_matmul_weights_q on the same inputs (same kernels,
same split counts, sums in the same order), on two calls in a row, the second
with a smaller input (the buffer keeps the first call's contents); calls
that need more than AIH_NOALLOC_SCRATCH_BYTES are refused before anything
runs; the call records into a HIP graph on a context whose workspace never
grew, where the allocating GEMM cannot.
"""
import ctypes

import numpy as np
import pytest

from aihost_amd import _native as nat
from aihost_amd import compute as C
from gpu_util import upload

pytestmark = pytest.mark.gpu

SENTINEL = np.float32(np.nan)


def weights(qtype, n, k, seed):
    return C.quantize(qtype, C.fill_normal(seed, n * k, 0.0, 0.02), n, k)


def run(device, fn, qtype, wb, n, k, xb, m, yb):
    """Fill Y with NaN, call `fn`, return (status, Y)."""
    yb.write(np.full(m * n, SENTINEL, np.float32))
    st = getattr(nat.lib(), fn)(device.handle, int(qtype), wb.get_pointer(), n, k, xb.get_pointer(), m,
                                yb.get_pointer())
    device.synchronize()
    return st, yb.read_range(0, m * n, np.float32)


# (type, N, K, first M, second M): the 3..8-column matvec with split partials,
# the 1..2-column matvec (no staging), the GEMM (fp16 copy of X)
CASES = [(nat.Q6_K, 4096, 14336, 8, 3), (nat.Q4_K, 14336, 4096, 5, 4), (nat.Q8_0, 1024, 4096, 2, 1),
         (nat.Q4_K, 4096, 4096, 512, 40), (nat.Q6_K, 1024, 14336, 576, 9)]


@pytest.mark.parametrize("qtype,n,k,m1,m2", CASES)
def test_noalloc_equals_matmul_weights_q_on_two_calls(device, qtype, n, k, m1, m2):
    wb = upload(device, weights(qtype, n, k, 31))
    x = C.fill_normal(32, m1 * k, 0.0, 1.0)
    xb = upload(device, x)
    x2b = upload(device, C.fill_normal(33, m2 * k, 0.0, 1.0))
    yb = device.create_buffer(m1 * n * 4)
    try:
        # two allocation-free calls in a row, the second smaller
        st1, a1 = run(device, "aih_matmul_weights_q_noalloc", qtype, wb, n, k, xb, m1, yb)
        st2, a2 = run(device, "aih_matmul_weights_q_noalloc", qtype, wb, n, k, x2b, m2, yb)
        assert (st1, st2) == (nat.AIH_OK, nat.AIH_OK), (nat.strerror(st1), nat.strerror(st2))
        _, b1 = run(device, "aih_matmul_weights_q", qtype, wb, n, k, xb, m1, yb)
        _, b2 = run(device, "aih_matmul_weights_q", qtype, wb, n, k, x2b, m2, yb)
        assert np.all(np.isfinite(a1)) and np.all(np.isfinite(a2))
        assert np.array_equal(a1, b1) and np.array_equal(a2, b2)
        # and once more after the allocating calls: same result again
        _, a3 = run(device, "aih_matmul_weights_q_noalloc", qtype, wb, n, k, x2b, m2, yb)
        assert np.array_equal(a3, b2)
    finally:
        for b in (wb, xb, x2b, yb):
            b.dispose()


def test_noalloc_refuses_more_than_its_buffer(device):
    n, k = 256, 14336
    wb = upload(device, weights(nat.Q4_K, n, k, 34))
    xb = upload(device, C.fill_normal(35, 1024 * k, 0.0, 1.0))
    yb = device.create_buffer(1024 * n * 4)
    try:
        # the GEMM's fp16 X copy with its row exponents is mpad * (2 K + 4)
        # bytes (mpad = M rounded up to 32)
        for m in (577, 1024):
            assert (m + 31) // 32 * 32 * (2 * k + 4) > nat.NOALLOC_SCRATCH_BYTES
            st, y = run(device, "aih_matmul_weights_q_noalloc", nat.Q4_K, wb, n, k, xb, m, yb)
            assert st == nat.AIH_E_SCRATCH, nat.strerror(st)
            assert np.all(np.isnan(y))                  # nothing ran
        st, y = run(device, "aih_matmul_weights_q_noalloc", nat.Q4_K, wb, n, k, xb, 576, yb)
        assert st == nat.AIH_OK and np.all(np.isfinite(y))
        # invalid arguments are checked as in aih_matmul_weights_q
        L = nat.lib()
        assert L.aih_matmul_weights_q_noalloc(device.handle, 3, wb.get_pointer(), n, k, xb.get_pointer(), 4,
                                              yb.get_pointer()) == nat.AIH_E_UNSUPPORTED
        assert L.aih_matmul_weights_q_noalloc(device.handle, nat.Q4_K, wb.get_pointer(), n, 100,
                                              xb.get_pointer(), 4, yb.get_pointer()) == nat.AIH_E_INVALID
        assert L.aih_matmul_weights_q_noalloc(device.handle, nat.Q4_K, wb.get_pointer(), n, k, None, 4,
                                              yb.get_pointer()) == nat.AIH_E_INVALID
    finally:
        for b in (wb, xb, yb):
            b.dispose()


def test_noalloc_records_into_a_graph_on_a_fresh_context():
    """A fresh context has no workspace: the allocating GEMM cannot be
    recorded (AIH_E_LIMIT); the allocation-free one can, and every replay
    gives the eager result."""
    L = nat.lib()
    dev = C.HipComputeDevice(0)
    n, k, m, mb = 2048, 4096, 64, 6
    wb = upload(dev, weights(nat.Q4_K, n, k, 36))
    xb = upload(dev, C.fill_normal(37, m * k, 0.0, 1.0))
    yg, yv = dev.create_buffer(m * n * 4), dev.create_buffer(mb * n * 4)
    graph = None
    try:
        h = dev.handle
        nat.check(L.aih_capture_begin(h), "capture")
        st_alloc = L.aih_matmul_weights_q(h, nat.Q4_K, wb.get_pointer(), n, k, xb.get_pointer(), m,
                                          yg.get_pointer())
        st_g = L.aih_matmul_weights_q_noalloc(h, nat.Q4_K, wb.get_pointer(), n, k, xb.get_pointer(), m,
                                              yg.get_pointer())
        st_v = L.aih_matmul_weights_q_noalloc(h, nat.Q4_K, wb.get_pointer(), n, k, xb.get_pointer(), mb,
                                              yv.get_pointer())
        g = ctypes.c_void_p()
        nat.check(L.aih_capture_end(h, ctypes.byref(g)), "capture end")
        graph = g.value
        assert st_alloc == nat.AIH_E_LIMIT
        assert (st_g, st_v) == (nat.AIH_OK, nat.AIH_OK), (nat.strerror(st_g), nat.strerror(st_v))
        _, eg = run(dev, "aih_matmul_weights_q", nat.Q4_K, wb, n, k, xb, m, yg)
        _, ev = run(dev, "aih_matmul_weights_q", nat.Q4_K, wb, n, k, xb, mb, yv)
        for _ in range(3):
            yg.write(np.full(m * n, SENTINEL, np.float32))
            yv.write(np.full(mb * n, SENTINEL, np.float32))
            nat.check(L.aih_graph_launch(h, graph), "replay")
            dev.synchronize()
            assert np.array_equal(yg.read_range(0, m * n, np.float32), eg)
            assert np.array_equal(yv.read_range(0, mb * n, np.float32), ev)
            # eager work between replays
            run(dev, "aih_matmul_weights_q", nat.Q4_K, wb, n, k, xb, 3, yv)
    finally:
        if graph:
            L.aih_graph_destroy(graph)
        for b in (wb, xb, yg, yv):
            b.dispose()
        dev.dispose()
