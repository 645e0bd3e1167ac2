"""Seeded random shapes through aih_matmul_weights_q, the seam that replaces
ComputeOps.MatMulWeights (ComputeOps.cs:275-309; TransformerBase.cs:254-290):
M from 1 to 400 routes to the one-or-two-column matvec, the 3..8-column
matrix-core matvec or the GEMM, for every format, with N off the tile
multiples and K any multiple of 64 (and of the format's block) up to 2048.
Each result against the oracle at its path's bar: 2e-5 for M <= 8
(fp32-equivalent arithmetic), 1e-3 for the GEMM (fp16 operands), and the
output buffer's bytes past M x N untouched.
"""
import numpy as np
import pytest

from aihost_amd import _native as nat
from aihost_amd import compute as C
from gpu_util import assert_close, synth_weight, upload

pytestmark = pytest.mark.gpu

TYPES = (nat.Q4_K, nat.Q6_K, nat.Q8_0, nat.Q4_0)


def cases(count=32, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        qtype = TYPES[i % 4]
        elems = 256 if qtype in (nat.Q4_K, nat.Q6_K) else 32
        # about half the cases take the GEMM (M > 8)
        m = int(rng.integers(9, 401)) if rng.random() < 0.5 else int(rng.integers(1, 9))
        # the kernels read 64-element units (K a multiple of 64, and of the
        # format's block)
        k = max(64, elems) * int(rng.integers(1, 2048 // max(64, elems) + 1))
        n = int(rng.integers(1, 2049))
        out.append((qtype, n, k, m, int(rng.integers(0, 2 ** 31))))
    return out


@pytest.mark.parametrize("qtype,n,k,m,seed", cases())
def test_matmul_weights_q_random_shape(device, orc, qtype, n, k, m, seed):
    w = synth_weight(qtype, n, k, seed=seed % 1000)
    x = C.fill_normal(seed % 997, m * k, 0.0, 1.0).reshape(m, k)
    pad = 64
    wb, xb = upload(device, w), upload(device, x)
    yb = device.create_buffer((m * n + pad) * 4)
    try:
        nat.check(nat.lib().aih_memset(device.handle, yb.get_pointer(), 0x7F, (m * n + pad) * 4), "memset")
        nat.check(nat.lib().aih_matmul_weights_q(device.handle, int(qtype), wb.get_pointer(), n, k,
                                                 xb.get_pointer(), m, yb.get_pointer()), "aih_matmul_weights_q")
        raw = yb.read_range(0, m * n + pad, np.float32)
    finally:
        for b in (wb, xb, yb):
            b.dispose()
    ref = orc.matvec(qtype, w, n, k, x, nthreads=8)
    assert_close(raw[:m * n].reshape(m, n), ref, 2e-5 if m <= 8 else 1e-3,
                 "type %d %dx%d M=%d" % (qtype, n, k, m))
    assert np.all(raw[m * n:].view(np.uint32) == 0x7F7F7F7F), "wrote past M x N"
