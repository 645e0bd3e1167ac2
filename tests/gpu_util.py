"""Helpers shared by the GPU tests (upload, call through the C ABI, compare)."""
import ctypes

import numpy as np

from aihost_amd import _native as nat
from aihost_amd import compute as C


def upload(device, arr):
    a = np.ascontiguousarray(arr)
    buf = device.create_buffer(max(16, a.nbytes))
    if a.nbytes:
        buf.write(a)
    return buf


def qmatvec(device, qtype, w_host, n, k, x_host, ldx=None, ldy=None):
    """Run aih_qmatvec on host inputs; returns Y[batch, ldy][:, :n]."""
    x_host = np.ascontiguousarray(np.atleast_2d(x_host), dtype=np.float32)
    batch = x_host.shape[0]
    ldx = ldx or k
    ldy = ldy or n
    xs = np.zeros((batch, ldx), dtype=np.float32)
    xs[:, :k] = x_host
    wb, xb = upload(device, w_host), upload(device, xs)
    yb = device.create_buffer(batch * ldy * 4)
    try:
        nat.check(nat.lib().aih_memset(device.handle, yb.get_pointer(), 0xFF, batch * ldy * 4), "memset")
        st = nat.lib().aih_qmatvec(device.handle, int(qtype), wb.get_pointer(), n, k, xb.get_pointer(), ldx,
                                   yb.get_pointer(), ldy, batch)
        nat.check(st, "aih_qmatvec")
        y = yb.read_range(0, batch * ldy, np.float32).reshape(batch, ldy)
    finally:
        for b in (wb, xb, yb):
            b.dispose()
    return y


def qgemm(device, qtype, w_host, n, k, x_host):
    x_host = np.ascontiguousarray(x_host, dtype=np.float32)
    m = x_host.shape[0]
    wb, xb = upload(device, w_host), upload(device, x_host)
    yb = device.create_buffer(m * n * 4)
    try:
        st = nat.lib().aih_qgemm(device.handle, int(qtype), wb.get_pointer(), n, k, xb.get_pointer(), m,
                                 yb.get_pointer())
        nat.check(st, "aih_qgemm")
        y = yb.read_range(0, m * n, np.float32).reshape(m, n)
    finally:
        for b in (wb, xb, yb):
            b.dispose()
    return y


def dequant(device, qtype, data, n, mode):
    qb = upload(device, data)
    ob = device.create_buffer(n * 4)
    try:
        nat.check(nat.lib().aih_dequantize(device.handle, int(qtype), qb.get_pointer(), ob.get_pointer(),
                                           ctypes.c_uint64(n), int(mode)), "aih_dequantize")
        return ob.read_range(0, n, np.float32)
    finally:
        qb.dispose()
        ob.dispose()


def assert_close(y, ref, tol=1e-3, what=""):
    """Normwise ||y - ref|| <= tol ||ref|| and max|y - ref| <= tol * max|ref|."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert y.shape == ref.shape
    assert np.all(np.isfinite(y)), what
    nrm = np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30)
    mx = np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30)
    assert nrm <= tol and mx <= tol, "%s normwise %.3g max %.3g" % (what, nrm, mx)
    return nrm, mx


def synth_weight(qtype, n, k, seed=42, std=0.02):
    w = C.fill_normal(seed, n * k, 0.0, std)
    return C.quantize(qtype, w, n, k)
