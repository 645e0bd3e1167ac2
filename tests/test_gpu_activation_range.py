"""Parity across the activation range the reference accepts.

The reference multiplies fp32 activations by fp32 weights
(ComputeShaders.cs:93-129, TransformerBase.cs:454-456): any finite fp32 row is
a valid input.  The batch-1/2 matvec holds x as 22-bit fixed point per
64-element unit and the batch-3..8 matvec as fp16 hi/lo pairs per 32-element
group, each with a power of two from the unit's or group's maximum; the GEMM
rounds x to fp16 with a power of two per row (a row above 65504 or far below 1
keeps its 11 significant bits).  Inputs here:

- one outlier per 64-element unit, 10^3 .. 10^4 times the rest;
- rows (batch columns) scaled to 1e5 and to 1e-6, alternating, so that one
  32-row block of the GEMM operand holds both;
- magnitudes log-uniform over 2^-40 .. 2^20, random signs.

Every output row (a batch column, a GEMM row) is compared on its own with the
oracle (fp32 sequential sums over the reference-decoded weights) at the bars of
the other parity tests -- 2e-5 for the matvec, 1e-3 for the GEMM, normwise and
in the maximum -- with no inf or NaN.

Operand images written one 32-column block at a time (the gate|up GEMM's SiLU
epilogue and the attention operand, read by the next GEMM) are checked bit for
bit against the host's rounding of the separate operators' fp32 outputs at the
exponents the image format prescribes (a row or block whose maximum lies in
[2^-12, 2^15) unscaled, else scaled to put it in [2^14, 2^15)), before and
after the pass that gives each row a single exponent.
"""
import numpy as np
import pytest

from aihost_amd import _native as nat
from gpu_util import qgemm, qmatvec, synth_weight, upload

pytestmark = pytest.mark.gpu

EPS = 1e-5
KINDS = ("outlier", "rows_1e5_1e-6", "rows_1e-6_1e5", "loguniform")


def activations(kind, rows, k, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    if kind == "outlier":
        units = k // 64
        pos = rng.integers(0, 64, (rows, units)) + 64 * np.arange(units)
        mag = 10.0 ** rng.uniform(3.0, 4.0, (rows, units)) * rng.choice([-1.0, 1.0], (rows, units))
        x[np.arange(rows)[:, None], pos] = mag.astype(np.float32)
    elif kind.startswith("rows_"):
        a, b = (1e5, 1e-6) if kind == "rows_1e5_1e-6" else (1e-6, 1e5)
        x *= np.where(np.arange(rows) % 2 == 0, a, b).astype(np.float32)[:, None]
    elif kind == "loguniform":
        e = rng.uniform(-40.0, 20.0, (rows, k))
        x = (np.exp2(e) * rng.choice([-1.0, 1.0], (rows, k))).astype(np.float32)
    else:
        raise ValueError(kind)
    return x


def check_rows(y, ref, tol, what):
    """Each row on its own: ||y - ref|| <= tol ||ref|| and max|y - ref| <=
    tol max|ref|; returns the worst of each."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.all(np.isfinite(y)), "%s: non-finite output" % what
    d = y - ref
    nrm = np.linalg.norm(d, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-300)
    mx = np.max(np.abs(d), axis=1) / np.maximum(np.max(np.abs(ref), axis=1), 1e-300)
    bad = np.nonzero((nrm > tol) | (mx > tol))[0]
    assert bad.size == 0, "%s: rows %s normwise %s max %s" % (what, bad[:8], nrm[bad[:8]], mx[bad[:8]])
    return float(nrm.max()), float(mx.max())


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("qtype,n,k,batch", [
    (nat.Q4_K, 4096, 4096, 1), (nat.Q4_K, 4096, 4096, 2),
    (nat.Q6_K, 1024, 14336, 5), (nat.Q6_K, 1024, 14336, 8),
    (nat.Q8_0, 2048, 4096, 1), (nat.Q8_0, 2048, 4096, 5),
    (nat.Q4_0, 2048, 4096, 2), (nat.Q4_0, 2048, 4096, 8),
])
def test_matvec_activation_range(device, orc, qtype, n, k, batch, kind):
    w = synth_weight(qtype, n, k, seed=n + k + batch)
    x = activations(kind, batch, k, seed=batch * 100 + KINDS.index(kind))
    y = qmatvec(device, qtype, w, n, k, x)[:, :n]
    ref = orc.matvec(qtype, w, n, k, x, nthreads=8)
    r64 = orc.matvec(qtype, w, n, k, x, nthreads=8, f64=True)
    nrm, mx = check_rows(y, ref, 2e-5, "type %d %dx%d b%d %s" % (qtype, n, k, batch, kind))
    o_nrm = max(np.linalg.norm(ref[b] - r64[b]) / np.linalg.norm(r64[b]) for b in range(batch))
    print("type=%d b%d %s: normwise %.3g max %.3g (oracle vs fp64 %.3g)" % (qtype, batch, kind, nrm, mx, o_nrm))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("qtype,n,k,m", [
    (nat.Q4_K, 4096, 4096, 512),      # the prefill workload (128-row tiles)
    (nat.Q6_K, 1024, 4096, 40),
    (nat.Q8_0, 640, 2048, 40),
    (nat.Q4_0, 6400, 1024, 300),      # 256-row tiles on a 256-CU device
])
def test_gemm_activation_range(device, orc, qtype, n, k, m, kind):
    w = synth_weight(qtype, n, k, seed=n + k + m)
    x = activations(kind, m, k, seed=m * 100 + KINDS.index(kind))
    y = qgemm(device, qtype, w, n, k, x)
    ref = orc.matvec(qtype, w, n, k, x, nthreads=16)
    nrm, mx = check_rows(y, ref, 1e-3, "type %d %dx%d M=%d %s" % (qtype, n, k, m, kind))
    print("type=%d M=%d %s: normwise %.3g max %.3g" % (qtype, m, kind, nrm, mx))


def test_gemm_split_k_rows_scaled(device, orc):
    """The down-projection shape, whose GEMM splits K over workgroups on a
    256-CU device: each split's partial sums carry the row exponents undone."""
    n, k, m = 4096, 14336, 512
    w = synth_weight(nat.Q4_K, n, k, seed=3)
    x = activations("rows_1e5_1e-6", m, k, seed=9)
    y = qgemm(device, nat.Q4_K, w, n, k, x)
    check_rows(y, orc.matvec(nat.Q4_K, w, n, k, x, nthreads=16), 1e-3, "split K")


# ---------------------------------------------------------------- operand images

def _exp_of(mx):
    """The image format's exponent for a maximum magnitude mx (array):
    0 inside [2^-12, 2^15) and for zero / non-finite, else the power of two
    that puts mx in [2^14, 2^15)."""
    mx = np.asarray(mx, np.float64)
    _, e = np.frexp(mx)
    out = 15 - e
    keep = (mx == 0) | ~np.isfinite(mx) | ((mx >= 2.0 ** -12) & (mx < 2.0 ** 15))
    return np.where(keep, 0, out).astype(np.int64)


def _block_exps(v):
    """Block exponents of rows v (M x K fp32) per 32-column block, as int8:
    -128 marks an all-zero block, the others are clamped to 127."""
    m, k = v.shape
    mx = np.max(np.abs(v.reshape(m, k // 32, 32)), axis=2)
    e = np.minimum(_exp_of(mx), 127)
    return np.where(mx == 0, -128, e)


def _slots(mpad, k):
    """Half index of element (m, k) of the fragment-order image."""
    m = np.arange(mpad)[:, None]
    kk = np.arange(k)[None, :]
    return (((m // 32) * (k // 16) + kk // 16) * 64 + m % 32 + 32 * ((kk // 8) % 2)) * 8 + kk % 8


def _read_image(device, buf, m, k):
    mpad = (m + 31) // 32 * 32
    raw = np.empty(nat.operand_bytes(m, k), np.uint8)
    nat.check(nat.lib().aih_memcpy_d2h(device.handle, raw.ctypes.data, buf.get_pointer(), raw.nbytes), "d2h")
    halves = raw[:2 * mpad * k].view(np.float16)
    vals = halves[_slots(mpad, k).ravel()].reshape(mpad, k)
    E = raw[2 * mpad * k:2 * mpad * k + 4 * mpad].view(np.int32)
    d = raw[2 * mpad * k + 4 * mpad:].view(np.int8).reshape(mpad, k // 32)
    return vals, E.copy(), d.copy()


def _write_image(device, vals, E, d, m, k):
    """An operand image buffer holding rows `vals` (mpad x k fp16), row
    exponents E and block exponents d (the layout _read_image reads)."""
    mpad = (m + 31) // 32 * 32
    raw = np.zeros(nat.operand_bytes(m, k), np.uint8)
    halves = raw[:2 * mpad * k].view(np.float16)
    halves[_slots(mpad, k).ravel()] = vals.reshape(-1)
    raw[2 * mpad * k:2 * mpad * k + 4 * mpad] = np.ascontiguousarray(E, np.int32).view(np.uint8)
    raw[2 * mpad * k + 4 * mpad:] = np.ascontiguousarray(d, np.int8).reshape(-1).view(np.uint8)
    return upload(device, raw)


def _gemm_from_image(device, qtype, w_buf, n, k, img, m):
    y = device.create_buffer(m * n * 4)
    try:
        nat.check(nat.lib().aih_qgemm_fused(device.handle, qtype, w_buf.get_pointer(), n, k, img.get_pointer(), None,
                                            EPS, m, nat.PRE_F16_OPERAND, nat.POST_STORE, y.get_pointer()), "gemm")
        return y.read_range(0, m * n, np.float32).reshape(m, n)
    finally:
        y.dispose()


def _expected_block_image(v, mpad):
    """Values of rows v rounded to fp16 at their block exponents (rows past
    M zero), and those exponents."""
    m, k = v.shape
    full = np.zeros((mpad, k), np.float32)
    full[:m] = v
    d = _block_exps(full)
    e = np.repeat(np.where(d == -128, 0, d), 32, axis=1)
    return np.ldexp(full, e.astype(np.int32)).astype(np.float16), d


def _expected_after_fixup(vals, d):
    """The single-exponent image: per row D = the smallest block exponent
    (all-zero blocks aside); each block of exponent d rescaled by 2^(D - d) in
    fp32 and rounded to fp16 once; E = D."""
    live = np.where(d == -128, 127, d).astype(np.int64)
    D = np.min(live, axis=1)
    odd = np.any((d != 0) & (d != -128), axis=1)
    D = np.where(odd, D, 0)
    shift = np.where((d == -128) | ~odd[:, None], 0, D[:, None] - d)
    f = np.repeat(np.ldexp(np.float32(1.0), shift.astype(np.int32)).astype(np.float32), 32, axis=1)
    out = (vals.astype(np.float32) * f).astype(np.float16)
    # rows already at one exponent are left as they are (block exponents too)
    return out, D.astype(np.int32), np.where(odd[:, None], 0, d).astype(np.int8)


@pytest.mark.parametrize("scale", [1.0, 1e3, 1e-4])
def test_silu_operand_image_and_down_gemm(device, orc, scale):
    """gate|up GEMM with the SiLU-pairs fp16 epilogue, then the down GEMM
    reading that image: the image holds SiLU(gate)*up of the separate
    operators (aih_rmsnorm, aih_qgemm, aih_silu_mul_pairs) rounded at its block
    exponents, bit for bit; the down GEMM first gives every row one exponent
    (checked bit for bit, and its output is bit for bit that of the same GEMM
    on the host's one-exponent image) and its output matches the oracle on
    the separate path's fp32 operand.  Norm weights scaled by 1e3 put the SiLU output far
    above 65504, by 1e-4 far below 2^-12."""
    L, h = nat.lib(), device.handle
    d, f, m = 512, 1024, 100
    mpad = (m + 31) // 32 * 32
    rng = np.random.default_rng(int(scale * 7) + 3)
    w_gu = synth_weight(nat.Q4_K, 2 * f, d, seed=21)
    w_dn = synth_weight(nat.Q6_K, d, f, seed=22)
    x = rng.standard_normal((m, d)).astype(np.float32)
    nw = ((1.0 + 0.1 * rng.standard_normal(d)) * scale).astype(np.float32)
    bufs = [upload(device, a) for a in (w_gu, w_dn, x, nw)]
    wgu, wdn, xb, nb = bufs
    xn, g, u = (device.create_buffer(n) for n in (m * d * 4, m * 2 * f * 4, m * f * 4))
    img = device.create_buffer(nat.operand_bytes(m, f))
    y = device.create_buffer(m * d * 4)
    try:
        nat.check(L.aih_rmsnorm(h, xb.get_pointer(), nb.get_pointer(), xn.get_pointer(), m, d, EPS), "rmsnorm")
        nat.check(L.aih_qgemm(h, nat.Q4_K, wgu.get_pointer(), 2 * f, d, xn.get_pointer(), m, g.get_pointer()), "gu")
        nat.check(L.aih_silu_mul_pairs(h, g.get_pointer(), u.get_pointer(), m, f), "silu pairs")
        nat.check(L.aih_qgemm_fused(h, nat.Q4_K, wgu.get_pointer(), 2 * f, d, xb.get_pointer(), nb.get_pointer(),
                                    EPS, m, nat.PRE_RMSNORM, nat.POST_SILU_PAIRS_F16, img.get_pointer()), "gu fused")
        uh = u.read_range(0, m * f, np.float32).reshape(m, f)
        assert np.all(np.isfinite(uh))
        vals, E, dd = _read_image(device, img, m, f)
        want, want_d = _expected_block_image(uh, mpad)
        assert np.array_equal(dd, want_d)
        assert np.array_equal(E, np.zeros(mpad, np.int32))
        assert np.array_equal(vals.view(np.uint16), want.view(np.uint16))
        if scale != 1.0:
            assert np.any((dd != 0) & (dd != -128)), "the scaled rows must leave the unscaled window"
        nat.check(L.aih_qgemm_fused(h, nat.Q6_K, wdn.get_pointer(), d, f, img.get_pointer(), None, EPS, m,
                                    nat.PRE_F16_OPERAND, nat.POST_STORE, y.get_pointer()), "down fused")
        vals2, E2, dd2 = _read_image(device, img, m, f)
        want2, wantE, want_d2 = _expected_after_fixup(vals, dd)
        assert np.array_equal(dd2, want_d2)
        assert np.array_equal(E2, wantE)
        assert np.array_equal(vals2.view(np.uint16), want2.view(np.uint16))
        yh = y.read_range(0, m * d, np.float32).reshape(m, d)
        fixed = _write_image(device, want2, wantE, want_d2, m, f)
        try:
            y_fixed = _gemm_from_image(device, nat.Q6_K, wdn, d, f, fixed, m)
        finally:
            fixed.dispose()
        assert np.array_equal(yh.view(np.uint32), y_fixed.view(np.uint32))
        nrm, mx = check_rows(yh, orc.matvec(nat.Q6_K, w_dn, d, f, uh, nthreads=8), 1e-3, "down, scale %g" % scale)
        print("scale %g: down GEMM from the image normwise %.3g max %.3g" % (scale, nrm, mx))
    finally:
        for b in bufs + [xn, g, u, img, y]:
            b.dispose()


@pytest.mark.parametrize("vscale", [1e6, 1e-8])
def test_attention_operand_image_wide_range(device, orc, vscale):
    """aih_attention_operand with V rows scaled far outside fp16's range: the
    image is the fp32 output of aih_attention_strided rounded at its block
    exponents, bit for bit, and the W_o GEMM from it matches the oracle on
    that fp32 output."""
    L, h = nat.lib(), device.handle
    n_heads, n_kv, hd, max_len, n_q = 8, 2, 128, 160, 70
    qd, kvd = n_heads * hd, n_kv * hd
    ld = qd + 2 * kvd
    mpad = (n_q + 31) // 32 * 32
    rng = np.random.default_rng(5)
    qkv = rng.standard_normal((n_q, ld)).astype(np.float32)
    kc = rng.standard_normal((max_len, kvd)).astype(np.float32)
    vc = (rng.standard_normal((max_len, kvd)) * vscale).astype(np.float32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    n_out = 256
    w = synth_weight(nat.Q4_K, n_out, qd, seed=6)
    bufs = [upload(device, a) for a in (qkv, kc, vc, w)]
    o = device.create_buffer(n_q * qd * 4)
    img = device.create_buffer(nat.operand_bytes(n_q, qd))
    y = device.create_buffer(n_q * n_out * 4)
    sf = int(L.aih_attention_scratch_floats(n_heads, max_len))
    sb = device.create_buffer(sf * 4)
    try:
        qs, kb, vb, wb = bufs
        nat.check(L.aih_attention_strided(h, qs.get_pointer(), ld, kb.get_pointer(), vb.get_pointer(),
                                          o.get_pointer(), n_q, n_heads, n_kv, hd, 30, None, max_len, scale,
                                          sb.get_pointer(), sf), "strided")
        nat.check(L.aih_attention_operand(h, qs.get_pointer(), ld, kb.get_pointer(), vb.get_pointer(),
                                          img.get_pointer(), n_q, n_heads, n_kv, hd, 30, None, max_len, scale),
                  "operand")
        out = o.read_range(0, n_q * qd, np.float32).reshape(n_q, qd)
        assert np.all(np.isfinite(out))
        vals, E, dd = _read_image(device, img, n_q, qd)
        want, want_d = _expected_block_image(out, mpad)
        assert np.array_equal(dd, want_d)
        assert np.array_equal(E, np.zeros(mpad, np.int32))
        assert np.array_equal(vals.view(np.uint16), want.view(np.uint16))
        assert np.any((dd != 0) & (dd != -128))
        nat.check(L.aih_qgemm_fused(h, nat.Q4_K, wb.get_pointer(), n_out, qd, img.get_pointer(), None, EPS, n_q,
                                    nat.PRE_F16_OPERAND, nat.POST_STORE, y.get_pointer()), "W_o")
        yh = y.read_range(0, n_q * n_out, np.float32).reshape(n_q, n_out)
        # bit for bit the GEMM of the host's one-exponent image
        want2, wantE, want_d2 = _expected_after_fixup(vals, dd)
        fixed = _write_image(device, want2, wantE, want_d2, n_q, qd)
        try:
            y_fixed = _gemm_from_image(device, nat.Q4_K, wb, n_out, qd, fixed, n_q)
        finally:
            fixed.dispose()
        assert np.array_equal(yh.view(np.uint32), y_fixed.view(np.uint32))
        check_rows(yh, orc.matvec(nat.Q4_K, w, n_out, qd, out, nthreads=8), 1e-3, "W_o, V x %g" % vscale)
    finally:
        for b in bufs + [o, img, y, sb]:
            b.dispose()


def test_fused_rmsnorm_operand_rows_outside_fp16(device, orc):
    """The RMSNorm operand writer (aih_qgemm_fused, AIH_PRE_RMSNORM) with norm
    weights of 1e6: rows far above 65504 reach the GEMM scaled, with the same
    bits as aih_rmsnorm followed by aih_qgemm."""
    L, h = nat.lib(), device.handle
    n, k, m = 512, 2048, 70
    rng = np.random.default_rng(8)
    w = synth_weight(nat.Q4_K, n, k, seed=8)
    x = rng.standard_normal((m, k)).astype(np.float32)
    nw = (rng.standard_normal(k) * 1e6).astype(np.float32)
    bufs = [upload(device, a) for a in (w, x, nw)]
    wb, xb, nb = bufs
    xn, y1, y2 = device.create_buffer(m * k * 4), device.create_buffer(m * n * 4), device.create_buffer(m * n * 4)
    try:
        nat.check(L.aih_rmsnorm(h, xb.get_pointer(), nb.get_pointer(), xn.get_pointer(), m, k, EPS), "rmsnorm")
        nat.check(L.aih_qgemm(h, nat.Q4_K, wb.get_pointer(), n, k, xn.get_pointer(), m, y1.get_pointer()), "qgemm")
        nat.check(L.aih_qgemm_fused(h, nat.Q4_K, wb.get_pointer(), n, k, xb.get_pointer(), nb.get_pointer(), EPS, m,
                                    nat.PRE_RMSNORM, nat.POST_STORE, y2.get_pointer()), "fused")
        a = y1.read_range(0, m * n, np.float32)
        b = y2.read_range(0, m * n, np.float32)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        xnh = xn.read_range(0, m * k, np.float32).reshape(m, k)
        assert np.max(np.abs(xnh)) > 65504.0
        check_rows(b.reshape(m, n), orc.matvec(nat.Q4_K, w, n, k, xnh, nthreads=8), 1e-3, "rmsnorm x 1e6")
    finally:
        for bb in bufs + [xn, y1, y2]:
            bb.dispose()
