"""Fused prefill steps against the separate operators they replace, bit for bit:

- aih_qgemm_fused with each prologue (RMSNorm, SiLU*up, SiLU of gate/up pairs)
  and epilogue (residual add) vs aih_rmsnorm / aih_silu_mul / aih_silu_mul_pairs,
  aih_qgemm and aih_add, on the 128-row and the 256-row GEMM tiles, with a
  partial last row block (rows past M are zero in the operand);
- aih_attention_strided reading the query block of a Q|K|V row in place vs
  aih_attention on a contiguous copy;
- aih_attention_operand vs aih_attention_strided's fp32 output rounded into
  the GEMM operand layout, and the W_o GEMM from either;
- aih_qgemm_qkv_rope vs aih_qgemm_fused + aih_rope_qkv (queries and caches);
- a decoder prefill through the fused layer vs the same prompt through the
  separate operators: logits and K/V caches identical.
"""
import numpy as np
import pytest

from aihost_amd import _native as nat
from aihost_amd import llama
from gpu_util import synth_weight, upload

pytestmark = pytest.mark.gpu

EPS = 1e-5


def _read(buf, n):
    return buf.read_range(0, n, np.float32)


def _check(st, what):
    nat.check(st, what)


def _read_ptr(device, ptr, n):
    out = np.empty(n, np.float32)
    nat.check(nat.lib().aih_memcpy_d2h(device.handle, out.ctypes.data, ptr, out.nbytes), "aih_memcpy_d2h")
    return out


def _separate(device, qtype, wb, n, k, m, pre, post, xb, x2b, y0):
    """The operators aih_qgemm_fused replaces, one after the other."""
    L, h = nat.lib(), device.handle
    opb = device.create_buffer(m * k * 4)
    yb = upload(device, y0)
    tmp = device.create_buffer(m * n * 4)
    try:
        if pre == nat.PRE_NONE:
            src = xb
        elif pre == nat.PRE_RMSNORM:
            _check(L.aih_rmsnorm(h, xb.get_pointer(), x2b.get_pointer(), opb.get_pointer(), m, k, EPS), "rmsnorm")
            src = opb
        elif pre == nat.PRE_SILU_MUL:
            _check(L.aih_silu_mul(h, xb.get_pointer(), x2b.get_pointer(), opb.get_pointer(), m * k), "silu_mul")
            src = opb
        else:
            _check(L.aih_silu_mul_pairs(h, xb.get_pointer(), opb.get_pointer(), m, k), "silu_mul_pairs")
            src = opb
        if post == nat.POST_STORE:
            _check(L.aih_qgemm(h, qtype, wb.get_pointer(), n, k, src.get_pointer(), m, yb.get_pointer()), "qgemm")
        else:
            _check(L.aih_qgemm(h, qtype, wb.get_pointer(), n, k, src.get_pointer(), m, tmp.get_pointer()), "qgemm")
            _check(L.aih_add(h, yb.get_pointer(), tmp.get_pointer(), yb.get_pointer(), m * n), "add")
        return _read(yb, m * n)
    finally:
        for b in (opb, yb, tmp):
            b.dispose()


def _fused(device, qtype, wb, n, k, m, pre, post, xb, x2b, y0):
    yb = upload(device, y0)
    try:
        _check(nat.lib().aih_qgemm_fused(device.handle, qtype, wb.get_pointer(), n, k, xb.get_pointer(),
                                         x2b.get_pointer() if x2b is not None else None, EPS, m, pre, post,
                                         yb.get_pointer()), "aih_qgemm_fused")
        return _read(yb, m * n)
    finally:
        yb.dispose()


MODES = [(nat.PRE_RMSNORM, nat.POST_STORE), (nat.PRE_NONE, nat.POST_ACCUMULATE),
         (nat.PRE_SILU_PAIRS, nat.POST_ACCUMULATE), (nat.PRE_SILU_MUL, nat.POST_STORE),
         (nat.PRE_RMSNORM, nat.POST_ACCUMULATE), (nat.PRE_NONE, nat.POST_STORE)]


# (Q4_K, 6400, 1024, 300) takes the 256-row tiles on a 256-CU device, and
# (Q4_K, 1024, 14336, 300) the 512-row tiles split over K (both paths split)
@pytest.mark.parametrize("qtype,n,k,m", [(nat.Q4_K, 192, 512, 40), (nat.Q6_K, 100, 768, 77),
                                         (nat.Q8_0, 70, 320, 9), (nat.Q4_K, 6400, 1024, 300),
                                         (nat.Q4_K, 1024, 14336, 300)])
def test_qgemm_fused_equals_separate_operators(device, qtype, n, k, m):
    # the tiling each case is there for, on a 256-CU device (elsewhere the
    # equality is checked on whatever tiling the device's CU count selects)
    want = {(6400, 1024, 300): (256, 1), (1024, 14336, 300): (512, 8)}.get((n, k, m))
    if want and device.info().compute_units == 256:
        assert nat.qgemm_plan(device.handle, n, k, m) == want
    rng = np.random.default_rng(n + k + m)
    w = synth_weight(qtype, n, k, seed=k)
    wb = upload(device, w)
    try:
        for pre, post in MODES:
            xw = 2 * k if pre == nat.PRE_SILU_PAIRS else k
            x = rng.standard_normal((m, xw)).astype(np.float32)
            x2 = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32) if pre == nat.PRE_RMSNORM else \
                rng.standard_normal((m, k)).astype(np.float32)
            y0 = rng.standard_normal((m, n)).astype(np.float32)
            xb, x2b = upload(device, x), upload(device, x2)
            try:
                x2_arg = x2b if pre in (nat.PRE_RMSNORM, nat.PRE_SILU_MUL) else None
                ref = _separate(device, qtype, wb, n, k, m, pre, post, xb, x2b, y0)
                got = _fused(device, qtype, wb, n, k, m, pre, post, xb, x2_arg, y0)
                assert np.isfinite(ref).all()
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
                    "type %d %dx%d M=%d pre %d post %d: %d of %d differ" % (
                        qtype, n, k, m, pre, post, int(np.sum(got != ref)), got.size)
            finally:
                xb.dispose()
                x2b.dispose()
    finally:
        wb.dispose()


# gate|up W of 2F rows (K = d), down W of d rows (K = F); (1024, 3072, 300)
# takes the 256-row tiles for gate|up on a 256-CU device, (512, 128, 40) the
# 128-row tiles
@pytest.mark.parametrize("d,f,m,qt_down", [(512, 128, 40, nat.Q8_0), (1024, 3072, 300, nat.Q4_K)])
def test_silu_pairs_operand_chain_equals_separate_operators(device, d, f, m, qt_down):
    L, h = nat.lib(), device.handle
    rng = np.random.default_rng(d + f + m)
    w_gu = synth_weight(nat.Q4_K, 2 * f, d, seed=d)
    w_dn = synth_weight(qt_down, d, f, seed=f)
    x = rng.standard_normal((m, d)).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    y0 = rng.standard_normal((m, d)).astype(np.float32)
    bufs = [upload(device, a) for a in (w_gu, w_dn, x, nw)]
    wgu, wdn, xb, nb = bufs
    xn, g, u, t = (device.create_buffer(n) for n in (m * d * 4, m * 2 * f * 4, m * f * 4, m * d * 4))
    ya, yb = upload(device, y0), upload(device, y0)
    try:
        _check(L.aih_rmsnorm(h, xb.get_pointer(), nb.get_pointer(), xn.get_pointer(), m, d, EPS), "rmsnorm")
        _check(L.aih_qgemm(h, nat.Q4_K, wgu.get_pointer(), 2 * f, d, xn.get_pointer(), m, g.get_pointer()), "gu")
        _check(L.aih_silu_mul_pairs(h, g.get_pointer(), u.get_pointer(), m, f), "silu pairs")
        _check(L.aih_qgemm(h, qt_down, wdn.get_pointer(), d, f, u.get_pointer(), m, t.get_pointer()), "down")
        _check(L.aih_add(h, ya.get_pointer(), t.get_pointer(), ya.get_pointer(), m * d), "add")
        # g (m x 2f floats) holds the operand image (mpad x 2f bytes)
        _check(L.aih_qgemm_fused(h, nat.Q4_K, wgu.get_pointer(), 2 * f, d, xb.get_pointer(), nb.get_pointer(), EPS,
                                 m, nat.PRE_RMSNORM, nat.POST_SILU_PAIRS_F16, g.get_pointer()), "gu fused")
        _check(L.aih_qgemm_fused(h, qt_down, wdn.get_pointer(), d, f, g.get_pointer(), None, EPS, m,
                                 nat.PRE_F16_OPERAND, nat.POST_ACCUMULATE, yb.get_pointer()), "down fused")
        ref, got = _read(ya, m * d), _read(yb, m * d)
        assert np.isfinite(ref).all()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "%d of %d differ" % (
            int(np.sum(got != ref)), got.size)
    finally:
        for b in bufs + [xn, g, u, t, ya, yb]:
            b.dispose()


def test_qgemm_fused_argument_errors(device):
    L, h = nat.lib(), device.handle
    n, k, m = 64, 256, 16
    wb = upload(device, synth_weight(nat.Q4_K, n, k))
    xb = device.create_buffer(m * 2 * k * 4)
    yb = device.create_buffer(m * n * 4)
    try:
        w, x, y = wb.get_pointer(), xb.get_pointer(), yb.get_pointer()
        assert L.aih_qgemm_fused(h, nat.Q4_K, w, n, k, x, None, EPS, m, nat.PRE_RMSNORM, 0, y) == nat.AIH_E_INVALID
        assert L.aih_qgemm_fused(h, nat.Q4_K, w, n, k, x, None, EPS, m, nat.PRE_SILU_MUL, 0, y) == nat.AIH_E_INVALID
        assert L.aih_qgemm_fused(h, nat.Q4_K, w, n, k, x, None, EPS, m, 0, nat.POST_SILU_PAIRS, y) == \
            nat.AIH_E_INVALID
        assert L.aih_qgemm_fused(h, nat.Q4_K, w, n, k, x + 4, None, EPS, m, 0, 0, y) == nat.AIH_E_INVALID
        assert L.aih_qgemm_fused(h, nat.F32, w, n, k, x, None, EPS, m, 0, 0, y) == nat.AIH_E_UNSUPPORTED
        # K a whole number of Q8_0 blocks but not of 64-element GEMM steps
        assert L.aih_qgemm_fused(h, nat.Q8_0, w, n, 96, x, None, EPS, m, 0, 0, y) == nat.AIH_E_LIMIT
        assert L.aih_qgemm_fused(h, nat.Q4_K, w, n, k, x, None, EPS, 0, nat.PRE_SILU_PAIRS, 0, y) == nat.AIH_OK
        assert L.aih_qgemm_fused(h, nat.Q4_K, w, n, k, x, None, EPS, m, 5, 0, y) == nat.AIH_E_INVALID
        assert L.aih_qgemm_fused(h, nat.Q4_K, w, n, k, x, None, EPS, m, 0, 4, y) == nat.AIH_E_INVALID
        # the SiLU-pairs operand needs N a multiple of 128
        assert L.aih_qgemm_fused(h, nat.Q4_K, w, n, k, x, None, EPS, m, 0, nat.POST_SILU_PAIRS_F16, y) == \
            nat.AIH_E_INVALID
    finally:
        for b in (wb, xb, yb):
            b.dispose()


# (n_heads, n_kv_heads, K, M, start, device position, table rows, cache rows, pre, type): the 128-row and
# wider tiles, a device position, and positions past the cache (no K/V store) and past the table (queries
# left unrotated, nothing stored)
QKV_CASES = [(4, 2, 256, 40, 0, None, 64, 64, nat.PRE_RMSNORM, nat.Q4_K),
             (8, 2, 512, 300, 5, None, 400, 400, nat.PRE_NONE, nat.Q6_K),
             (32, 8, 4096, 512, 0, 3, 640, 640, nat.PRE_RMSNORM, nat.Q4_K),
             (4, 2, 256, 70, 0, 40, 100, 80, nat.PRE_RMSNORM, nat.Q8_0)]


@pytest.mark.parametrize("nh,nkv,k,m,start,dpos,trows,crows,pre,qtype", QKV_CASES)
def test_qkv_rope_gemm_equals_gemm_then_rope(device, nh, nkv, k, m, start, dpos, trows, crows, pre, qtype):
    """aih_qgemm_qkv_rope against aih_qgemm_fused (store) + aih_rope_qkv: the
    rotated queries and both caches bit for bit; the key and value columns of
    its Q are left as they were."""
    L, h = nat.lib(), device.handle
    hd = 128
    qd, kvd = nh * hd, nkv * hd
    n = qd + 2 * kvd
    rng = np.random.default_rng(nh + k + m)
    w = synth_weight(qtype, n, k, seed=k + 1)
    x = rng.standard_normal((m, k)).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    cache0 = rng.standard_normal((crows, kvd)).astype(np.float32)
    q0 = np.full((m, n), 7.0, np.float32)
    bufs = [upload(device, a) for a in (w, x, nw, cache0, cache0, cache0, cache0, q0, q0)]
    wb, xb, nb, ka, va, kb, vb, qa, qb = bufs
    tb = device.create_buffer(trows * hd * 4)
    pb = upload(device, np.array([dpos if dpos is not None else 0], np.int32))
    try:
        _check(L.aih_rope_table(h, tb.get_pointer(), trows, hd, 10000.0), "rope table")
        pos = pb.get_pointer() if dpos is not None else None
        x2 = nb.get_pointer() if pre == nat.PRE_RMSNORM else None
        _check(L.aih_qgemm_fused(h, qtype, wb.get_pointer(), n, k, xb.get_pointer(), x2, EPS, m, pre,
                                 nat.POST_STORE, qa.get_pointer()), "qgemm_fused")
        qp = qa.get_pointer()
        _check(L.aih_rope_qkv(h, qp, n, qp + qd * 4, n, qp + (qd + kvd) * 4, n, ka.get_pointer(), va.get_pointer(), m,
                              nh, nkv, hd, start, pos, tb.get_pointer(), trows, crows), "rope_qkv")
        _check(L.aih_qgemm_qkv_rope(h, qtype, wb.get_pointer(), k, xb.get_pointer(), x2, EPS, m, pre,
                                    qb.get_pointer(), kb.get_pointer(), vb.get_pointer(), nh, nkv, hd, start, pos,
                                    tb.get_pointer(), trows, crows), "qgemm_qkv_rope")
        qa_h, qb_h = _read(qa, m * n).reshape(m, n), _read(qb, m * n).reshape(m, n)
        assert np.isfinite(qa_h).all()
        assert np.array_equal(qb_h[:, :qd].view(np.uint32), qa_h[:, :qd].view(np.uint32)), \
            "%d of %d queries differ" % (int(np.sum(qb_h[:, :qd] != qa_h[:, :qd])), m * qd)
        assert np.all(qb_h[:, qd:] == 7.0)
        for a_, b_, what in ((ka, kb, "K"), (va, vb, "V")):
            ca, cb = _read(a_, crows * kvd), _read(b_, crows * kvd)
            assert np.array_equal(cb.view(np.uint32), ca.view(np.uint32)), "%s cache: %d differ" % (
                what, int(np.sum(ca != cb)))
        p0 = start + (dpos or 0)
        stored = [r for r in range(m) if 0 <= p0 + r < min(trows, crows)]
        if stored:
            assert not np.array_equal(_read(kb, crows * kvd).reshape(crows, kvd)[p0 + stored[0]],
                                      cache0[p0 + stored[0]]), "row %d was not stored" % (p0 + stored[0])
    finally:
        for b_ in bufs + [tb, pb]:
            b_.dispose()


def test_qkv_rope_gemm_argument_errors(device):
    L, h = nat.lib(), device.handle
    wb = upload(device, synth_weight(nat.Q4_K, 1024, 256))
    xb = device.create_buffer(16 * 1024 * 4)
    try:
        w, x = wb.get_pointer(), xb.get_pointer()
        f = L.aih_qgemm_qkv_rope
        # head_dim 48: a 32-column block could hold the end of the queries
        assert f(h, nat.Q4_K, w, 256, x, None, EPS, 8, 0, x, x, x, 8, 4, 48, 0, None, x, 64, 64) == \
            nat.AIH_E_UNSUPPORTED
        assert f(h, nat.Q4_K, w, 256, x, None, EPS, 8, nat.PRE_SILU_MUL, x, x, x, 4, 2, 128, 0, None, x, 64, 64) == \
            nat.AIH_E_INVALID
        assert f(h, nat.Q4_K, w, 256, x, None, EPS, 8, nat.PRE_RMSNORM, x, x, x, 4, 2, 128, 0, None, x, 64, 64) == \
            nat.AIH_E_INVALID                                            # RMSNorm without weights
        assert f(h, nat.Q4_K, w, 256, x, None, EPS, 8, 0, x, x, x, 4, 2, 128, 60, None, x, 64, 64) == \
            nat.AIH_E_LIMIT                                              # rows past the cache
        assert f(h, nat.F32, w, 256, x, None, EPS, 8, 0, x, x, x, 4, 2, 128, 0, None, x, 64, 64) == \
            nat.AIH_E_UNSUPPORTED
        assert f(h, nat.Q4_K, w, 256, x, None, EPS, 0, 0, x, x, x, 4, 2, 128, 0, None, x, 64, 64) == nat.AIH_OK
        device.synchronize()
    finally:
        wb.dispose()
        xb.dispose()


@pytest.mark.parametrize("n_q,start", [(100, 0), (70, 30)])
def test_attention_strided_equals_contiguous(device, n_q, start):
    L, h = nat.lib(), device.handle
    n_heads, n_kv, hd, max_len = 8, 2, 128, 160
    qd, kvd = n_heads * hd, n_kv * hd
    ld = qd + 2 * kvd
    rng = np.random.default_rng(n_q + start)
    qkv = rng.standard_normal((n_q, ld)).astype(np.float32)
    kc = rng.standard_normal((max_len, kvd)).astype(np.float32)
    vc = rng.standard_normal((max_len, kvd)).astype(np.float32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    bufs = [upload(device, a) for a in (qkv, np.ascontiguousarray(qkv[:, :qd]), kc, vc)]
    o1, o2 = device.create_buffer(n_q * qd * 4), device.create_buffer(n_q * qd * 4)
    sf = int(L.aih_attention_scratch_floats(n_heads, max_len))
    sb = device.create_buffer(sf * 4)
    try:
        qs, qc, kb, vb = bufs
        _check(L.aih_attention_strided(h, qs.get_pointer(), ld, kb.get_pointer(), vb.get_pointer(), o1.get_pointer(),
                                       n_q, n_heads, n_kv, hd, start, None, max_len, scale, sb.get_pointer(), sf),
               "strided")
        _check(L.aih_attention(h, qc.get_pointer(), kb.get_pointer(), vb.get_pointer(), o2.get_pointer(), n_q,
                               n_heads, n_kv, hd, start, None, max_len, scale, sb.get_pointer(), sf), "contiguous")
        a, b = _read(o1, n_q * qd), _read(o2, n_q * qd)
        assert np.isfinite(b).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert L.aih_attention_strided(h, qs.get_pointer(), qd - 4, kb.get_pointer(), vb.get_pointer(),
                                       o1.get_pointer(), n_q, n_heads, n_kv, hd, start, None, max_len, scale,
                                       sb.get_pointer(), sf) == nat.AIH_E_INVALID
        assert L.aih_attention_strided(h, qs.get_pointer(), ld + 2, kb.get_pointer(), vb.get_pointer(),
                                       o1.get_pointer(), n_q, n_heads, n_kv, hd, start, None, max_len, scale,
                                       sb.get_pointer(), sf) == nat.AIH_E_INVALID
    finally:
        for x in bufs + [o1, o2, sb]:
            x.dispose()


def _operand_image(x, mpad):
    """x (M x K fp32) as the fp16 MFMA fragment-order operand of mpad rows
    (rows past M zero): element (m, k) at half ((m/32 * K/16 + k/16) * 64 +
    m%32 + 32 * (k/8 % 2)) * 8 + k%8."""
    m_, k_ = x.shape
    img = np.zeros(mpad * k_, np.float16)
    m = np.arange(mpad)[:, None]
    k = np.arange(k_)[None, :]
    idx = (((m // 32) * (k_ // 16) + k // 16) * 64 + m % 32 + 32 * ((k // 8) % 2)) * 8 + k % 8
    full = np.zeros((mpad, k_), np.float32)
    full[:m_] = x
    img[idx.ravel()] = full.ravel().astype(np.float16)
    return img


# (300, 0) has split query tiles (three or more key tiles), (70, 30) a
# partial last row block, (2, 100) two rows
@pytest.mark.parametrize("n_q,start", [(300, 0), (70, 30), (2, 100)])
def test_attention_operand_equals_fp32_output_rounded(device, n_q, start):
    """aih_attention_operand: the fp32 output of aih_attention_strided,
    rounded to fp16 in the GEMM operand layout, bit for bit, and through the
    W_o GEMM the bits of the fp32 path."""
    L, h = nat.lib(), device.handle
    n_heads, n_kv, hd, max_len = 8, 2, 128, 320
    qd, kvd = n_heads * hd, n_kv * hd
    ld = qd + 2 * kvd
    rng = np.random.default_rng(n_q + start + 7)
    qkv = rng.standard_normal((n_q, ld)).astype(np.float32)
    kc = rng.standard_normal((max_len, kvd)).astype(np.float32)
    vc = rng.standard_normal((max_len, kvd)).astype(np.float32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    mpad = (n_q + 31) // 32 * 32
    n_out = 192
    w = synth_weight(nat.Q4_K, n_out, qd, seed=5)
    bufs = [upload(device, a) for a in (qkv, kc, vc, w)]
    o = device.create_buffer(n_q * qd * 4)
    # every half of the values must be written; the exponents follow them
    raw = np.zeros(nat.operand_bytes(n_q, qd), np.uint8)
    raw[:2 * mpad * qd].view(np.float16)[:] = np.float16(np.nan)
    xt = upload(device, raw)
    y1, y2 = device.create_buffer(n_q * n_out * 4), device.create_buffer(n_q * n_out * 4)
    sf = int(L.aih_attention_scratch_floats(n_heads, max_len))
    sb = device.create_buffer(sf * 4)
    try:
        qs, kb, vb, wb = bufs
        _check(L.aih_attention_strided(h, qs.get_pointer(), ld, kb.get_pointer(), vb.get_pointer(), o.get_pointer(),
                                       n_q, n_heads, n_kv, hd, start, None, max_len, scale, sb.get_pointer(), sf),
               "strided")
        _check(L.aih_attention_operand(h, qs.get_pointer(), ld, kb.get_pointer(), vb.get_pointer(), xt.get_pointer(),
                                       n_q, n_heads, n_kv, hd, start, None, max_len, scale), "operand")
        out = _read(o, n_q * qd).reshape(n_q, qd)
        img = np.empty(mpad * qd, np.float16)
        nat.check(L.aih_memcpy_d2h(h, img.ctypes.data, xt.get_pointer(), img.nbytes), "d2h")
        assert np.isfinite(out).all()
        assert np.array_equal(img.view(np.uint16), _operand_image(out, mpad).view(np.uint16))
        # rows and blocks of these values need no scaling: exponents 0, and
        # the all-zero blocks of the rows past n_q marked -128
        ex = np.empty(4 * mpad + mpad * qd // 32, np.uint8)
        nat.check(L.aih_memcpy_d2h(h, ex.ctypes.data, xt.get_pointer() + 2 * mpad * qd, ex.nbytes), "d2h")
        assert np.array_equal(ex[:4 * mpad].view(np.int32), np.zeros(mpad, np.int32))
        blocks = ex[4 * mpad:].view(np.int8).reshape(mpad, qd // 32)
        assert np.all(blocks[:n_q] == 0) and np.all(blocks[n_q:] == -128)
        _check(L.aih_qgemm_fused(h, nat.Q4_K, wb.get_pointer(), n_out, qd, o.get_pointer(), None, EPS, n_q,
                                 nat.PRE_NONE, nat.POST_STORE, y1.get_pointer()), "fp32 X")
        _check(L.aih_qgemm_fused(h, nat.Q4_K, wb.get_pointer(), n_out, qd, xt.get_pointer(), None, EPS, n_q,
                                 nat.PRE_F16_OPERAND, nat.POST_STORE, y2.get_pointer()), "operand X")
        a, b = _read(y1, n_q * n_out), _read(y2, n_q * n_out)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert L.aih_attention_operand(h, qs.get_pointer(), ld, kb.get_pointer(), vb.get_pointer(),
                                       xt.get_pointer() + 8, n_q, n_heads, n_kv, hd, start, None, max_len,
                                       scale) == nat.AIH_E_INVALID
    finally:
        for b in bufs + [o, xt, y1, y2, sb]:
            b.dispose()


CFG = llama.LlamaConfig(n_layers=2, dim=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=1024, vocab=1000)


def test_fused_prefill_layer_equals_separate_operators(device):
    w = llama.synth_weights(CFG, seed=11)
    dw = llama.DeviceWeights(device, w)
    ids = np.random.default_rng(4).integers(0, CFG.vocab, 45).astype(np.int32)
    out = []
    try:
        for fused in (True, False):
            dec = llama.LlamaDecoder(device, CFG, dw, 96, 48)
            try:
                dec.fused_prefill = fused
                tok = dec.prefill(ids)
                logits = dec.read_logits()
                # the rows the prompt wrote (the rest of a cache is whatever the
                # allocation held: never read, as attention masks keys past p)
                caches = [np.concatenate([_read_ptr(device, b, len(ids) * CFG.kv_dim) for b in (dec.kc[l], dec.vc[l])])
                          for l in range(CFG.n_layers)]
                out.append((tok, logits, caches))
            finally:
                dec.dispose()
    finally:
        dw.dispose()
    (t1, l1, c1), (t2, l2, c2) = out
    assert t1 == t2
    assert np.isfinite(l2).all()
    assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32))
    for a, b in zip(c1, c2):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
