"""Decoder operators (aih_rmsnorm, aih_rope_table, aih_rope, aih_store_rows,
aih_silu_mul, aih_silu_mul_pairs, aih_add, aih_attention,
aih_attention_decode_qkv, aih_embed_q, aih_argmax) vs the oracle
(oracle/llama.py) through the C ABI.

Bars: bit-exact for the row store, add, embedding gather and RoPE applied
from the same table (the same fp32 formula, no contraction); RoPE table
entries within 1 ulp (double pow/cos/sin on both sides, then rounded);
RMSNorm and SiLU*up within 2e-6 relative (fp32 tree sums and expf against
exact sums and numpy's exp); attention within 1e-5 normwise against a
float64 evaluation.  Shapes are the decoder's (32 query / 8 KV heads of
128, hidden 4096, FFN 14336) plus edge cases: one key, split boundaries of
the decode kernel (63/64/65/640 keys), positions from device memory, rows
past the cache, ids out of range, argmax ties and NaN.  The fused decode
attention (RoPE, cache store and attention in one operator) is bit-exact to
aih_rope_qkv + aih_attention for query groups of 1, 2, 4 and 8 heads.
"""
import ctypes

import numpy as np
import pytest

from aihost_amd import _native as nat
from aihost_amd import compute as C
from gpu_util import upload
from oracle import llama as ol

pytestmark = pytest.mark.gpu
L = None


@pytest.fixture(autouse=True)
def _lib():
    global L
    L = nat.lib()


class Bufs:
    def __init__(self, device):
        self.device, self.b = device, []

    def up(self, arr):
        b = upload(self.device, arr)
        self.b.append(b)
        return b.get_pointer()

    def empty(self, nbytes, fill=0xFF):
        b = self.device.create_buffer(max(16, nbytes))
        self.b.append(b)
        nat.check(L.aih_memset(self.device.handle, b.get_pointer(), fill, max(16, nbytes)), "memset")
        return b.get_pointer()

    def read(self, ptr, count, dtype=np.float32):
        out = np.empty(count, dtype=dtype)
        nat.check(L.aih_memcpy_d2h(self.device.handle, out.ctypes.data, ptr, out.nbytes), "d2h")
        return out

    def close(self):
        for b in self.b:
            b.dispose()


@pytest.fixture
def bufs(device):
    b = Bufs(device)
    yield b
    b.close()


def rnd(seed, *shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


@pytest.mark.parametrize("rows,cols", [(1, 4096), (512, 4096), (3, 1000), (2, 14336)])
def test_rmsnorm(device, bufs, rows, cols):
    x, w = rnd(rows, rows, cols), 1.0 + rnd(cols, cols, scale=0.02)
    X, W, Y = bufs.up(x), bufs.up(w), bufs.empty(rows * cols * 4)
    nat.check(L.aih_rmsnorm(device.handle, X, W, Y, rows, cols, 1e-5), "rmsnorm")
    y = bufs.read(Y, rows * cols).reshape(rows, cols)
    ref = ol.rmsnorm(x, w, 1e-5)
    assert np.max(np.abs(y - ref) / (np.abs(ref) + 1e-30)) < 2e-6
    nat.check(L.aih_rmsnorm(device.handle, X, W, X, rows, cols, 1e-5), "rmsnorm in place")
    assert np.array_equal(bufs.read(X, rows * cols).reshape(rows, cols), y)


def test_rope_table_matches_oracle(device, bufs):
    T = bufs.empty(640 * 128 * 4)
    nat.check(L.aih_rope_table(device.handle, T, 640, 128, 10000.0), "rope_table")
    t = bufs.read(T, 640 * 128).reshape(640, 64, 2)
    ref = ol.rope_table(640, 128, 10000.0)
    ulps = np.abs(t.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1, ulps.max()


def _table(device, bufs, max_pos=700):
    T = bufs.empty(max_pos * 128 * 4)
    nat.check(L.aih_rope_table(device.handle, T, max_pos, 128, 10000.0), "rope_table")
    return T, bufs.read(T, max_pos * 128).reshape(max_pos, 64, 2)


@pytest.mark.parametrize("rows,heads,start", [(512, 32, 0), (1, 8, 577), (7, 32, 100)])
def test_rope_exact_from_the_same_table(device, bufs, rows, heads, start):
    T, t = _table(device, bufs)
    x = rnd(rows + heads, rows, heads * 128)
    X, Y = bufs.up(x), bufs.empty(x.nbytes)
    nat.check(L.aih_rope(device.handle, X, heads * 128, Y, heads * 128, rows, heads, 128, start, None, T, 700, 0,
                         rows), "rope")
    ref = ol.rope(x, list(range(start, start + rows)), heads, 128, t)
    assert np.array_equal(bufs.read(Y, x.size).reshape(x.shape), ref)


def test_rope_into_cache_at_device_position(device, bufs):
    T, t = _table(device, bufs)
    rows, heads, max_len, p = 3, 8, 64, 60          # positions 60, 61, 62, 63 -> the 4th is past the cache
    x = rnd(5, rows + 1, heads * 128)
    X, C_ = bufs.up(x), bufs.empty(max_len * heads * 128 * 4, fill=0)
    P = bufs.up(np.array([p], np.int32))
    nat.check(L.aih_rope(device.handle, X, heads * 128, C_, heads * 128, rows + 1, heads, 128, 1, P, T, 700, 1,
                         max_len), "rope -> cache")
    c = bufs.read(C_, max_len * heads * 128).reshape(max_len, heads * 128)
    ref = ol.rope(x[:3], [61, 62, 63], heads, 128, t)
    assert np.array_equal(c[61:64], ref) and not c[:61].any()     # row 3 (position 64) skipped
    with pytest.raises(nat.AihError):                               # host-known position past the cache
        nat.check(L.aih_rope(device.handle, X, heads * 128, C_, heads * 128, 2, heads, 128, 63, None, T, 700, 1,
                             max_len), "rope")


def test_store_rows_and_add_exact(device, bufs):
    x = rnd(6, 4, 1024)
    X, Y = bufs.up(x), bufs.empty(10 * 1024 * 4, fill=0)
    P = bufs.up(np.array([5], np.int32))
    nat.check(L.aih_store_rows(device.handle, X, 4, 1024, Y, 10, 2, P), "store_rows")   # rows 7, 8, 9 (+10 skipped)
    y = bufs.read(Y, 10 * 1024).reshape(10, 1024)
    assert np.array_equal(y[7:10], x[:3]) and not y[:7].any()
    a, b = rnd(7, 4096 * 3), rnd(8, 4096 * 3)
    A, B, S = bufs.up(a), bufs.up(b), bufs.empty(a.nbytes)
    nat.check(L.aih_add(device.handle, A, B, S, a.size), "add")
    assert np.array_equal(bufs.read(S, a.size), a + b)


def test_silu_mul(device, bufs):
    g = np.concatenate([rnd(9, 14336 * 2, scale=3.0), np.array([0.0, 88.0, -88.0, -200.0, 20.0], np.float32)])
    u = rnd(10, g.size)
    G, U = bufs.up(g), bufs.up(u)
    nat.check(L.aih_silu_mul(device.handle, G, U, G, g.size), "silu_mul in place")
    y = bufs.read(G, g.size)
    ref = ol.silu_mul(g, u)
    assert np.max(np.abs(y - ref) / (np.abs(ref) + 1e-30)) < 2e-6


def test_silu_and_mul_separately(device, bufs):
    """aih_silu (in place) then aih_mul: the reference's SiLU and Multiply
    operators one after the other, bit for bit the fused aih_silu_mul."""
    g = np.concatenate([rnd(19, 14336, scale=3.0), np.array([0.0, 88.0, -88.0, -200.0, 20.0], np.float32)])
    u = rnd(20, g.size)
    G, U, F = bufs.up(g), bufs.up(u), bufs.up(g)
    nat.check(L.aih_silu(device.handle, G, G, g.size), "silu in place")
    s = bufs.read(G, g.size)
    ref = ol.silu_mul(g, np.ones_like(g))
    assert np.max(np.abs(s - ref) / (np.abs(ref) + 1e-30)) < 2e-6
    nat.check(L.aih_mul(device.handle, G, U, G, g.size), "mul in place")
    assert np.array_equal(bufs.read(G, g.size), s * u)
    nat.check(L.aih_silu_mul(device.handle, F, U, F, g.size), "silu_mul")
    assert np.array_equal(bufs.read(G, g.size).view(np.uint32), bufs.read(F, g.size).view(np.uint32))
    assert L.aih_silu(device.handle, G, G, -1) == nat.AIH_E_INVALID
    assert L.aih_mul(device.handle, None, U, G, 4) == nat.AIH_E_INVALID
    assert L.aih_mul(device.handle, G, U, G, 0) == nat.AIH_OK


def test_embed_f32_table(device, bufs):
    """aih_embed_q on an fp32 table (ComputeOps.EmbeddingLookup): rows by id,
    zeros for ids outside the table."""
    vocab, dim = 300, 4096
    tab = rnd(21, vocab, dim)
    ids = np.array([5, 0, 299, 5, 300, -3, 17], np.int32)
    T, I = bufs.up(tab), bufs.up(ids)
    Y = bufs.empty(len(ids) * dim * 4)
    nat.check(L.aih_embed_q(device.handle, nat.F32, T, vocab, dim, I, len(ids), Y), "embed f32")
    y = bufs.read(Y, len(ids) * dim).reshape(len(ids), dim)
    ok = (ids >= 0) & (ids < vocab)
    assert np.array_equal(y[ok], tab[ids[ok]])
    assert not y[~ok].any()


def test_silu_mul_pairs(device, bufs):
    # rows of interleaved (gate, up) columns, as a GEMM over gate/up rows
    # interleaved writes them; bit-exact to aih_silu_mul on the split halves
    rows, n = 3, 14336
    x = rnd(12, rows, 2 * n, scale=3.0)
    x[0, :10:2] = [0.0, 88.0, -88.0, -200.0, 20.0]
    X, Y = bufs.up(x), bufs.empty(rows * n * 4)
    nat.check(L.aih_silu_mul_pairs(device.handle, X, Y, rows, n), "silu_mul_pairs")
    y = bufs.read(Y, rows * n).reshape(rows, n)
    ref = ol.silu_mul(x[:, 0::2], x[:, 1::2])
    assert np.max(np.abs(y - ref) / (np.abs(ref) + 1e-30)) < 2e-6
    G, U = bufs.up(np.ascontiguousarray(x[:, 0::2])), bufs.up(np.ascontiguousarray(x[:, 1::2]))
    nat.check(L.aih_silu_mul(device.handle, G, U, G, rows * n), "silu_mul")
    assert np.array_equal(bufs.read(G, rows * n).reshape(rows, n), y)
    assert L.aih_silu_mul_pairs(device.handle, X, Y, -1, n) == nat.AIH_E_INVALID
    assert L.aih_silu_mul_pairs(device.handle, X, Y, 0, n) == nat.AIH_OK


def _attn(device, bufs, n_q, start, L_cache, nh=32, nkv=8, pos_dev=None, seed=11):
    kvd = nkv * 128
    q = rnd(seed, n_q, nh * 128)
    K, V = rnd(seed + 1, L_cache, kvd), rnd(seed + 2, L_cache, kvd)
    return _attn_of(device, bufs, q, K, V, start, nh, nkv, pos_dev)


def _run_attn(device, bufs, q, K, V, start, nh, nkv):
    n_q, L_cache = q.shape[0], K.shape[0]
    Q, KC, VC = bufs.up(q), bufs.up(K), bufs.up(V)
    O = bufs.empty(q.nbytes)
    nsc = int(L.aih_attention_scratch_floats(nh, L_cache))
    S = bufs.empty(nsc * 4)
    scale = float(np.float32(1) / np.sqrt(np.float32(128)))
    nat.check(L.aih_attention(device.handle, Q, KC, VC, O, n_q, nh, nkv, 128, start, None, L_cache, scale, S, nsc),
              "attention")
    return bufs.read(O, q.size).reshape(q.shape)


def _attn_of(device, bufs, q, K, V, start, nh, nkv, pos_dev=None):
    n_q, L_cache = q.shape[0], K.shape[0]
    Q, KC, VC = bufs.up(q), bufs.up(K), bufs.up(V)
    O = bufs.empty(q.nbytes)
    nsc = int(L.aih_attention_scratch_floats(nh, L_cache))
    S = bufs.empty(nsc * 4)
    scale = float(np.float32(1) / np.sqrt(np.float32(128)))
    P = None
    if pos_dev is not None:
        P = bufs.up(np.array([pos_dev], np.int32))
    nat.check(L.aih_attention(device.handle, Q, KC, VC, O, n_q, nh, nkv, 128, start, P, L_cache, scale, S, nsc),
              "attention")
    o = bufs.read(O, q.size).reshape(q.shape)
    p0 = start + (pos_dev or 0)
    ref = ol.attention(q, K, V, list(range(p0, p0 + n_q)), nh, nkv, 128)
    err = np.linalg.norm(o - ref) / np.linalg.norm(ref)
    assert err < 1e-5, err
    return o


@pytest.mark.parametrize("keys", [1, 2, 63, 64, 65, 200, 640])
def test_attention_decode_split_boundaries(device, bufs, keys):
    _attn(device, bufs, 1, keys - 1, 640)


@pytest.mark.parametrize("keys", [4096, 5000, 9000])
def test_attention_decode_long_context(device, bufs, keys):
    # more keys than 64 splits of 64: each split walks several sub-chunks
    _attn(device, bufs, 1, keys - 1, 9000, nh=8, nkv=2)


def test_attention_decode_scratch_reused(device, bufs):
    # one scratch serves consecutive calls at different positions
    kvd = 8 * 128
    K, V = rnd(21, 640, kvd), rnd(22, 640, kvd)
    KC, VC = bufs.up(K), bufs.up(V)
    nsc = int(L.aih_attention_scratch_floats(32, 640))
    S = bufs.empty(nsc * 4)
    scale = float(np.float32(1) / np.sqrt(np.float32(128)))
    for i, p in enumerate((100, 639, 7, 300)):
        q = rnd(30 + i, 1, 32 * 128)
        Q, O = bufs.up(q), bufs.empty(q.nbytes)
        nat.check(L.aih_attention(device.handle, Q, KC, VC, O, 1, 32, 8, 128, p, None, 640, scale, S, nsc), "attn")
        ref = ol.attention(q, K, V, [p], 32, 8, 128)
        o = bufs.read(O, q.size).reshape(q.shape)
        assert np.linalg.norm(o - ref) / np.linalg.norm(ref) < 1e-5


@pytest.mark.parametrize("n_q,start", [(512, 0), (100, 0), (65, 40), (2, 7), (128, 512), (17, 600)])
def test_attention_prefill(device, bufs, n_q, start):
    # query tiles of 64 and key tiles of 64: full and partial tiles of both,
    # rows that end at the cache's last row (start + n_q = 640)
    _attn(device, bufs, n_q, start, 640)


def test_attention_prefill_power_of_two_invariance(device, bufs):
    # the products run on fp16 hi/lo operands with per-row (Q) and per-tile
    # (K, V) powers of two: scaling Q by 2^a, K by 2^-a and V by 2^b changes
    # no rounding, so the output is the unscaled one times 2^b, bit for bit
    nh, nkv, n_q, L_cache = 8, 2, 200, 256
    q, K, V = rnd(51, n_q, nh * 128), rnd(52, L_cache, nkv * 128), rnd(53, L_cache, nkv * 128)
    base = _run_attn(device, bufs, q, K, V, 0, nh, nkv)
    for a, b in [(40, -30), (-60, 50), (7, 0)]:
        o = _run_attn(device, bufs, q * np.float32(2.0 ** a), K * np.float32(2.0 ** -a), V * np.float32(2.0 ** b),
                      0, nh, nkv)
        assert np.array_equal(o, base * np.float32(2.0 ** b)), (a, b)


def test_attention_prefill_value_magnitudes(device, bufs):
    # V tiles of 64 keys from 1e-6 to 1e6 times N(0, 1), and rows of Q from
    # 1e-3 to 1: every row (including those that see only the smallest
    # tiles) within 1e-5 of the oracle, row by row
    nh, nkv, n_q, L_cache = 4, 2, 320, 320
    q, K, V = rnd(61, n_q, nh * 128), rnd(62, L_cache, nkv * 128), rnd(63, L_cache, nkv * 128)
    V *= (10.0 ** (3 * ((np.arange(L_cache) // 64) % 5 - 2))).astype(np.float32)[:, None]
    q *= (10.0 ** -(np.arange(n_q) % 4)).astype(np.float32)[:, None]
    o = _run_attn(device, bufs, q, K, V, 0, nh, nkv)
    ref = ol.attention(q, K, V, list(range(n_q)), nh, nkv, 128)
    err = np.linalg.norm(o - ref, axis=1) / np.linalg.norm(ref, axis=1)
    assert err.max() < 1e-5, err.max()


def test_attention_prefill_captured_on_a_fresh_context(device, bufs):
    # captured on a fresh context, whose workspace never grew: the tiled
    # attention needs none; replays of the graph, with eager calls between
    # them, all within 1e-5 of the oracle
    nh, nkv, n_q, L_cache, start = 32, 8, 300, 640, 40
    q, K, V = rnd(71, n_q, nh * 128), rnd(72, L_cache, nkv * 128), rnd(73, L_cache, nkv * 128)
    Q, KC, VC, O = bufs.up(q), bufs.up(K), bufs.up(V), bufs.empty(q.nbytes)
    ref = ol.attention(q, K, V, list(range(start, start + n_q)), nh, nkv, 128)
    scale = float(np.float32(1) / np.sqrt(np.float32(128)))
    fresh = C.HipComputeDevice(0)
    try:
        h = fresh.handle
        nat.check(L.aih_capture_begin(h), "capture_begin")
        rc = L.aih_attention(h, Q, KC, VC, O, n_q, nh, nkv, 128, start, None, L_cache, scale, None, 0)
        g = ctypes.c_void_p()
        nat.check(L.aih_capture_end(h, ctypes.byref(g)), "capture_end")
        nat.check(rc, "attention (captured)")
        for _ in range(3):
            nat.check(L.aih_memset(device.handle, O, 0xFF, q.nbytes), "memset")   # NaN until written
            device.synchronize()
            nat.check(L.aih_graph_launch(h, g.value), "graph_launch")
            fresh.synchronize()
            o = bufs.read(O, q.size).reshape(q.shape)
            assert np.linalg.norm(o - ref) / np.linalg.norm(ref) < 1e-5
            _attn(device, bufs, 70, 3, 640)   # eager work between the replays
        nat.check(L.aih_graph_destroy(g.value), "graph_destroy")
    finally:
        fresh.dispose()


def test_attention_prefill_at_device_position(device, bufs):
    _attn(device, bufs, 70, 3, 640, pos_dev=20)


def test_attention_gqa_small(device, bufs):
    _attn(device, bufs, 40, 0, 64, nh=4, nkv=2)
    _attn(device, bufs, 1, 39, 64, nh=4, nkv=2)


def test_attention_argument_errors(device, bufs):
    X = bufs.empty(4096 * 4)
    h = device.handle
    assert L.aih_attention(h, X, X, X, X, 1, 32, 8, 64, 0, None, 8, 1.0, X, 4096) == nat.AIH_E_UNSUPPORTED
    assert L.aih_attention(h, X, X, X, X, 1, 32, 5, 128, 0, None, 8, 1.0, X, 4096) == nat.AIH_E_INVALID
    assert L.aih_attention(h, X, X, X, X, 4, 32, 8, 128, 6, None, 8, 1.0, X, 4096) == nat.AIH_E_LIMIT
    assert L.aih_attention(h, X, X, X, X, 1, 32, 8, 128, 0, None, 8, 1.0, None, 0) == nat.AIH_E_INVALID
    device.synchronize()


@pytest.mark.parametrize("qtype,dim", [(nat.Q4_K, 4096), (nat.Q6_K, 512), (nat.Q8_0, 96), (nat.Q4_0, 64)])
def test_embed_bit_exact(device, bufs, qtype, dim):
    vocab = 300
    tab = C.quantize(qtype, C.fill_normal(12, vocab * dim, 0.0, 0.02), vocab, dim)
    ids = np.array([5, 0, 299, 5, 300, -3, 17], np.int32)
    T, I = bufs.up(tab), bufs.up(ids)
    Y = bufs.empty(len(ids) * dim * 4)
    nat.check(L.aih_embed_q(device.handle, qtype, T, vocab, dim, I, len(ids), Y), "embed")
    y = bufs.read(Y, len(ids) * dim).reshape(len(ids), dim)
    assert np.array_equal(y, ol.embed(qtype, tab, vocab, dim, ids))


def test_argmax_ties_nan_and_history(device, bufs):
    x = rnd(13, 32000)
    x[[100, 2000, 31999]] = 50.0                  # ties: the first index wins
    x[7] = np.nan
    X, T = bufs.up(x), bufs.empty(16)
    H, P = bufs.empty(64, fill=0), bufs.up(np.array([10], np.int32))
    nat.check(L.aih_argmax(device.handle, X, x.size, T, P, H, 8, 9), "argmax")
    assert bufs.read(T, 1, np.int32)[0] == 100 == ol.argmax(x)
    assert bufs.read(P, 1, np.int32)[0] == 11
    h = bufs.read(H, 8, np.int32)
    assert h[1] == 100 and not np.delete(h, 1).any()         # history[10 - 9]
    y = np.full(5, -np.inf, np.float32)
    Y = bufs.up(y)
    nat.check(L.aih_argmax(device.handle, Y, 5, T, None, None, 0, 0), "argmax")
    assert bufs.read(T, 1, np.int32)[0] == 0


# pad = 2: rows 2 floats longer than the three blocks, so the row stride is
# not a multiple of 4 floats (the scalar kernel instead of the 16-byte one)
@pytest.mark.parametrize("rows,start,pos_dev,pad", [(1, 0, 517, 0), (40, 0, None, 0), (3, 61, None, 0),
                                                    (40, 0, None, 2)])
def test_rope_qkv_equals_separate_ops(device, bufs, rows, start, pos_dev, pad):
    nh, nkv, hd, max_len = 32, 8, 128, 640
    qd, kvd = nh * hd, nkv * hd
    T, t = _table(device, bufs, 640)
    fused = rnd(40 + rows, rows, qd + 2 * kvd + pad)         # one fused projection output per row
    q, k, v = fused[:, :qd], fused[:, qd:qd + kvd], fused[:, qd + kvd:qd + 2 * kvd]
    F = bufs.up(fused)
    KC, VC = bufs.empty(max_len * kvd * 4, fill=0), bufs.empty(max_len * kvd * 4, fill=0)
    P = bufs.up(np.array([pos_dev], np.int32)) if pos_dev is not None else None
    ld = qd + 2 * kvd + pad
    nat.check(L.aih_rope_qkv(device.handle, F, ld, F + qd * 4, ld, F + (qd + kvd) * 4, ld, KC, VC, rows, nh, nkv, hd,
                             start, P, T, 640, max_len), "rope_qkv")
    p0 = start + (pos_dev or 0)
    pos = list(range(p0, p0 + rows))
    out = bufs.read(F, fused.size).reshape(fused.shape)
    kc = bufs.read(KC, max_len * kvd).reshape(max_len, kvd)
    vc = bufs.read(VC, max_len * kvd).reshape(max_len, kvd)
    assert np.array_equal(out[:, :qd], ol.rope(q, pos, nh, hd, t))
    assert np.array_equal(out[:, qd:], fused[:, qd:])                     # K and V inputs untouched
    assert np.array_equal(kc[p0:p0 + rows], ol.rope(k, pos, nkv, hd, t))
    assert np.array_equal(vc[p0:p0 + rows], v)
    assert not kc[:p0].any() and not vc[p0 + rows:].any()


def _decode_qkv_pair(device, bufs, nh, nkv, max_len, p, pos_dev=False, seed=50, table_rows=None):
    """Run aih_attention_decode_qkv and, on a copy of the same caches,
    aih_rope_qkv + aih_attention (one row); return both outputs and caches."""
    hd = 128
    qd, kvd = nh * hd, nkv * hd
    table_rows = table_rows or max_len
    T, t = _table(device, bufs, table_rows)
    fused = rnd(seed, 1, qd + 2 * kvd)
    K, V = rnd(seed + 1, max_len, kvd), rnd(seed + 2, max_len, kvd)
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    nsc = int(L.aih_attention_scratch_floats(nh, max_len))
    start, P = (0, bufs.up(np.array([p], np.int32))) if pos_dev else (p, None)
    res = []
    for fused_path in (True, False):
        F, KC, VC = bufs.up(fused), bufs.up(K), bufs.up(V)
        O, S = bufs.empty(qd * 4), bufs.empty(nsc * 4)
        if fused_path:
            nat.check(L.aih_attention_decode_qkv(device.handle, F, KC, VC, O, nh, nkv, hd, start, P, T, table_rows,
                                                 max_len, scale, S, nsc), "attention_decode_qkv")
            assert np.array_equal(bufs.read(F, fused.size), fused.reshape(-1))   # QKV not modified
        else:
            ld = qd + 2 * kvd
            nat.check(L.aih_rope_qkv(device.handle, F, ld, F + qd * 4, ld, F + (qd + kvd) * 4, ld, KC, VC, 1, nh, nkv,
                                     hd, start, P, T, table_rows, max_len), "rope_qkv")
            nat.check(L.aih_attention(device.handle, F, KC, VC, O, 1, nh, nkv, hd, start, P, max_len, scale, S, nsc),
                      "attention")
        res.append((bufs.read(O, qd), bufs.read(KC, max_len * kvd).reshape(max_len, kvd),
                    bufs.read(VC, max_len * kvd).reshape(max_len, kvd)))
    return res, fused, K, V, t


@pytest.mark.parametrize("nh,nkv", [(32, 8), (8, 4), (4, 4), (32, 4)])
@pytest.mark.parametrize("p", [0, 63, 64, 65, 517, 639])
def test_attention_decode_qkv_equals_separate_ops(device, bufs, nh, nkv, p):
    (o, kc, vc), (o2, kc2, vc2) = _decode_qkv_pair(device, bufs, nh, nkv, 640, p, pos_dev=p % 2 == 1)[0]
    assert np.array_equal(o, o2)
    assert np.array_equal(kc, kc2) and np.array_equal(vc, vc2)


def test_attention_decode_qkv_vs_oracle(device, bufs):
    nh, nkv, p, max_len = 32, 8, 300, 640
    res, fused, K, V, t = _decode_qkv_pair(device, bufs, nh, nkv, max_len, p, pos_dev=True, seed=60)
    o, kc, vc = res[0]
    qd, kvd = nh * 128, nkv * 128
    q = ol.rope(fused[:, :qd], [p], nh, 128, t)
    K, V = K.copy(), V.copy()
    K[p] = ol.rope(fused[:, qd:qd + kvd], [p], nkv, 128, t)[0]
    V[p] = fused[0, qd + kvd:]
    assert np.array_equal(kc, K) and np.array_equal(vc, V)      # only row p written
    ref = ol.attention(q, K, V, [p], nh, nkv, 128)[0]
    assert np.linalg.norm(o - ref) / np.linalg.norm(ref) < 1e-5


def test_attention_decode_qkv_long_context_and_past_the_cache(device, bufs):
    # several sub-chunks per split; a position past the cache attends to the
    # whole cache and stores nothing, like the separate operators
    for p in (8999, 5000, 9000, 9100):
        (o, kc, vc), (o2, kc2, vc2) = _decode_qkv_pair(device, bufs, 8, 2, 9000, p, pos_dev=True, seed=p,
                                                       table_rows=9200)[0]
        assert np.array_equal(o, o2), p
        assert np.array_equal(kc, kc2) and np.array_equal(vc, vc2), p


def test_attention_decode_qkv_argument_errors(device, bufs):
    X = bufs.empty(8192 * 4)
    h = device.handle
    f = L.aih_attention_decode_qkv
    assert f(h, X, X, X, X, 12, 4, 128, 0, None, X, 8, 8, 1.0, X, 8192) == nat.AIH_E_UNSUPPORTED    # group of 3
    assert f(h, X, X, X, X, 32, 8, 64, 0, None, X, 8, 8, 1.0, X, 8192) == nat.AIH_E_UNSUPPORTED
    assert f(h, X, X, X, X, 32, 5, 128, 0, None, X, 8, 8, 1.0, X, 8192) == nat.AIH_E_INVALID
    assert f(h, X, X, X, X, 32, 8, 128, 0, None, X, 4, 8, 1.0, X, 8192) == nat.AIH_E_LIMIT       # table too short
    assert f(h, X, X, X, X, 32, 8, 128, 8, None, X, 8, 8, 1.0, X, 8192) == nat.AIH_E_LIMIT       # start past the cache
    assert f(h, X, X, X, X, 32, 8, 128, 0, None, X, 8, 8, 1.0, X, 100) == nat.AIH_E_INVALID      # scratch too small
    device.synchronize()


@pytest.mark.parametrize("nh,nkv,keys", [(12, 4, 100), (6, 1, 640), (24, 8, 65), (8, 8, 1)])
def test_attention_decode_other_group_sizes(device, bufs, nh, nkv, keys):
    # groups of 3 and 6 heads take the one-workgroup-per-head kernel; 1 the
    # grouped one with a single head
    _attn(device, bufs, 1, keys - 1, 640, nh=nh, nkv=nkv)


@pytest.mark.parametrize("n,where", [(1, 0), (32768, 32767), (32769, 32768), (100000, 70001), (128256, 5)])
def test_argmax_sizes(device, bufs, n, where):
    # one and several rounds of the batched scan; the maximum anywhere
    x = rnd(n % 97 + 3, n)
    x[where] = 99.0
    X, T = bufs.up(x), bufs.empty(16)
    nat.check(L.aih_argmax(device.handle, X, n, T, None, None, 0, 0), "argmax")
    assert bufs.read(T, 1, np.int32)[0] == where == ol.argmax(x)


def test_argmax_all_nan_gives_zero(device, bufs):
    x = np.full(40000, np.nan, np.float32)
    X, T = bufs.up(x), bufs.empty(16, fill=0x7F)
    nat.check(L.aih_argmax(device.handle, X, x.size, T, None, None, 0, 0), "argmax")
    assert bufs.read(T, 1, np.int32)[0] == 0


@pytest.mark.parametrize("n,where,offset", [(32003, 32002, 0), (10, 9, 1), (70001, 70000, 0), (70001, 3, 3)])
def test_argmax_unaligned_and_tails(device, bufs, n, where, offset):
    # vector path with a 1-3 element tail, and an X not 16-byte aligned
    x = rnd(n + offset, n + offset)
    x[offset + where] = 77.0
    X, T = bufs.up(x), bufs.empty(16)
    nat.check(L.aih_argmax(device.handle, X + 4 * offset, n, T, None, None, 0, 0), "argmax")
    assert bufs.read(T, 1, np.int32)[0] == where == ol.argmax(x[offset:])
