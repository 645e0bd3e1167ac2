"""Pins of the oracle's decoder operators (oracle/llama.py) by closed forms
and invariants, each chosen so that a plausible slip fails: half-split
instead of interleaved RoPE pairs, a missing attention scale, a wrong KV head
for grouped queries, an off-by-one causal mask, a sum instead of a mean in
RMSNorm, argmax ties resolved to the last index."""
import numpy as np
import pytest

from oracle import llama as ol
from oracle import oracle as orc


def test_rmsnorm_hand_computed_and_invariants():
    y = ol.rmsnorm(np.array([[3.0, 4.0]], np.float32), np.array([1.0, 2.0], np.float32), eps=0.0)
    rms = np.sqrt((9 + 16) / 2)                      # mean of squares, not the sum
    assert np.allclose(y, [[3 / rms, 2 * 4 / rms]], rtol=1e-6)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 64)).astype(np.float32)
    w = rng.standard_normal(64).astype(np.float32)
    assert np.allclose(ol.rmsnorm(7.5 * x, w, 0.0), ol.rmsnorm(x, w, 0.0), rtol=1e-5)   # scale invariance
    c = np.full((1, 16), 0.5, np.float32)                                              # constant row, eps kept
    assert np.allclose(ol.rmsnorm(c, np.ones(16, np.float32), 1e-5), 0.5 / np.sqrt(0.25 + 1e-5), rtol=1e-6)


def test_rope_table_closed_form():
    t = ol.rope_table(50, 128, 10000.0)
    assert np.array_equal(t[0, :, 0], np.ones(64, np.float32)) and np.array_equal(t[0, :, 1], np.zeros(64, np.float32))
    p = np.arange(50)
    assert np.allclose(t[:, 0, 0], np.cos(p), atol=1e-7) and np.allclose(t[:, 0, 1], np.sin(p), atol=1e-7)  # freq_0 = 1
    f5 = 10000.0 ** (-10 / 128)                                                   # pair 5: 1/theta^(2*5/128)
    assert np.allclose(t[:, 5, 0], np.cos(p * f5), atol=2e-6)


def test_rope_interleaved_pairs_and_rotation_properties():
    t = ol.rope_table(64, 128)
    x = np.zeros((1, 2 * 128), np.float32)
    x[0, 0] = 1.0                       # element 0 of head 0 pairs with element 1, not element 64
    y = ol.rope(x, [3], 2, 128, t)
    assert np.isclose(y[0, 0], np.cos(3.0), atol=1e-6) and np.isclose(y[0, 1], np.sin(3.0), atol=1e-6)
    assert np.count_nonzero(y) == 2
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 4 * 128)).astype(np.float32)
    assert np.array_equal(ol.rope(x, [0, 0, 0, 0], 4, 128, t), x)            # position 0 is the identity
    y = ol.rope(x, [5, 17, 33, 63], 4, 128, t)
    pn = lambda a: np.hypot(a[:, 0::2], a[:, 1::2])
    assert np.allclose(pn(y), pn(x), rtol=1e-5)                             # each pair keeps its norm
    # rotations compose: rotating by a then by b equals rotating by a + b
    y2 = ol.rope(ol.rope(x, [5, 6, 7, 8], 4, 128, t), [10, 20, 30, 40], 4, 128, t)
    assert np.allclose(y2, ol.rope(x, [15, 26, 37, 48], 4, 128, t), atol=1e-4)


def _kv(L, nkv, hd, rng):
    return rng.standard_normal((L, nkv * hd)).astype(np.float32), rng.standard_normal((L, nkv * hd)).astype(np.float32)


def test_attention_single_key_and_gqa_mapping():
    rng = np.random.default_rng(2)
    nh, nkv, hd = 8, 2, 128
    K, V = _kv(4, nkv, hd, rng)
    q = rng.standard_normal((1, nh * hd)).astype(np.float32)
    o = ol.attention(q, K, V, [0], nh, nkv, hd).reshape(nh, hd)
    for h in range(nh):                 # one key: the output is its value, of KV head h // 4
        assert np.allclose(o[h], V[0, (h // 4) * hd:(h // 4 + 1) * hd], atol=1e-6)


def test_attention_uniform_scores_mean_and_scale():
    rng = np.random.default_rng(3)
    nh, nkv, hd = 2, 1, 128
    K = np.zeros((6, hd), np.float32)
    V = rng.standard_normal((6, hd)).astype(np.float32)
    q = rng.standard_normal((1, nh * hd)).astype(np.float32)
    o = ol.attention(q, K, V, [5], nh, nkv, hd).reshape(nh, hd)
    assert np.allclose(o, V.mean(0), atol=1e-6)                              # equal scores -> mean of V
    K = np.zeros((2, hd), np.float32)
    K[1, 0] = 1.0
    qq = np.zeros((1, hd), np.float32)
    qq[0, 0] = 2.0                       # scores 0 and 2/sqrt(128)
    o = ol.attention(qq, K, V[:2], [1], 1, 1, hd)
    s = 2.0 / np.sqrt(128.0)
    w1 = np.exp(s) / (1 + np.exp(s))
    assert np.allclose(o[0], (1 - w1) * V[0] + w1 * V[1], atol=1e-6)


def test_attention_is_causal():
    rng = np.random.default_rng(4)
    nh, nkv, hd = 4, 2, 128
    K, V = _kv(10, nkv, hd, rng)
    q = rng.standard_normal((3, nh * hd)).astype(np.float32)
    o = ol.attention(q, K, V, [2, 3, 4], nh, nkv, hd)
    K2, V2 = K.copy(), V.copy()
    K2[5:] = 99.0
    V2[5:] = -7.0                        # rows after the last query position
    assert np.array_equal(ol.attention(q, K2, V2, [2, 3, 4], nh, nkv, hd), o)
    K2[4] = 0.0                          # row 4 is visible to the last query only
    o2 = ol.attention(q, K2, V, [2, 3, 4], nh, nkv, hd)
    assert np.array_equal(o2[:2], o[:2]) and not np.allclose(o2[2], o[2])


def test_silu_mul_known_points():
    g = np.array([0.0, 1.0, -1.0, 30.0, -100.0], np.float32)
    u = np.array([3.0, 2.0, 1.0, 1.0, 5.0], np.float32)
    y = ol.silu_mul(g, u)
    assert y[0] == 0.0
    assert np.isclose(y[1], 2.0 / (1.0 + np.exp(-1.0)), rtol=1e-6)
    assert np.isclose(y[2], -1.0 / (1.0 + np.exp(1.0)), rtol=1e-6)
    assert np.isclose(y[3], 30.0, rtol=1e-6) and abs(y[4]) < 1e-30


def test_argmax_first_index_and_nan():
    assert ol.argmax([1.0, 5.0, 5.0, 2.0]) == 1
    assert ol.argmax([np.nan, -1.0, -1.0]) == 1
    assert ol.argmax([-np.inf, -np.inf]) == 0


def test_embed_rows_are_dequantized_rows():
    from aihost_amd import compute as C
    vocab, dim = 7, 256
    q = C.quantize(C.GGUFTensorType.Q4_K, C.fill_normal(9, vocab * dim, 0.0, 0.02), vocab, dim)
    e = ol.embed(orc.Q4_K, q, vocab, dim, [3, 0, 6, 9, -1])
    full = orc.dequantize(orc.Q4_K, q, vocab * dim).reshape(vocab, dim)
    assert np.array_equal(e[:3], full[[3, 0, 6]]) and not e[3:].any()


def test_oracle_forward_incremental_equals_full_prefill():
    """Decoding token by token through the KV cache gives the same last-row
    logits as one prefill of the whole sequence (cache bookkeeping of the
    oracle decoder)."""
    from aihost_amd import llama
    cfg = llama.LlamaConfig(n_layers=2, dim=256, n_heads=2, n_kv_heads=1, head_dim=128, ffn=512, vocab=50)
    w = llama.synth_weights(cfg, seed=8)
    ids = [3, 17, 4, 49, 0]
    table = ol.rope_table(16, 128)

    def fresh():
        return ol.Model(cfg, w), [(np.zeros((16, cfg.kv_dim), np.float32), np.zeros((16, cfg.kv_dim), np.float32))
                                  for _ in range(cfg.n_layers)]

    m, kv = fresh()
    full = m.forward(ids, 0, kv, table)
    m, kv = fresh()
    m.forward(ids[:2], 0, kv, table)
    for i in range(2, len(ids)):
        step = m.forward([ids[i]], i, kv, table)
    assert np.allclose(step, full, rtol=1e-5, atol=1e-6)
    assert full.shape == (1, cfg.vocab)


# -- composition of Model.forward (ComputeOps.TransformerLayer, ComputeOps.cs:
# 1250-1356, then TransformerBase.ForwardHead, TransformerBase.cs:168-191),
# pinned by special cases with closed forms.  The expected values below are
# written from the definitions (mean-square normalisation, the GQA head
# expansion, the SiLU), not through the oracle's operators.

def _small_model(seed, n_layers=2):
    from aihost_amd import llama
    cfg = llama.LlamaConfig(n_layers=n_layers, dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=48)
    w = dict(llama.synth_weights(cfg, seed=seed))
    # norm weights well away from 1 and different per norm, so that a swapped
    # or dropped norm weight changes the result
    rng = np.random.default_rng(seed)
    for name, (qt, a, r, c) in list(w.items()):
        if qt == orc.F32:
            w[name] = (qt, rng.uniform(0.5, 1.5, a.size).astype(np.float32), r, c)
    return cfg, w


def _zeroed(w, names):
    out = dict(w)
    for n in names:
        qt, a, r, c = out[n]
        out[n] = (qt, np.zeros_like(a), r, c)
    return out


def _run(cfg, w, ids, start=0, max_len=16, kv=None, model=None):
    m = model or ol.Model(cfg, w)
    if kv is None:
        kv = [(np.zeros((max_len, cfg.kv_dim), np.float32), np.zeros((max_len, cfg.kv_dim), np.float32))
              for _ in range(cfg.n_layers)]
    return m.forward(list(ids), start, kv, ol.rope_table(max_len, cfg.head_dim, cfg.theta), last_only=False), m


def _deq(w, name):
    qt, a, r, c = w[name]
    return orc.dequantize(qt, a, r * c).reshape(r, c).astype(np.float64)


def _norm(x, g, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(g, np.float64)


def _head(cfg, w, x):
    return _norm(x, w["output_norm"][1], cfg.eps) @ _deq(w, "output").T


def _embed_rows(w, ids):
    return _deq(w, "token_embd")[list(ids)]


def test_forward_zero_output_projections_is_identity_layers():
    """W_o = W_down = 0: attention and FFN add nothing, so every layer passes
    x through and the logits are head(rmsnorm(embedding)).  A missing
    residual (x replaced by the sublayer output) gives zero logits; a
    missing output norm or the wrong norm weight changes them."""
    cfg, w = _small_model(21)
    w = _zeroed(w, ["blk.%d.%s" % (l, s) for l in range(cfg.n_layers) for s in ("attn_output", "ffn_down")])
    ids = [5, 0, 47, 12]
    got, _ = _run(cfg, w, ids)
    want = _head(cfg, w, _embed_rows(w, ids))
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_forward_single_token_attention_returns_v():
    """One token at position 0: each head's only visible key is its own, the
    softmax weight is 1, and attention returns the cached V row of the KV
    head h // (n_heads / n_kv_heads) -- Q, K and RoPE drop out.  With the
    FFN written out (SiLU(gate) * up, down, residual), one layer has a closed
    form; two layers apply it twice.  Catches a swapped attn/ffn norm
    weight, a wrong GQA head, a missing residual and V being rotated."""
    cfg, w = _small_model(22)
    x = _embed_rows(w, [7])
    for l in range(cfg.n_layers):
        p = "blk.%d." % l
        v = _norm(x, w[p + "attn_norm"][1], cfg.eps) @ _deq(w, p + "attn_v").T
        hd, group = cfg.head_dim, cfg.n_heads // cfg.n_kv_heads
        a = np.concatenate([v[:, (h // group) * hd:(h // group + 1) * hd] for h in range(cfg.n_heads)], axis=1)
        x = x + a @ _deq(w, p + "attn_output").T
        xn = _norm(x, w[p + "ffn_norm"][1], cfg.eps)
        g, u = xn @ _deq(w, p + "ffn_gate").T, xn @ _deq(w, p + "ffn_up").T
        x = x + (g / (1.0 + np.exp(-g)) * u) @ _deq(w, p + "ffn_down").T
    want = _head(cfg, w, x)
    got, _ = _run(cfg, w, [7])
    assert np.allclose(got, want, rtol=2e-5, atol=2e-5 * np.abs(want).max())
    # and Q, K truly drop out: zeroing them changes nothing for one token
    w0 = _zeroed(w, ["blk.%d.%s" % (l, s) for l in range(cfg.n_layers) for s in ("attn_q", "attn_k")])
    assert np.array_equal(_run(cfg, w0, [7])[0], got)


def test_forward_zero_gate_removes_the_ffn():
    """Zero gate weights: SiLU(0) = 0, so the FFN adds exactly nothing, and
    the result equals the model with W_down = 0 as well (for any prompt),
    while W_up cannot matter.  With the attention also removed (W_o = 0) the
    logits are head(rmsnorm(embedding)) again."""
    cfg, w = _small_model(23)
    ids = [3, 9, 9, 30, 1]
    layers = range(cfg.n_layers)
    wg = _zeroed(w, ["blk.%d.ffn_gate" % l for l in layers])
    a, _ = _run(cfg, wg, ids)
    b, _ = _run(cfg, _zeroed(wg, ["blk.%d.ffn_down" % l for l in layers]), ids)
    c, _ = _run(cfg, _zeroed(wg, ["blk.%d.ffn_up" % l for l in layers]), ids)
    assert np.array_equal(a, b) and np.array_equal(a, c)
    full, _ = _run(cfg, w, ids)
    assert not np.allclose(full, a, rtol=1e-3)                       # the FFN does contribute normally
    d, _ = _run(cfg, _zeroed(wg, ["blk.%d.attn_output" % l for l in layers]), ids)
    want = _head(cfg, w, _embed_rows(w, ids))
    assert np.allclose(d, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_forward_caches_rotated_keys_and_plain_values():
    """Layer 0's input for a token is its embedding wherever it stands, so
    the cached rows of one token at positions 0 and 3 are related in closed
    form: V rows equal, and each K pair (2i, 2i+1), read as a complex
    number, turned by the angle 3 * theta^(-2i/head_dim).  Catches K stored
    before RoPE (rows equal), V rotated, RoPE at the wrong position and
    half-split pairs."""
    cfg, w = _small_model(24, n_layers=1)
    ids = [17, 2, 30, 17]
    max_len = 8
    kv = [(np.zeros((max_len, cfg.kv_dim), np.float32), np.zeros((max_len, cfg.kv_dim), np.float32))]
    ol.Model(cfg, w).forward(ids, 0, kv, ol.rope_table(max_len, cfg.head_dim, cfg.theta))
    K, V = kv[0]
    assert np.array_equal(V[0], V[3]) and not np.array_equal(V[0], V[1])
    assert not np.allclose(K[0], K[3])
    hd = cfg.head_dim
    ang = 3.0 * cfg.theta ** (-np.arange(hd // 2) * 2.0 / hd)
    k0 = K[0].astype(np.float64).reshape(cfg.n_kv_heads, hd // 2, 2)
    k3 = K[3].astype(np.float64).reshape(cfg.n_kv_heads, hd // 2, 2)
    z0, z3 = k0[..., 0] + 1j * k0[..., 1], k3[..., 0] + 1j * k3[..., 1]
    assert np.allclose(z3, z0 * np.exp(1j * ang), atol=2e-6 * np.abs(z0).max())
    assert not K[4:].any() and not V[4:].any()           # nothing past the prompt is written


def test_forward_last_row_sees_key_order_through_rope():
    """One layer: without RoPE the last query's attention is a function of
    the set of earlier keys, so swapping the first two tokens could not
    change the last row.  With RoPE it does."""
    cfg, w = _small_model(26, n_layers=1)
    a, m = _run(cfg, w, [4, 40, 11, 2])
    b, _ = _run(cfg, w, [40, 4, 11, 2], model=m)
    assert not np.allclose(a[-1], b[-1], rtol=1e-4)


def test_forward_prefill_rows_equal_incremental_rows():
    """Every row of a multi-token forward (last_only=False) equals the
    logits of the same position decoded one token at a time."""
    cfg, w = _small_model(25)
    ids = [8, 1, 44, 20]
    full, m = _run(cfg, w, ids, max_len=8)
    kv = [(np.zeros((8, cfg.kv_dim), np.float32), np.zeros((8, cfg.kv_dim), np.float32))
          for _ in range(cfg.n_layers)]
    table = ol.rope_table(8, cfg.head_dim, cfg.theta)
    for i, t in enumerate(ids):
        row = m.forward([t], i, kv, table)
        assert np.allclose(row[0], full[i], rtol=1e-5, atol=1e-5 * np.abs(full[i]).max()), i
