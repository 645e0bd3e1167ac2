"""The reference's ComputeOps operators on the HIP device, in the reference's
own order and binding layout.

ComputeOps dispatches every operator through GetOrCreateKernel
(ComputeOps.cs:1362-1372), which hands one of ComputeShaders' GLSL sources to
IComputeDevice.CreateKernel.  On the HIP device each such source becomes a
kernel object that runs a library operation over the same bindings
(aihost_amd.compute.LibraryKernel); the tests here drive that table through
the mirror's ComputeOps, written as the reference writes its operators
(params structs, bindings, dispatch sizes):

- each operator against the oracle: Copy, ConcatAxis0 and EmbeddingLookup
  bit for bit, LayerNorm / RoPEFull / SiLU against the numpy restatement of
  their shaders, FusedMHAGenerate and the prefill attention against the
  fp64 attention, dequantization dispatched in chunks of 32768 groups with
  the element-offset buffer (ComputeOps.cs:761-861) bit for bit;
- a whole forward pass in ComputeOps.TransformerLayer order
  (ComputeOps.cs:1250-1356) with InferenceEngine's concatenating KV cache
  (InferenceEngine.cs:585-622), the quantized embedding lookup, the output
  norm and the head: a 5-token prompt and 3 decode steps against the
  oracle's Model.forward.  Every matmul has at most 8 rows (the
  fp32-equivalent matvec), attention is fp32, so the logits agree to about
  1e-5 normwise; bound 1e-4.
"""
import numpy as np
import pytest

from aihost_amd import _native as nat
from aihost_amd import compute as C
from aihost_amd import llama
from oracle import llama as ol

pytestmark = pytest.mark.gpu


@pytest.fixture()
def ops(device):
    o = C.ComputeOps(device)
    yield o
    o.flush()


def t(device, a):
    return C.Tensor.from_data(device, np.ascontiguousarray(a, np.float32))


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(np.asarray(b, np.float64)))


def test_copy_concat_add_mul_exact(device, ops):
    rng = np.random.default_rng(1)
    a, b = rng.standard_normal((7, 300)).astype(np.float32), rng.standard_normal((5, 300)).astype(np.float32)
    ta, tb = t(device, a), t(device, b)
    c = ops.clone(ta)
    cat = ops.concat(ta, tb, 0)
    assert cat.shape == (12, 300)
    s = ops.add(ta, c)
    m = ops.multiply(ta, c)
    with pytest.raises(NotImplementedError):
        ops.concat(ta, tb, 1)
    assert np.array_equal(c.read(), a)
    assert np.array_equal(cat.read(), np.concatenate([a, b]))
    assert np.array_equal(s.read(), a + a)
    assert np.array_equal(m.read(), a * a)
    for x in (ta, tb, c, cat, s, m):
        x.dispose()


def test_layer_norm_rope_silu(device, ops):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((6, 512)).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    tx, tw = t(device, x), t(device, w)
    ops.layer_norm(tx, tw)
    y = tx.read()
    assert np.max(np.abs(y - ol.rmsnorm(x, w)) / (np.abs(ol.rmsnorm(x, w)) + 1e-6)) < 1e-5
    # RoPE of 4 heads of 128 at positions 37..42 (start 37)
    q = rng.standard_normal((6, 512)).astype(np.float32)
    tq = t(device, q)
    ops.apply_rope_full(tq, 37, 4, 128)
    ref = ol.rope(q, list(range(37, 43)), 4, 128, ol.rope_table(64, 128))
    assert np.max(np.abs(tq.read() - ref)) < 1e-5
    g = (3.0 * rng.standard_normal(1000)).astype(np.float32)
    tg = t(device, g)
    ops.silu(tg)
    sref = ol.silu_mul(g, np.ones_like(g))
    assert np.max(np.abs(tg.read() - sref) / (np.abs(sref) + 1e-30)) < 2e-6
    for a in (tx, tw, tq, tg):
        a.dispose()


@pytest.mark.parametrize("seq,start", [(1, 40), (9, 32)])
def test_attention(device, ops, seq, start):
    """One row through FusedMHAGenerate (keys 0 .. kvSeqLen-1), more rows
    through the prefill route (row i sees keys 0 .. start + i)."""
    rng = np.random.default_rng(seq + start)
    nh, nkv, hd = 8, 2, 128
    L = start + seq
    q = rng.standard_normal((seq, nh * hd)).astype(np.float32)
    k = rng.standard_normal((L, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((L, nkv * hd)).astype(np.float32)
    tq, tk, tv = t(device, q), t(device, k), t(device, v)
    o = ops.multi_head_attention(tq, tk, tv, nh, start)
    ref = ol.attention(q, k, v, list(range(start, start + seq)), nh, nkv, hd)
    assert rel(o.read(), ref) < 1e-5
    for a in (tq, tk, tv, o):
        a.dispose()


def test_embedding_lookups(device, ops):
    rng = np.random.default_rng(3)
    vocab, dim = 300, 512
    tab = rng.standard_normal((vocab, dim)).astype(np.float32)
    ids = np.array([5, 0, 299, 5, 17], np.int32)
    tt = C.Tensor.from_data(device, tab, (dim, vocab))          # GGUF dims [dModel, vocab]
    e = ops.embedding_lookup(ids, tt)
    assert np.array_equal(e.read(), tab[ids])
    qtab = C.quantize(C.DataType.Q4_K, C.fill_normal(4, vocab * dim, 0.0, 0.02), vocab, dim)
    tq = C.Tensor.from_quantized(device, qtab, dim, vocab, C.DataType.Q4_K)
    eq = ops.embedding_lookup_from_quantized(ids, tq)
    assert np.array_equal(eq.read(), ol.embed(nat.Q4_K, qtab, vocab, dim, ids))
    for a in (tt, e, tq, eq):
        a.dispose()


@pytest.mark.parametrize("qtype,dt", [(nat.Q4_K, "DequantizeQ4K"), (nat.Q6_K, "DequantizeQ6K")])
def test_dequantize_in_chunks_with_element_offsets(device, ops, qtype, dt):
    """DequantizeInto's chunked dispatch (ComputeOps.cs:761-861): chunks of at
    most 32768 groups of 256 elements, each with its element offset in a
    one-word buffer."""
    n_rows, k = 300, 65536                       # 76800 groups: three chunks
    q = C.quantize(qtype, C.fill_normal(5, n_rows * k, 0.0, 0.02), n_rows, k)
    qb = device.create_buffer(q.nbytes)
    qb.write(q)
    out = device.create_buffer(n_rows * k * 4)
    total_groups = n_rows * k // 256
    kern = device.create_kernel(dt)
    for g0 in range(0, total_groups, 32768):
        groups = min(32768, total_groups - g0)
        off = ops._params("I", g0 * 256)
        kern.set_argument(0, qb)
        kern.set_argument(1, out)
        kern.set_argument(2, off)
        kern.dispatch([groups])
    got = out.read_range(0, n_rows * k, np.float32)
    assert np.array_equal(got.view(np.uint32), ol.orc.dequantize(qtype, q, n_rows * k).view(np.uint32))
    with pytest.raises(NotImplementedError):
        device.create_kernel("MatMulWeightsF32")
    qb.dispose()
    out.dispose()


CFG = llama.LlamaConfig(n_layers=2, dim=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=1024, vocab=1000)


def test_forward_in_reference_operator_order(device, ops):
    w = llama.synth_weights(CFG, seed=13)
    model = ol.Model(CFG, w)
    tensors = {}
    for name, (qt, data, r, c) in w.items():
        if qt == llama.F32:
            tensors[name] = C.Tensor.from_data(device, np.asarray(data, np.float32).reshape(-1))
        else:
            tensors[name] = C.Tensor.from_quantized(device, data, c, r, qt)
    cache = C.KVCache(ops)
    ids = list(np.random.default_rng(14).integers(0, CFG.vocab, 5))
    max_len = 16
    kv = [(np.zeros((max_len, CFG.kv_dim), np.float32), np.zeros((max_len, CFG.kv_dim), np.float32))
          for _ in range(CFG.n_layers)]
    table = ol.rope_table(max_len, CFG.head_dim, CFG.theta)

    def forward(tokens, start):
        # TransformerBase.Forward (TransformerBase.cs:193-246) on the HIP device
        x = ops.embedding_lookup_from_quantized(tokens, tensors["token_embd"], "embeddings")
        for l in range(CFG.n_layers):
            p = "blk.%d." % l
            nxt = ops.transformer_layer(x, tensors[p + "attn_norm"], tensors[p + "attn_q"], tensors[p + "attn_k"],
                                        tensors[p + "attn_v"], tensors[p + "attn_output"], tensors[p + "ffn_norm"],
                                        tensors[p + "ffn_gate"], tensors[p + "ffn_up"], tensors[p + "ffn_down"],
                                        CFG.n_heads, start, cache, l)
            ops._deferred.append(x.buffer)
            x = nxt
        ops.layer_norm(x, tensors["output_norm"])
        logits = ops.matmul_weights(x, tensors["output"], "logits")
        # InferenceEngine.ExtractLastToken (InferenceEngine.cs:336-342): Tensor.ReadRow
        last = logits.buffer.read_range((logits.shape[0] - 1) * CFG.vocab * 4, CFG.vocab, np.float32)
        ops._deferred += [x.buffer, logits.buffer]
        ops.flush()
        return last

    try:
        got = forward(ids, 0)
        ref = model.forward(ids, 0, kv, table)[0]
        errs = [rel(got, ref)]
        pos = len(ids)
        for _ in range(3):
            tok = ol.argmax(ref)
            got = forward([tok], pos)
            ref = model.forward([tok], pos, kv, table)[0]
            errs.append(rel(got, ref))
            pos += 1
        assert cache.sequence_length == pos
        print("reference-order forward, normwise logits error:", ["%.2e" % e for e in errs])
        assert max(errs) < 1e-4, errs
    finally:
        cache.dispose()
        for x in tensors.values():
            x.dispose()
