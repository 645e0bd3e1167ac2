"""CPU restatement (numpy) of the reference's Llama decoder operators and
forward pass -- the checker for the HIP decoder path.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by the smoke check and by the
CPU-baseline leg of bench.py, never by the library itself.

Operators (paths relative to the reference repository):
  rmsnorm        AIHost/AIHost/Compute/ComputeShaders.cs:247-278 (LayerNorm
                 shader: x / sqrt(mean(x^2) + eps) * w), eps 1e-5 from
                 ComputeOps.cs:1261
  rope_table     ComputeShaders.cs:517-543 (rope_full: freq = 1/pow(theta,
                 2i/d), angle = pos * freq, fp32); cos/sin taken in float64
                 and rounded, where the GLSL leaves their precision open
  rope           the same shader: interleaved pairs (2i, 2i+1),
                 y0 = x0*c - x1*s, y1 = x0*s + x1*c in fp32
  attention      ComputeOps.MultiHeadAttention (ComputeOps.cs:1055-1102):
                 per head, scores = Q_h K_h^T * (1/sqrt(head_dim)), causal mask
                 j > start + i (ComputeShaders.cs: causal_mask), row softmax,
                 times V_h; KV head = h / (n_heads / n_kv_heads); the decode
                 kernel FusedMHAGenerate (ComputeShaders.cs:656-733) computes
                 the same for one row.  Evaluated in float64.
  silu_mul       ComputeShaders.cs:280-307 (x * (1/(1+exp(-x)))) followed by
                 the element-wise Multiply of ComputeOps.FeedForward
                 (ComputeOps.cs:1218-1241), fp32
  embed          ComputeOps.EmbeddingLookupFromQuantized (ComputeOps.cs:1399-1454):
                 dequantized rows of the table (the oracle's dequantizer)
  argmax         greedy choice over the last logits row (InferenceEngine.cs:
                 340-390 with a greedy configuration): first maximum, NaN never
                 wins
  forward        ComputeOps.TransformerLayer (ComputeOps.cs:1250-1356) per layer,
                 then TransformerBase.ForwardHead (TransformerBase.cs:168-191):
                 output norm and head matmul

Parity pins (tests/test_oracle_llama.py): closed forms and invariants --
RMSNorm of scaled and constant rows, RoPE at position 0 (identity), norm
preservation, composition of rotations and a hand-computed pair rotation,
attention with one key, equal keys, causality and the GQA head mapping,
SiLU at known points, argmax ties -- each chosen so that a plausible slip
(half-split instead of interleaved pairs, a missing scale, a wrong KV head,
an off-by-one mask) fails one of them.  The composition in Model.forward is
pinned by special cases with closed forms: W_o = W_down = 0 makes every
layer the identity (logits = head(rmsnorm(embedding))); one token at
position 0 makes attention return V of the grouped KV head, so a layer is
written out by hand; zero gate weights remove the FFN exactly; the cached K
rows of one token at two positions are the same complex pairs turned by the
position difference, V rows equal; swapping two earlier tokens changes a
one-layer model's last row only through RoPE.  Planted slips (a dropped
residual, swapped norm weights, RoPE after the cache store, a rotated V,
gate and up swapped, no output norm) each fail at least one of them.
"""
import numpy as np

from . import oracle as orc

f32 = np.float32


def rmsnorm(x, w, eps=1e-5):
    """Row-wise RMSNorm in fp32 with the sum of squares taken exactly."""
    x = np.asarray(x, dtype=f32)
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    rms = np.sqrt((ss / x.shape[-1] + eps)).astype(f32)
    return (x / rms) * np.asarray(w, dtype=f32)


def rope_table(max_pos, head_dim, theta=10000.0):
    """[max_pos, head_dim/2, 2] of (cos, sin), angle in the reference's fp32 steps."""
    half = head_dim // 2
    i = np.arange(half)
    e = (2 * i).astype(f32) / f32(head_dim)
    pw = np.power(np.float64(f32(theta)), e.astype(np.float64)).astype(f32)
    freq = f32(1.0) / pw
    pos = np.arange(max_pos).astype(f32)
    ang = pos[:, None] * freq[None, :]           # fp32 product
    out = np.empty((max_pos, half, 2), dtype=f32)
    out[..., 0] = np.cos(ang.astype(np.float64)).astype(f32)
    out[..., 1] = np.sin(ang.astype(np.float64)).astype(f32)
    return out


def rope(x, positions, n_heads, head_dim, table):
    """x: [rows, n_heads*head_dim]; row r rotated at positions[r]."""
    x = np.asarray(x, dtype=f32).reshape(len(positions), n_heads, head_dim // 2, 2)
    cs = table[np.asarray(positions)][:, None, :, :]          # [rows, 1, half, 2]
    c, s = cs[..., 0], cs[..., 1]
    x0, x1 = x[..., 0], x[..., 1]
    y = np.empty_like(x)
    y[..., 0] = x0 * c - x1 * s
    y[..., 1] = x0 * s + x1 * c
    return y.reshape(len(positions), n_heads * head_dim)


def attention(q, kc, vc, positions, n_heads, n_kv_heads, head_dim, scale=None):
    """q: [rows, n_heads*hd]; kc/vc: [L, n_kv_heads*hd] (cache rows 0..);
    query row i attends to cache rows 0..positions[i]."""
    if scale is None:
        scale = 1.0 / np.sqrt(np.float32(head_dim))
    q = np.asarray(q, dtype=np.float64).reshape(len(positions), n_heads, head_dim)
    k = np.asarray(kc, dtype=np.float64).reshape(-1, n_kv_heads, head_dim)
    v = np.asarray(vc, dtype=np.float64).reshape(-1, n_kv_heads, head_dim)
    group = n_heads // n_kv_heads
    pos = np.asarray(positions)
    L = int(pos.max()) + 1
    # row r sees cache rows 0..pos[r]: later keys get weight exactly 0
    mask = np.arange(L)[None, :] > pos[:, None]
    out = np.empty_like(q)
    for h in range(n_heads):
        kvh = h // group
        s = (q[:, h, :] @ k[:L, kvh, :].T) * float(scale)
        s[mask] = -np.inf
        s = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h, :] = (s / s.sum(axis=1, keepdims=True)) @ v[:L, kvh, :]
    return out.reshape(len(positions), n_heads * head_dim).astype(f32)


def silu_mul(g, u):
    g = np.asarray(g, dtype=f32)
    with np.errstate(over="ignore"):
        sig = f32(1.0) / (f32(1.0) + np.exp(-g))
    return (g * sig) * np.asarray(u, dtype=f32)


def embed(qtype, table, vocab, dim, ids):
    rb = orc.row_bytes(qtype, dim)
    out = np.zeros((len(ids), dim), dtype=f32)
    t = np.asarray(table, dtype=np.uint8)
    for i, tok in enumerate(ids):
        if 0 <= tok < vocab:
            out[i] = orc.dequantize(qtype, t[tok * rb:(tok + 1) * rb], dim)
    return out


def argmax(x):
    x = np.asarray(x, dtype=f32)
    return int(np.argmax(np.where(np.isnan(x), -np.inf, x)))


class Model:
    """A Llama decoder held as quantized host weights (same layout as the GGUF
    tensors: rows = output features) -- the oracle twin of aihost_amd.llama."""

    def __init__(self, cfg, weights):
        self.cfg = cfg
        self.w = weights
        self._deq = {}

    def mat(self, name):
        """Dequantized [out, in] matrix of a quantized weight, held as float64
        (exact: every dequantized value is a float32).  Cached per packed
        array, so layers that share one array (synthetic models with a few
        distinct layer sets) share one matrix."""
        qtype, data, n, k = self.w[name]
        key = id(data)
        if key not in self._deq:
            m = orc.dequantize(qtype, data, n * k).reshape(n, k).astype(np.float64)
            self._deq[key] = (data, m)          # the array is kept, so its id stays unique
        return self._deq[key][1]

    def vec(self, name):
        """A fp32 weight vector (norm weights)."""
        return np.asarray(self.w[name][1], dtype=f32).reshape(-1)

    def matmul(self, name, x):
        """x @ W^T in float64, rounded once to float32."""
        return (np.asarray(x, dtype=np.float64) @ self.mat(name).T).astype(f32)

    def forward(self, ids, start, kv, table, last_only=True):
        """Embed ids at positions start.., run every layer (appending to the
        KV cache lists kv[l] = (K, V) arrays of cache rows), return logits of
        the last row (or every row)."""
        c = self.cfg
        qt, data, vocab, dim = self.w["token_embd"]
        x = embed(qt, data, vocab, dim, ids)
        pos = list(range(start, start + len(ids)))
        for l in range(c.n_layers):
            p = "blk.%d." % l
            xn = rmsnorm(x, self.vec(p + "attn_norm"), c.eps)
            q = self.matmul(p + "attn_q", xn)
            k = self.matmul(p + "attn_k", xn)
            v = self.matmul(p + "attn_v", xn)
            q = rope(q, pos, c.n_heads, c.head_dim, table)
            k = rope(k, pos, c.n_kv_heads, c.head_dim, table)
            K, V = kv[l]
            K[start:start + len(ids)] = k
            V[start:start + len(ids)] = v
            a = attention(q, K, V, pos, c.n_heads, c.n_kv_heads, c.head_dim)
            x = x + self.matmul(p + "attn_output", a)
            xn = rmsnorm(x, self.vec(p + "ffn_norm"), c.eps)
            g = silu_mul(self.matmul(p + "ffn_gate", xn), self.matmul(p + "ffn_up", xn))
            x = x + self.matmul(p + "ffn_down", g)
        rows = x[-1:] if last_only else x
        xn = rmsnorm(rows, self.vec("output_norm"), c.eps)
        return self.matmul("output", xn)
