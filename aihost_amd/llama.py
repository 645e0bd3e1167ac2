"""Llama-family decoder on the HIP library: prefill and greedy decode with
every weight matmul on the fused quantized kernels.

Mirrors the reference's layer and head (paths relative to the reference
repository):
  LlamaDecoder.layer     LlamaFormat.ApplyLayer (AIHost/AIHost/Compute/Formats/
                         LlamaFormat.cs:24-87) -> ComputeOps.TransformerLayer
                         (AIHost/AIHost/Compute/ComputeOps.cs:1250-1356):
                         x -> RMSNorm -> Q/K/V -> RoPE(Q, K) -> KV cache ->
                         GQA attention -> W_o -> +x -> RMSNorm -> SiLU(gate)*up
                         -> down -> +x
  LlamaDecoder.head      TransformerBase.ForwardHead (TransformerBase.cs:168-191):
                         output norm, then the vocabulary projection
  LlamaDecoder.prefill / decode
                         InferenceEngine.RunGenerationLoop (AIHost/AIHost/Inference/
                         InferenceEngine.cs:213-334) with greedy sampling

Routing seam.  The reference dequantizes every weight to F32 per use
(TransformerBase.TempF32, TransformerBase.cs:254-271) before MatMulWeights;
here quantized weights go straight to aih_matmul_weights_q (the fused matvec
for M <= 8, the fused GEMM above), and the KV cache is preallocated and
appended in place instead of concatenated (InferenceEngine.cs:598-622).

Differences of scope, on purpose: prefill computes logits for the last row
only (the greedy choice reads nothing else); a decode step is captured once
into a HIP graph -- its position and input token live in device memory and
the argmax step advances them -- and replayed per token.
"""
import ctypes
from dataclasses import dataclass

import numpy as np

from . import _native as nat
from .compute import HipComputeDevice, fill_normal, quantize, row_bytes  # noqa: F401

Q4_K, Q6_K, F32 = nat.Q4_K, nat.Q6_K, nat.F32


@dataclass(frozen=True)
class LlamaConfig:
    n_layers: int
    dim: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    eps: float = 1e-5
    theta: float = 10000.0

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim


# 32 layers, hidden 4096, 32/8 heads of 128, SwiGLU 14336, vocab 32000.
LLAMA_8B_SHAPE = LlamaConfig(n_layers=32, dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=32000)


def layer_tensors(cfg):
    """(suffix, qtype, rows, cols) of the weights of one layer; rows are
    output features (GGUF dims [cols, rows])."""
    d, kv, f = cfg.dim, cfg.kv_dim, cfg.ffn
    qd = cfg.n_heads * cfg.head_dim
    return [("attn_norm", F32, 1, d), ("attn_q", Q4_K, qd, d), ("attn_k", Q4_K, kv, d), ("attn_v", Q4_K, kv, d),
            ("attn_output", Q4_K, d, qd), ("ffn_norm", F32, 1, d), ("ffn_gate", Q4_K, f, d), ("ffn_up", Q4_K, f, d),
            ("ffn_down", Q4_K, d, f)]


def synth_weights(cfg, seed=42, distinct_layers=None, head_type=Q6_K):
    """Host weights of a random-init decoder: matrices N(0, 0.02) quantized to
    Q4_K (the head to `head_type`), norm weights 1 + N(0, 0.02) in fp32.

    Returns {name: (qtype, array, rows, cols)} with GGUF tensor names.  With
    distinct_layers = m, only m layer sets are generated and layer l reuses set
    l % m (the device still holds a separate copy per layer)."""
    m = cfg.n_layers if distinct_layers is None else max(1, min(distinct_layers, cfg.n_layers))
    out = {}
    s = seed

    def make(qtype, rows, cols):
        nonlocal s
        s += 1
        if qtype == F32:
            return 1.0 + fill_normal(s, rows * cols, 0.0, 0.02)
        return quantize(qtype, fill_normal(s, rows * cols, 0.0, 0.02), rows, cols)

    out["token_embd"] = (Q4_K, make(Q4_K, cfg.vocab, cfg.dim), cfg.vocab, cfg.dim)
    sets = []
    for _ in range(m):
        sets.append({suf: (qt, make(qt, r, c), r, c) for suf, qt, r, c in layer_tensors(cfg)})
    for l in range(cfg.n_layers):
        for suf, t in sets[l % m].items():
            out["blk.%d.%s" % (l, suf)] = t
    out["output_norm"] = (F32, make(F32, 1, cfg.dim), 1, cfg.dim)
    out["output"] = (head_type, make(head_type, cfg.vocab, cfg.dim), cfg.vocab, cfg.dim)
    return out


# Weights of a layer that share their input and are stored in one device
# buffer, so that a decode step runs one matvec over them:
#   "concat"      Q|K|V back to back (outputs land back to back too); the
#                 members stay reachable as views of the buffer
#   "interleave"  gate and up rows interleaved (row 2i = gate row i, row
#                 2i+1 = up row i), the layout aih_qmatvec_fused's SiLU-pairs
#                 epilogue and aih_silu_mul_pairs read; the members are not
#                 separate matrices any more
FUSED_GROUPS = (("attn_qkv", "concat", ("attn_q", "attn_k", "attn_v")),
                ("ffn_gate_up", "interleave", ("ffn_gate", "ffn_up")))


def interleave_rows(arrs, rows):
    """Packed row-major matrices of `rows` rows each -> one byte array with
    their rows interleaved: row i of matrix j lands at row i*len(arrs) + j
    (for gate/up: row 2i = gate row i, row 2i+1 = up row i)."""
    mats = [np.ascontiguousarray(a).reshape(-1).view(np.uint8) for a in arrs]
    if any(m.size != mats[0].size for m in mats) or mats[0].size % rows:
        raise ValueError("interleave_rows: matrices of different sizes or a size not divisible by rows")
    rb = mats[0].size // rows
    return np.stack([m.reshape(rows, rb) for m in mats], axis=1).reshape(-1)


class DeviceWeights:
    """Every tensor of a weight dict in device memory, packed blocks verbatim
    (as aih_upload_tensor places them from a GGUF file).  The matrices of each
    FUSED_GROUPS group of a layer share one buffer, reachable under the group
    name ("blk.<l>.attn_qkv", ...), when they have one format and width (and,
    to interleave, one height); otherwise they are stored separately.
    Entries are (qtype, device pointer, rows, cols)."""

    def __init__(self, device, weights):
        self.device = device
        self.t = {}
        self._owned = []
        grouped = {}
        for name in weights:
            if name.startswith("blk."):
                pre, suf = name.rsplit(".", 1)
                for gname, layout, members in FUSED_GROUPS:
                    if suf in members:
                        grouped.setdefault((pre + "." + gname, layout, members), {})[suf] = name
        try:
            done = set()
            for (gname, layout, members), found in grouped.items():
                if len(found) != len(members):
                    continue
                names = [found[m] for m in members]
                qts = {weights[n][0] for n in names}
                cols = {weights[n][3] for n in names}
                rows = {weights[n][2] for n in names}
                if len(qts) != 1 or len(cols) != 1 or (layout == "interleave" and len(rows) != 1):
                    continue
                arrs = [np.ascontiguousarray(weights[n][1]) for n in names]
                qt, c = qts.pop(), cols.pop()
                buf = self._alloc(sum(a.nbytes for a in arrs))
                if layout == "concat":
                    off = 0
                    for n, a in zip(names, arrs):
                        self._upload(buf.get_pointer() + off, a, n)
                        self.t[n] = (qt, buf.get_pointer() + off, weights[n][2], c)
                        off += a.nbytes
                else:
                    self._upload(buf.get_pointer(), interleave_rows(arrs, rows.pop()), gname)
                done.update(names)
                self.t[gname] = (qt, buf.get_pointer(), sum(weights[n][2] for n in names), c)
            for name, (qt, arr, r, c) in weights.items():
                if name in done:
                    continue
                buf = self._alloc(np.ascontiguousarray(arr).nbytes)
                self._upload(buf.get_pointer(), arr, name)
                self.t[name] = (qt, buf.get_pointer(), r, c)
        except Exception:
            self.dispose()
            raise

    def _alloc(self, nbytes):
        b = self.device.create_buffer(max(16, nbytes))
        self._owned.append(b)
        return b

    def _upload(self, ptr, arr, name):
        a = np.ascontiguousarray(arr)
        nat.check(nat.lib().aih_upload_tensor(self.device.handle, ptr, a.ctypes.data, a.nbytes),
                  "aih_upload_tensor(%s)" % name)

    def __getitem__(self, name):
        return self.t[name]

    def __contains__(self, name):
        return name in self.t

    def ptr(self, name):
        return self.t[name][1]

    def nbytes(self):
        return sum(b.size for b in self._owned)

    def dispose(self):
        for b in self._owned:
            b.dispose()
        self._owned = []
        self.t = {}


class LlamaDecoder:
    """Prefill + greedy decode of one sequence of up to max_len positions."""

    def __init__(self, device, cfg, weights, max_len, max_prefill):
        if cfg.head_dim != 128:
            raise ValueError("the attention kernels need head_dim 128")
        if max_prefill > max_len:
            raise ValueError("max_prefill > max_len")
        self.dev, self.cfg, self.w = device, cfg, weights
        self.max_len, self.max_prefill = int(max_len), int(max_prefill)
        self.L = nat.lib()
        self.h = device.handle
        self._bufs = []
        c, P = cfg, self.max_prefill

        def buf(nbytes):
            b = device.create_buffer(max(16, int(nbytes)))
            self._bufs.append(b)
            return b.get_pointer()

        qd = c.n_heads * c.head_dim
        self.x, self.xn = buf(P * c.dim * 4), buf(P * c.dim * 4)
        self.q, self.att, self.tmp = buf(P * qd * 4), buf(P * qd * 4), buf(P * c.dim * 4)
        self.k, self.v = buf(P * c.kv_dim * 4), buf(P * c.kv_dim * 4)
        # prefill: gate and up (interleaved with a fused gate|up buffer), then
        # SiLU(gate) * up in self.up
        # (the fused prefill keeps the down GEMM's operand image in self.gate)
        self.gate = buf(max(P * 2 * c.ffn * 4, nat.operand_bytes(P, c.ffn)))
        self.up = buf(P * c.ffn * 4)
        # the attention output as the W_o GEMM's fp16 operand image (fused prefill)
        self.att16 = buf(nat.operand_bytes(P, qd))
        # outputs of the fused Q|K|V projection (one row in decode, up to
        # max_prefill rows in the fused prefill) and of the decode gate|up
        # (SiLU-pairs) matvec
        self.qkv = buf(P * (qd + 2 * c.kv_dim) * 4)
        self.gu = buf(c.ffn * 4)
        self.logits = buf(c.vocab * 4)
        self.kc = [buf(self.max_len * c.kv_dim * 4) for _ in range(c.n_layers)]
        self.vc = [buf(self.max_len * c.kv_dim * 4) for _ in range(c.n_layers)]
        self.scratch_floats = int(self.L.aih_attention_scratch_floats(c.n_heads, self.max_len))
        nat.check(self.scratch_floats if self.scratch_floats < 0 else 0, "aih_attention_scratch_floats")
        self.scratch = buf(self.scratch_floats * 4)
        self.table = buf(self.max_len * c.head_dim * 4)
        self.ids = buf(P * 4)
        self.token = buf(4)
        self.pos = buf(4)
        self.history_len = self.max_len
        self.history = buf(self.history_len * 4)
        self.scale = float(np.float32(1.0) / np.sqrt(np.float32(c.head_dim)))
        nat.check(self.L.aih_rope_table(self.h, self.table, self.max_len, c.head_dim, c.theta), "aih_rope_table")
        self.n_prompt = 0
        # host mirror of the device position: the next decode step runs at
        # this position (prefill sets it to the prompt length, every decode
        # step advances it, as the argmax step advances *pos on the device)
        self.position = 0
        self.graph = None
        # The SiLU-pairs epilogue pairs the row teams of a workgroup: 8 teams
        # for widths up to 4096, 4 up to 8192, 2 up to 16384; the fused gate|up
        # height 2*ffn must be a multiple of the team count.
        teams = 8 if c.dim <= 4096 else 4 if c.dim <= 8192 else 2 if c.dim <= 16384 else 0
        self.pairs_epilogue = teams > 0 and (2 * c.ffn) % teams == 0
        # the fused decode attention serves query groups of 1, 2, 4 or 8 heads
        self.fused_attention = c.n_heads // c.n_kv_heads in (1, 2, 4, 8)
        # prompts of more than 8 rows (the GEMM's range) run the fused prefill
        # layer (_prefill_layer_fused); False selects the separate operators
        self.fused_prefill = True

    # -- operators (thin checked wrappers)
    def _mm(self, name, X, M, Y):
        qt, ptr, n, k = self.w[name]
        nat.check(self.L.aih_matmul_weights_q(self.h, qt, ptr, n, k, X, M, Y), "matmul %s" % name)

    def _norm(self, name, X, Y, rows):
        nat.check(self.L.aih_rmsnorm(self.h, X, self.w.ptr(name), Y, rows, self.cfg.dim, self.cfg.eps),
                  "rmsnorm %s" % name)

    def _mmf(self, name, X, X2, pre, post, Y):
        """Decode matvec with a fused prologue (RMSNorm or SiLU*up) and
        epilogue (residual add or SiLU of gate/up pairs), aih_qmatvec_fused."""
        qt, ptr, n, k = self.w[name]
        nat.check(self.L.aih_qmatvec_fused(self.h, qt, ptr, n, k, X, X2, self.cfg.eps, pre, post, Y),
                  "fused matvec %s" % name)

    def _mmx(self, name, X, X2, pre, post, M, Y):
        """Prefill GEMM with a fused prologue (RMSNorm, SiLU*up, SiLU of
        gate/up pairs) and epilogue (residual add), aih_qgemm_fused."""
        qt, ptr, n, k = self.w[name]
        nat.check(self.L.aih_qgemm_fused(self.h, qt, ptr, n, k, X, X2, self.cfg.eps, M, pre, post, Y),
                  "fused GEMM %s" % name)

    def _prefill_layer_fused(self, l, rows, start, pos):
        """One layer over `rows` > 8 prompt rows in five GEMM-centred steps: the
        Q|K|V GEMM with the attention RMSNorm computed into its operand and
        RoPE and the cache store in its epilogue, attention reading the query block in place and
        writing the W_o GEMM's fp16 operand, the W_o GEMM adding into x, the gate|up GEMM with the FFN RMSNorm in its
        operand and SiLU(gate)*up written as the down GEMM's fp16 operand, the
        down GEMM adding into x.
        Bit for bit the result of the separate operators (layer()), except
        where a product of more than 256 rows splits K over workgroups here
        (aih_qgemm_fused: the 8B shape's down projection at 512 rows) and not
        there (aih_matmul_weights_q): its sums then differ by the fp32
        rounding of their order."""
        c, L, h, p = self.cfg, self.L, self.h, "blk.%d." % l
        qd = c.n_heads * c.head_dim
        ld = qd + 2 * c.kv_dim
        # the Q|K|V GEMM with RoPE and the cache store in its epilogue (aih_qgemm_fused + aih_rope_qkv)
        qt, wp, n, k = self.w[p + "attn_qkv"]
        assert n == ld
        nat.check(L.aih_qgemm_qkv_rope(h, qt, wp, k, self.x, self.w.ptr(p + "attn_norm"), c.eps, rows,
                                       nat.PRE_RMSNORM, self.qkv, self.kc[l], self.vc[l], c.n_heads, c.n_kv_heads,
                                       c.head_dim, start, pos, self.table, self.max_len, self.max_len),
                  "Q|K|V GEMM + rope -> cache")
        q = self.qkv
        nat.check(L.aih_attention_operand(h, q, ld, self.kc[l], self.vc[l], self.att16, rows, c.n_heads,
                                          c.n_kv_heads, c.head_dim, start, pos, self.max_len, self.scale),
                  "attention")
        self._mmx(p + "attn_output", self.att16, None, nat.PRE_F16_OPERAND, nat.POST_ACCUMULATE, rows, self.x)
        norm = self.w.ptr(p + "ffn_norm")
        if p + "ffn_gate_up" in self.w and (2 * c.ffn) % 128 == 0:
            # SiLU(gate)*up leaves the gate|up GEMM as the down GEMM's fp16 operand
            self._mmx(p + "ffn_gate_up", self.x, norm, nat.PRE_RMSNORM, nat.POST_SILU_PAIRS_F16, rows, self.gate)
            self._mmx(p + "ffn_down", self.gate, None, nat.PRE_F16_OPERAND, nat.POST_ACCUMULATE, rows, self.x)
        elif p + "ffn_gate_up" in self.w:
            self._mmx(p + "ffn_gate_up", self.x, norm, nat.PRE_RMSNORM, nat.POST_STORE, rows, self.gate)
            self._mmx(p + "ffn_down", self.gate, None, nat.PRE_SILU_PAIRS, nat.POST_ACCUMULATE, rows, self.x)
        else:
            self._mmx(p + "ffn_gate", self.x, norm, nat.PRE_RMSNORM, nat.POST_STORE, rows, self.gate)
            self._mmx(p + "ffn_up", self.x, norm, nat.PRE_RMSNORM, nat.POST_STORE, rows, self.up)
            self._mmx(p + "ffn_down", self.gate, self.up, nat.PRE_SILU_MUL, nat.POST_ACCUMULATE, rows, self.x)

    def layer(self, l, rows, start, pos):
        """One decoder layer over `rows` activation rows at positions start..
        (+*pos when pos is a device pointer).  A single row (decode) runs as
        six kernels: Q|K|V matvec with the attention RMSNorm fused in,
        attention with RoPE and the KV cache store fused in (two kernels),
        W_o matvec adding into x, gate|up matvec with the FFN RMSNorm fused in
        and SiLU(gate)*up as its epilogue, down matvec adding into x.
        More than 8 rows (prefill) run _prefill_layer_fused; with
        fused_prefill off, or up to 8 rows, the matmuls and the separate
        operators."""
        c, L, h, p = self.cfg, self.L, self.h, "blk.%d." % l
        qd = c.n_heads * c.head_dim
        if self.fused_prefill and rows > 8 and p + "attn_qkv" in self.w:
            self._prefill_layer_fused(l, rows, start, pos)
            return
        decode = rows == 1 and p + "attn_qkv" in self.w
        if decode:
            self._mmf(p + "attn_qkv", self.x, self.w.ptr(p + "attn_norm"), nat.PRE_RMSNORM, nat.POST_STORE,
                      self.qkv)
            q, k, v = self.qkv, self.qkv + qd * 4, self.qkv + (qd + c.kv_dim) * 4
        else:
            self._norm(p + "attn_norm", self.x, self.xn, rows)
            self._mm(p + "attn_q", self.xn, rows, self.q)
            self._mm(p + "attn_k", self.xn, rows, self.k)
            self._mm(p + "attn_v", self.xn, rows, self.v)
            q, k, v = self.q, self.k, self.v
        if decode and self.fused_attention:
            nat.check(L.aih_attention_decode_qkv(h, self.qkv, self.kc[l], self.vc[l], self.att, c.n_heads,
                                                 c.n_kv_heads, c.head_dim, start, pos, self.table, self.max_len,
                                                 self.max_len, self.scale, self.scratch, self.scratch_floats),
                      "rope + cache store + attention")
        else:
            nat.check(L.aih_rope_qkv(h, q, qd, k, c.kv_dim, v, c.kv_dim, self.kc[l], self.vc[l], rows, c.n_heads,
                                     c.n_kv_heads, c.head_dim, start, pos, self.table, self.max_len, self.max_len),
                      "rope q, k -> cache, v -> cache")
            nat.check(L.aih_attention(h, q, self.kc[l], self.vc[l], self.att, rows, c.n_heads, c.n_kv_heads,
                                      c.head_dim, start, pos, self.max_len, self.scale, self.scratch,
                                      self.scratch_floats), "attention")
        if decode:
            self._mmf(p + "attn_output", self.att, None, nat.PRE_NONE, nat.POST_ACCUMULATE, self.x)
        else:
            self._mm(p + "attn_output", self.att, rows, self.tmp)
            nat.check(L.aih_add(h, self.x, self.tmp, self.x, rows * c.dim), "residual")
        if decode and self.pairs_epilogue and p + "ffn_gate_up" in self.w:
            self._mmf(p + "ffn_gate_up", self.x, self.w.ptr(p + "ffn_norm"), nat.PRE_RMSNORM,
                      nat.POST_SILU_PAIRS, self.gu)
            self._mmf(p + "ffn_down", self.gu, None, nat.PRE_NONE, nat.POST_ACCUMULATE, self.x)
            return
        self._norm(p + "ffn_norm", self.x, self.xn, rows)
        if p + "ffn_gate_up" in self.w:
            self._mm(p + "ffn_gate_up", self.xn, rows, self.gate)
            nat.check(L.aih_silu_mul_pairs(h, self.gate, self.up, rows, c.ffn), "silu*up (pairs)")
        else:
            self._mm(p + "ffn_gate", self.xn, rows, self.gate)
            self._mm(p + "ffn_up", self.xn, rows, self.up)
            nat.check(L.aih_silu_mul(h, self.gate, self.up, self.up, rows * c.ffn), "silu*up")
        self._mm(p + "ffn_down", self.up, rows, self.tmp)
        nat.check(L.aih_add(h, self.x, self.tmp, self.x, rows * c.dim), "residual")

    def head(self, row_ptr, pos, hist_offset):
        """Output norm + vocabulary projection of one row, then the greedy
        token (and history / position update when pos is given)."""
        c = self.cfg
        self._mmf("output", row_ptr, self.w.ptr("output_norm"), nat.PRE_RMSNORM, nat.POST_STORE, self.logits)
        nat.check(self.L.aih_argmax(self.h, self.logits, c.vocab, self.token, pos, self.history, self.history_len,
                                    hist_offset), "argmax")

    def prefill(self, ids, read=True):
        """Run the prompt; return the first generated token (host int), or
        None with read=False (nothing waits for the device then)."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        n = len(ids)
        if not 0 < n <= self.max_prefill:
            raise ValueError("prompt of %d tokens (max %d)" % (n, self.max_prefill))
        c = self.cfg
        if self.graph is not None and n != self.n_prompt:   # recorded for another prompt length
            self.L.aih_graph_destroy(self.graph)
            self.graph = None
        nat.check(self.L.aih_memcpy_h2d(self.h, self.ids, ids.ctypes.data, ids.nbytes), "ids")
        qt, tb, vocab, dim = self.w["token_embd"]
        nat.check(self.L.aih_embed_q(self.h, qt, tb, vocab, dim, self.ids, n, self.x), "embed")
        for l in range(c.n_layers):
            self.layer(l, n, 0, None)
        # decode bookkeeping: the first token is history[0]; position becomes n
        p = np.array([n - 1], dtype=np.int32)
        nat.check(self.L.aih_memcpy_h2d(self.h, self.pos, p.ctypes.data, 4), "pos")
        self.n_prompt = n
        self.position = n
        self.head(self.x + (n - 1) * c.dim * 4, self.pos, n - 1)
        return self.read_token() if read else None

    def _step(self):
        """The launches of one greedy decode step, reading its token and
        position from device memory (what capture() records; no host
        bookkeeping)."""
        c = self.cfg
        qt, tb, vocab, dim = self.w["token_embd"]
        nat.check(self.L.aih_embed_q(self.h, qt, tb, vocab, dim, self.token, 1, self.x), "embed")
        for l in range(c.n_layers):
            self.layer(l, 1, 0, self.pos)
        self.head(self.x, self.pos, self.n_prompt - 1)

    def capture(self):
        """Record one decode step (_step) into a HIP graph (after prefill)."""
        if self.graph is not None:
            return self.graph
        g = ctypes.c_void_p()
        nat.check(self.L.aih_capture_begin(self.h), "aih_capture_begin")
        try:
            self._step()
        finally:
            st = self.L.aih_capture_end(self.h, ctypes.byref(g))
        nat.check(st, "aih_capture_end")
        self.graph = g.value
        return self.graph

    def decode(self, steps, use_graph=True):
        """Run `steps` greedy decode steps on the device; returns nothing (the
        tokens accumulate in the device history, see tokens()).  Raises
        ValueError, before anything runs, when the steps would pass max_len,
        counting the steps already decoded since the last prefill."""
        if self.n_prompt == 0:
            raise ValueError("decode before prefill")
        if steps < 0 or self.position + steps > self.max_len:
            raise ValueError("decode of %d steps from position %d passes max_len %d"
                             % (steps, self.position, self.max_len))
        if use_graph:
            g = self.capture()
            for _ in range(steps):
                nat.check(self.L.aih_graph_launch(self.h, g), "aih_graph_launch")
                self.position += 1
        else:
            for _ in range(steps):
                self._step()
                self.position += 1

    def decode_step(self):
        """One eager greedy decode step (decode(1, use_graph=False)): counted
        against max_len like every other step."""
        self.decode(1, use_graph=False)

    def read_token(self):
        t = np.empty(1, dtype=np.int32)
        nat.check(self.L.aih_memcpy_d2h(self.h, t.ctypes.data, self.token, 4), "token")
        return int(t[0])

    def tokens(self, count):
        """history[0..count): the first generated token and the decoded ones."""
        t = np.empty(count, dtype=np.int32)
        nat.check(self.L.aih_memcpy_d2h(self.h, t.ctypes.data, self.history, 4 * count), "history")
        return t

    def read_logits(self):
        out = np.empty(self.cfg.vocab, dtype=np.float32)
        nat.check(self.L.aih_memcpy_d2h(self.h, out.ctypes.data, self.logits, out.nbytes), "logits")
        return out

    def read(self, ptr, count):
        out = np.empty(count, dtype=np.float32)
        nat.check(self.L.aih_memcpy_d2h(self.h, out.ctypes.data, ptr, out.nbytes), "read")
        return out

    def dispose(self):
        if self.graph is not None:
            self.L.aih_graph_destroy(self.graph)
            self.graph = None
        for b in self._bufs:
            b.dispose()
        self._bufs = []
