"""Host-side pieces of the device decoder that need no GPU: the gate/up row
interleave the SiLU-pairs epilogue reads, and the weight synthesis layout."""
import numpy as np
import pytest

from aihost_amd import llama
from aihost_amd import _native as nat
from oracle import oracle as orc


def test_interleave_rows_layout():
    rows, rb = 5, 144
    g = np.arange(rows * rb, dtype=np.uint8).reshape(rows, rb)
    u = (g.astype(np.int32) * 7 % 251).astype(np.uint8)
    out = llama.interleave_rows([g, u], rows).reshape(2 * rows, rb)
    assert np.array_equal(out[0::2], g)
    assert np.array_equal(out[1::2], u)
    with pytest.raises(ValueError):
        llama.interleave_rows([g, u[:-1]], rows)


def test_interleaved_quantized_rows_dequantize_as_pairs():
    # the interleaved buffer is itself a valid packed matrix of 2*rows rows:
    # its even rows dequantize to the gate matrix, its odd rows to up
    rows, k = 6, 256
    gate = llama.quantize(nat.Q4_K, llama.fill_normal(1, rows * k, 0.0, 0.02), rows, k)
    up = llama.quantize(nat.Q4_K, llama.fill_normal(2, rows * k, 0.0, 0.02), rows, k)
    both = llama.interleave_rows([gate, up], rows)
    d = orc.dequantize(nat.Q4_K, both, 2 * rows * k).reshape(2 * rows, k)
    assert np.array_equal(d[0::2], orc.dequantize(nat.Q4_K, gate, rows * k).reshape(rows, k))
    assert np.array_equal(d[1::2], orc.dequantize(nat.Q4_K, up, rows * k).reshape(rows, k))


def test_synth_weights_shapes_and_sharing():
    cfg = llama.LlamaConfig(n_layers=3, dim=256, n_heads=2, n_kv_heads=1, head_dim=128, ffn=512, vocab=300)
    w = llama.synth_weights(cfg, seed=1, distinct_layers=2)
    for l in range(3):
        for suf, qt, r, c in llama.layer_tensors(cfg):
            t = w["blk.%d.%s" % (l, suf)]
            assert t[0] == qt and t[2] == r and t[3] == c
            if qt == nat.F32:
                assert t[1].size == r * c
            else:
                assert t[1].nbytes == r * llama.row_bytes(qt, c)
    # layer 2 reuses set 0
    assert w["blk.2.ffn_up"][1] is w["blk.0.ffn_up"][1]
    assert w["output"][0] == nat.Q6_K and w["token_embd"][2:] == (300, 256)
