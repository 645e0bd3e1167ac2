"""End-to-end Llama decoder (aihost_amd.llama) on a small random model vs the
oracle decoder (oracle/llama.py): prefill through the fused GEMM (M > 8),
decode through the fused matvec, a captured decode graph against the same
steps run eagerly.

Bars: the last-row logits of prefill and of every decode step within 3e-3
normwise of the oracle's (each layer has seven weight matmuls bounded by
1e-3 with fp16-rounded activations, and their errors compose over the
layers and the head); graph replays bit-identical to eager steps; greedy
tokens equal to the oracle's wherever the oracle's top-2 margin exceeds the
tolerance.
"""
import numpy as np
import pytest

from aihost_amd import llama
from oracle import llama as ol

pytestmark = pytest.mark.gpu

CFG = llama.LlamaConfig(n_layers=2, dim=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=1024, vocab=1000)
TOL = 3e-3


@pytest.fixture(scope="module")
def model(device):
    w = llama.synth_weights(CFG, seed=5)
    dw = llama.DeviceWeights(device, w)
    yield w, dw
    dw.dispose()


def oracle_setup(w, max_len):
    m = ol.Model(CFG, w)
    kv = [(np.zeros((max_len, CFG.kv_dim), np.float32), np.zeros((max_len, CFG.kv_dim), np.float32))
          for _ in range(CFG.n_layers)]
    return m, kv, ol.rope_table(max_len, CFG.head_dim, CFG.theta)


def rel(a, b):
    return np.linalg.norm(a - b) / np.linalg.norm(b)


def test_prefill_and_decode_match_oracle(device, model):
    w, dw = model
    max_len = 96
    ids = np.random.default_rng(3).integers(0, CFG.vocab, 40).astype(np.int32)
    dec = llama.LlamaDecoder(device, CFG, dw, max_len, 48)
    try:
        t0 = dec.prefill(ids)
        m, kv, table = oracle_setup(w, max_len)
        ref = m.forward(list(ids), 0, kv, table)[0]
        got = dec.read_logits()
        assert rel(got, ref) < TOL, rel(got, ref)
        assert t0 == int(np.argmax(got))
        tokens = [t0]
        for step in range(6):
            dec.decode(1, use_graph=False)
            got = dec.read_logits()
            ref = m.forward([tokens[-1]], len(ids) + step, kv, table)[0]
            assert rel(got, ref) < TOL, (step, rel(got, ref))
            top = np.sort(ref)[-2:]
            tok = int(np.argmax(got))
            if top[1] - top[0] > TOL * np.linalg.norm(ref) / np.sqrt(ref.size) * 10:
                assert tok == int(np.argmax(ref)), step
            tokens.append(tok)
        assert list(dec.tokens(7)) == tokens
    finally:
        dec.dispose()


def test_graph_replays_equal_eager_steps(device, model):
    _, dw = model
    ids = np.random.default_rng(4).integers(0, CFG.vocab, 12).astype(np.int32)
    runs = []
    for use_graph in (False, True, True):
        dec = llama.LlamaDecoder(device, CFG, dw, 64, 16)
        try:
            dec.prefill(ids)
            dec.decode(9, use_graph=use_graph)
            runs.append((dec.tokens(10).copy(), dec.read_logits().copy()))
        finally:
            dec.dispose()
    for toks, lg in runs[1:]:
        assert np.array_equal(toks, runs[0][0])
        assert np.array_equal(lg, runs[0][1])


def test_second_prompt_recaptures(device, model):
    _, dw = model
    dec = llama.LlamaDecoder(device, CFG, dw, 64, 16)
    try:
        a = np.random.default_rng(6).integers(0, CFG.vocab, 10).astype(np.int32)
        b = np.random.default_rng(7).integers(0, CFG.vocab, 5).astype(np.int32)
        dec.prefill(a)
        dec.decode(3)
        first = dec.tokens(4).copy()
        dec.prefill(b)
        dec.decode(3)
        second = dec.tokens(4).copy()
        fresh = llama.LlamaDecoder(device, CFG, dw, 64, 16)
        try:
            fresh.prefill(b)
            fresh.decode(3, use_graph=False)
            assert np.array_equal(second, fresh.tokens(4))
        finally:
            fresh.dispose()
        assert first.shape == (4,)
    finally:
        dec.dispose()


def test_limits(device, model):
    _, dw = model
    dec = llama.LlamaDecoder(device, CFG, dw, 20, 16)
    try:
        with pytest.raises(ValueError):
            dec.prefill(np.zeros(17, np.int32))
        dec.prefill(np.zeros(16, np.int32))
        with pytest.raises(ValueError):
            dec.decode(5)
        dec.decode(1, use_graph=False)        # position 16
        dec.decode_step()                     # position 17: counted like decode()
        assert dec.position == 18
        with pytest.raises(ValueError):       # steps already decoded count
            dec.decode(3)
        dec.decode(2)                         # positions 18, 19: the last cache row
        with pytest.raises(ValueError):
            dec.decode(1, use_graph=False)
        with pytest.raises(ValueError):
            dec.decode_step()
        assert dec.position == 20
    finally:
        dec.dispose()
