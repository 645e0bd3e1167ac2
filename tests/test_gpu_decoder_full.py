"""The Llama decoder at its full shape -- 32 layers, hidden 4096, 32 query /
8 KV heads of 128, SwiGLU 14336, vocab 32000, Q4_K weights with a Q6_K head
-- against the oracle decoder (oracle/llama.py, Model.forward).

Random-init weights with two distinct layer sets (layer l uses set l % 2; the
device still holds 32 separate layer copies, and the oracle keeps each set's
dequantized matrices once).

  * Teacher-forced logits: a prompt, then decode steps whose input token is
    the oracle's greedy token (written to the device before each step), two
    launched eagerly and two replayed from the captured graph; the logits of
    the prefill and of every step against the oracle's, normwise.
      - 8-token prompt: the prefill matmuls run on the matvec kernels, whose
        arithmetic is fp32-equivalent (at most 1.5e-6 normwise per product
        against fp64), as is every other operator.  The same 32 layers and
        head amplify a per-product error about 17-fold (the ratio of the
        fp16 figures below), so about 2.5e-5 is expected; measured 1.1e-5 to
        1.5e-5.  Bound TOL_FP32 = 6e-5.
      - 16-token prompt: the prefill matmuls run on the GEMM, which rounds X
        and the dequantized W to fp16 (2.9e-4 normwise per product at these
        shapes).  Through 32 layers and the head that grows to 5.1e-3 on the
        prefill logits and 3.5e-3 to 4.1e-3 on the decode steps (they read
        the prefill's K/V rows): figures of the oracle itself run with its
        multi-row matmuls' operands rounded to fp16, at this seed; measured
        on the GPU 4.9e-3, then 4.2e-3 to 3.5e-3.  Bound TOL_FP16 = 1e-2.
      - 512-token prompt (the benchmark's): the prefill takes the paths a
        short prompt never reaches -- the gate|up GEMM on 512-row tiles, the
        down GEMM split over K with its summing pass, attention query tiles
        whose key range is split between two halves of a workgroup -- then
        four teacher-forced decode steps over the 512 cached rows.  The
        oracle run with its multi-row matmuls' operands rounded to fp16
        (the only rounding that differs) is 5.9e-3 from the exact oracle on
        the prefill logits at this seed and 3.5e-3 to 4.2e-3 on the decode
        steps, about the size it is at 16 tokens: the per-product rounding
        does not grow with the prompt.  Measured on the GPU 5.8e-3, then
        4.2e-3 to 3.5e-3.  Bound TOL_FP16.
  * The benchmark's workload, a 512-token prompt and 128 greedy tokens:
    graph replays give the same tokens and final logits, bit for bit, as the
    same steps launched eagerly.
"""
import numpy as np
import pytest

from aihost_amd import _native as nat
from aihost_amd import llama
from oracle import llama as ol

pytestmark = pytest.mark.gpu

CFG = llama.LLAMA_8B_SHAPE
TOL_FP32 = 6e-5
TOL_FP16 = 1e-2


@pytest.fixture(scope="module")
def full_model(device):
    w = llama.synth_weights(CFG, seed=11, distinct_layers=2)
    dw = llama.DeviceWeights(device, w)
    yield ol.Model(CFG, w), dw          # one oracle model: its dequantized matrices are kept across tests
    dw.dispose()


def rel(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(b.astype(np.float64)))


def set_token(device, dec, tok):
    t = np.array([tok], dtype=np.int32)
    nat.check(nat.lib().aih_memcpy_h2d(device.handle, dec.token, t.ctypes.data, 4), "token")


def teacher_forced_errors(device, m, dw, n_prompt, steps=4, seed=12):
    max_len = n_prompt + steps
    ids = np.random.default_rng(seed).integers(0, CFG.vocab, n_prompt).astype(np.int32)
    dec = llama.LlamaDecoder(device, CFG, dw, max_len, n_prompt)
    try:
        first = dec.prefill(ids)
        got = dec.read_logits()
        assert first == int(np.argmax(got))
        kv = [(np.zeros((max_len, CFG.kv_dim), np.float32), np.zeros((max_len, CFG.kv_dim), np.float32))
              for _ in range(CFG.n_layers)]
        table = ol.rope_table(max_len, CFG.head_dim, CFG.theta)
        ref = m.forward(list(ids), 0, kv, table)[0]
        errs = [rel(got, ref)]
        for step in range(steps):
            tok = ol.argmax(ref)
            set_token(device, dec, tok)
            dec.decode(1, use_graph=step >= steps // 2)     # two eager steps, then graph replays
            got = dec.read_logits()
            assert np.all(np.isfinite(got))
            ref = m.forward([tok], n_prompt + step, kv, table)[0]
            errs.append(rel(got, ref))
        print("%d-token prompt: normwise logits error, prefill then decode steps:" % n_prompt,
              ["%.2e" % e for e in errs])
        return errs
    finally:
        dec.dispose()


@pytest.mark.timeout(600)
def test_full_shape_fp32_path_matches_oracle(device, full_model):
    m, dw = full_model
    assert CFG.n_layers == 32 and CFG.dim == 4096 and CFG.ffn == 14336 and CFG.vocab == 32000
    assert dw["blk.31.ffn_down"][0] == nat.Q4_K and dw["output"][0] == nat.Q6_K
    errs = teacher_forced_errors(device, m, dw, 8)
    assert max(errs) < TOL_FP32, errs


@pytest.mark.timeout(600)
def test_full_shape_gemm_prefill_matches_oracle(device, full_model):
    m, dw = full_model
    errs = teacher_forced_errors(device, m, dw, 16)
    assert max(errs) < TOL_FP16, errs


@pytest.mark.timeout(900)
def test_full_workload_prompt_matches_oracle(device, full_model):
    m, dw = full_model
    if device.info().compute_units == 256:
        # the tilings this prompt length is here for
        assert nat.qgemm_plan(device.handle, 2 * CFG.ffn, CFG.dim, 512) == (512, 1)
        assert nat.qgemm_plan(device.handle, CFG.dim, CFG.ffn, 512)[1] > 1
    errs = teacher_forced_errors(device, m, dw, 512, steps=4)
    assert max(errs) < TOL_FP16, errs


@pytest.mark.timeout(600)
def test_full_workload_graph_replays_equal_eager_steps(device, full_model):
    _, dw = full_model
    prompt, gen = 512, 128
    ids = np.random.default_rng(43).integers(0, CFG.vocab, prompt).astype(np.int32)
    runs = []
    for use_graph in (False, True):
        dec = llama.LlamaDecoder(device, CFG, dw, prompt + gen, prompt)
        try:
            first = dec.prefill(ids)
            dec.decode(gen, use_graph=use_graph)
            toks = dec.tokens(gen + 1).copy()
            runs.append((first, toks, dec.read_logits().copy()))
        finally:
            dec.dispose()
    (f0, t0, l0), (f1, t1, l1) = runs
    assert f0 == f1 == t0[0]
    assert np.array_equal(t0, t1)
    assert np.array_equal(l0, l1)
    assert t0.min() >= 0 and t0.max() < CFG.vocab
    assert int(np.argmax(l0)) == t0[-1]
