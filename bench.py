#!/usr/bin/env python3
"""Benchmark of the fused GGUF quantized matvec on one MI355X.

Headline workload: Q4_K decode matvec, W = 14336 x 4096 (GGUF dims
[4096, 14336], the FFN up-projection), batch 1.  One step = one aih_qmatvec
over one weight copy.  Weights are synthetic N(0, 0.02) (seed 42) quantized to
Q4_K; x is N(0, 1) (seed 43).  Twelve copies of the weight (396 MB, more than
the 256 MB Infinity Cache) are used in rotation so every step streams its
weights from HBM.  Launches are captured once in a HIP graph of G launches
over the copies (G = the largest divisor of --steps up to 120) and the timed
region is exactly steps / G whole replays, bracketed by stream
synchronisation and HIP events on the library's stream.  Within a graph the
kernels run back to back; every launch pays the fixed cost of a kernel
boundary (reported beside the result: the same grid launched with nothing to
read).

Algorithmic bytes per step: packed W (14336 * 2304 B) + x (4096 * 4 B) +
y (14336 * 4 B) = 33,103,872 B.  value = those bytes / wall time per step;
roofline.achieved = those bytes / HIP-event time per launch.

Arithmetic: the weight codes are multiplied exactly (v_dot4_i32_i8) with x
held as three signed-byte limbs of a per-64-element fixed-point form, the
products summed in int32; block scales, mins and the limb weights are applied
in fp32 (normwise error against an fp64 product about 1e-6).

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "quant matvec GB/s (% HBM peak) + decode tokens/s, Q4_K 4096x14336, 1 GPU"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK = 2.5e15     # dense fp16 MFMA FLOP/s
COPIES = 12
GRAPH_LAUNCHES = 120     # most launches per captured graph
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "qmatvec_q4k_14336x4096_b1_hbm_traffic.md")


def graph_size(steps, cap=GRAPH_LAUNCHES):
    """Launches per graph: the largest divisor of `steps` up to `cap`, so that
    the timed region is a whole number of replays."""
    for g in range(max(1, min(cap, steps)), 0, -1):
        if steps % g == 0:
            return g
    return 1


def algorithmic_bytes(qtype, n, k, batch):
    from aihost_amd import compute as C
    return n * C.row_bytes(qtype, k) + batch * k * 4 + batch * n * 4


class MatvecBench:
    """Rotating weight copies + one captured graph of `launches` calls."""

    def __init__(self, dev, qtype, n, k, batch, copies=COPIES, launches=GRAPH_LAUNCHES, seed_w=42, seed_x=43):
        from aihost_amd import _native as nat
        from aihost_amd import compute as C
        self.nat, self.dev = nat, dev
        self.qtype, self.n, self.k, self.batch = qtype, n, k, batch
        self.packed = C.quantize(qtype, C.fill_normal(seed_w, n * k, 0.0, 0.02), n, k)
        self.x_host = C.fill_normal(seed_x, batch * k, 0.0, 1.0)
        self.w = [dev.create_buffer(self.packed.nbytes) for _ in range(copies)]
        for b in self.w:
            b.write(self.packed)
        self.x = dev.create_buffer(self.x_host.nbytes)
        self.x.write(self.x_host)
        self.y = dev.create_buffer(batch * n * 4)
        self._launch(self.w[0])   # sizes the library's workspace (batch 3..8), which cannot grow during capture
        dev.synchronize()
        L, h = nat.lib(), dev.handle
        nat.check(L.aih_capture_begin(h), "aih_capture_begin")
        for i in range(launches):
            self._launch(self.w[i % copies])
        g = ctypes.c_void_p()
        nat.check(L.aih_capture_end(h, ctypes.byref(g)), "aih_capture_end")
        self.graph = g.value
        self.copies = copies
        self.launches = launches

    def _launch(self, wbuf):
        st = self.nat.lib().aih_qmatvec(self.dev.handle, self.qtype, wbuf.get_pointer(), self.n, self.k,
                                        self.x.get_pointer(), self.k, self.y.get_pointer(), self.n, self.batch)
        self.nat.check(st, "aih_qmatvec")

    def replay(self, n):
        L, h = self.nat.lib(), self.dev.handle
        for _ in range(n):
            self.nat.check(L.aih_graph_launch(h, self.graph), "aih_graph_launch")

    def run(self, steps):
        """Exactly `steps` calls: steps / launches whole graph replays."""
        if steps % self.launches:
            raise ValueError("steps (%d) must be a multiple of the graph size (%d)" % (steps, self.launches))
        self.replay(steps // self.launches)

    def time(self, steps, warmup):
        """(wall ms, HIP-event ms) per call over `steps` calls, after at
        least `warmup` untimed calls (whole replays); the events bracket the
        timed replays on the library's stream."""
        L, h = self.nat.lib(), self.dev.handle
        self.replay(-(-warmup // self.launches))
        self.dev.synchronize()
        t0 = time.perf_counter()
        self.nat.check(L.aih_event_record(h, 0), "event")
        self.run(steps)
        self.nat.check(L.aih_event_record(h, 1), "event")
        self.dev.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3
        ev = ctypes.c_float()
        self.nat.check(L.aih_event_elapsed(h, 0, 1, ctypes.byref(ev)), "event")
        return wall_ms / steps, ev.value / steps

    def output(self):
        return self.y.read_range(0, self.batch * self.n, np.float32)

    def close(self):
        self.nat.lib().aih_graph_destroy(self.graph)
        for b in self.w + [self.x, self.y]:
            b.dispose()


class StreamBench:
    """The read ceiling: aih_probe_stream_read over rotating copies of a
    buffer (nbytes = 0: launches that read nothing), graphs as MatvecBench."""

    def __init__(self, dev, nbytes, nontemporal, copies=COPIES, launches=GRAPH_LAUNCHES):
        from aihost_amd import _native as nat
        self.nat, self.dev, self.nbytes = nat, dev, nbytes
        self.src = [dev.create_buffer(max(16, nbytes)) for _ in range(copies if nbytes else 1)]
        for b in self.src:
            nat.check(nat.lib().aih_memset(dev.handle, b.get_pointer(), 1, max(16, nbytes)), "aih_memset")
        self.out = dev.create_buffer(8192 * 4)
        L, h = nat.lib(), dev.handle
        self._launch(0, nontemporal)
        dev.synchronize()
        nat.check(L.aih_capture_begin(h), "aih_capture_begin")
        for i in range(launches):
            self._launch(i, nontemporal)
        g = ctypes.c_void_p()
        nat.check(L.aih_capture_end(h, ctypes.byref(g)), "aih_capture_end")
        self.graph, self.launches = g.value, launches

    def _launch(self, i, nontemporal):
        b = self.src[i % len(self.src)]
        self.nat.check(self.nat.lib().aih_probe_stream_read(self.dev.handle, b.get_pointer(), self.nbytes,
                                                            int(nontemporal), self.out.get_pointer()),
                       "aih_probe_stream_read")

    def time(self, graphs, warmup=2):
        L, h = self.nat.lib(), self.dev.handle
        for _ in range(warmup):
            self.nat.check(L.aih_graph_launch(h, self.graph), "aih_graph_launch")
        self.dev.synchronize()
        self.nat.check(L.aih_event_record(h, 0), "event")
        for _ in range(graphs):
            self.nat.check(L.aih_graph_launch(h, self.graph), "aih_graph_launch")
        self.nat.check(L.aih_event_record(h, 1), "event")
        self.dev.synchronize()
        ev = ctypes.c_float()
        self.nat.check(L.aih_event_elapsed(h, 0, 1, ctypes.byref(ev)), "event")
        return ev.value / (graphs * self.launches)

    def close(self):
        self.nat.lib().aih_graph_destroy(self.graph)
        for b in self.src + [self.out]:
            b.dispose()


class GemmBench:
    """Prefill GEMM on one weight copy: a graph of `launches` aih_qgemm calls."""

    def __init__(self, dev, qtype, n, k, m, launches=20, seed_w=42, seed_x=43):
        from aihost_amd import _native as nat
        from aihost_amd import compute as C
        self.nat, self.dev = nat, dev
        self.qtype, self.n, self.k, self.m = qtype, n, k, m
        packed = C.quantize(qtype, C.fill_normal(seed_w, n * k, 0.0, 0.02), n, k)
        xh = C.fill_normal(seed_x, m * k, 0.0, 1.0)
        self.w = dev.create_buffer(packed.nbytes)
        self.w.write(packed)
        self.x = dev.create_buffer(xh.nbytes)
        self.x.write(xh)
        self.y = dev.create_buffer(m * n * 4)
        self._launch()   # sizes the library's workspace, which cannot grow during capture
        dev.synchronize()
        L, h = nat.lib(), dev.handle
        nat.check(L.aih_capture_begin(h), "aih_capture_begin")
        for _ in range(launches):
            self._launch()
        g = ctypes.c_void_p()
        nat.check(L.aih_capture_end(h, ctypes.byref(g)), "aih_capture_end")
        self.graph, self.launches = g.value, launches

    def _launch(self):
        st = self.nat.lib().aih_qgemm(self.dev.handle, self.qtype, self.w.get_pointer(), self.n, self.k,
                                      self.x.get_pointer(), self.m, self.y.get_pointer())
        self.nat.check(st, "aih_qgemm")

    def time(self, graphs, warmup=2):
        L, h = self.nat.lib(), self.dev.handle
        for _ in range(warmup):
            self.nat.check(L.aih_graph_launch(h, self.graph), "aih_graph_launch")
        self.dev.synchronize()
        self.nat.check(L.aih_event_record(h, 0), "event")
        for _ in range(graphs):
            self.nat.check(L.aih_graph_launch(h, self.graph), "aih_graph_launch")
        self.nat.check(L.aih_event_record(h, 1), "event")
        self.dev.synchronize()
        ev = ctypes.c_float()
        self.nat.check(L.aih_event_elapsed(h, 0, 1, ctypes.byref(ev)), "event")
        return ev.value / (graphs * self.launches)

    def close(self):
        self.nat.lib().aih_graph_destroy(self.graph)
        for b in (self.w, self.x, self.y):
            b.dispose()


def measured_traffic():
    """HBM bytes per launch of the headline kernel from the committed counter
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by a copy kernel of known
    size), or None when the summary is absent."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def gemm_leg(dev):
    """Prefill GEMM: Q4_K W 4096x4096, X 512x4096 (MFMA-bound; fp16 operands,
    fp32 accumulation), graph replays of 20 calls."""
    from aihost_amd import _native as nat
    gb = GemmBench(dev, nat.Q4_K, 4096, 4096, 512)
    ms = gb.time(10)
    gb.close()
    flops = 2.0 * 512 * 4096 * 4096
    return {"q4_k_gemm_4096x4096_m512": {"TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
                                         "us_per_call": round(ms * 1e3, 2),
                                         "frac_mfma_peak": round(flops / (ms * 1e-3) / MFMA_F16_PEAK, 4)}}


_VENDOR_GEMM = r"""
import json, sys, torch
out = {}
for m, n, k in json.loads(sys.argv[1]):
    a = torch.randn(m, k, device="cuda", dtype=torch.float16)
    w = torch.randn(n, k, device="cuda", dtype=torch.float16)
    for _ in range(10):
        torch.nn.functional.linear(a, w)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(50):
        torch.nn.functional.linear(a, w)
    e.record()
    torch.cuda.synchronize()
    out["%dx%d_m%d" % (n, k, m)] = s.elapsed_time(e) * 1e3 / 50
    del a, w
print(json.dumps(out))
"""


GEMM_SHAPES = ((4096, 4096), (6144, 4096), (28672, 4096), (4096, 14336))


def vendor_gemm(m=512):
    """Microseconds per call of the vendor fp16 GEMM at GEMM_SHAPES, from a
    child process; started before this process touches the GPU."""
    import subprocess
    child = subprocess.run([sys.executable, "-c", _VENDOR_GEMM, json.dumps([[m, n, k] for n, k in GEMM_SHAPES])],
                           capture_output=True, text=True, timeout=600)
    if child.returncode != 0:
        return {"vendor_error": (child.stderr.strip().splitlines() or ["exit %d" % child.returncode])[-1]}
    return json.loads(child.stdout.strip().splitlines()[-1])


def gemm_shapes_leg(dev, vendor):
    """The fused Q4_K GEMM at the Llama-8B prefill shapes (M = 512: Q|K|V
    6144x4096, W_o 4096x4096, gate|up 28672x4096, down 4096x14336) beside the
    vendor library's fp16 GEMM on fp16 weights with no dequantization
    (torch.nn.functional.linear, which calls hipBLASLt; `vendor` from
    vendor_gemm, a child process, since torch brings its own HIP runtime): a
    practical ceiling for the matrix cores at these shapes."""
    from aihost_amd import _native as nat
    m = 512
    out = {}
    for n, k in GEMM_SHAPES:
        flops = 2.0 * m * n * k
        gb = GemmBench(dev, nat.Q4_K, n, k, m)
        ms = gb.time(10)
        gb.close()
        key = "%dx%d_m%d" % (n, k, m)
        r = {"q4_k_fused_us_per_call": round(ms * 1e3, 1),
             "q4_k_fused_TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1)}
        if key in vendor:
            r["vendor_fp16_us_per_call"] = round(vendor[key], 1)
            r["vendor_fp16_TFLOP/s"] = round(flops / (vendor[key] * 1e-6) / 1e12, 1)
        out[key] = r
    if "vendor_error" in vendor:
        out["vendor_error"] = vendor["vendor_error"]
    return out


def small_batch_leg(dev, steps=600):
    """Q6_K 4096x14336 at 4 and 8 activation columns (the matrix-core kernel
    and its sum of the K splits), graphs of 60 calls: 120 kernel nodes, a size
    the kernel tracer handles."""
    from aihost_amd import _native as nat
    out = {}
    for b in (4, 8):
        mb = MatvecBench(dev, nat.Q6_K, 4096, 14336, b, launches=60)
        s, kern = mb.time(steps, 60)
        by = algorithmic_bytes(nat.Q6_K, 4096, 14336, b)
        out["q6_k_4096x14336_b%d" % b] = {"GB/s": round(by / (s * 1e-3) / 1e9, 1), "us_per_call": round(s * 1e3, 3),
                                          "launch": "hipGraph of 60 calls, replayed"}
        mb.close()
    return out


def row_bytes_total(n, k):
    from aihost_amd import _native as nat
    from aihost_amd import compute as C
    return n * C.row_bytes(nat.Q4_K, k)


def ceilings(dev, nbytes, steps):
    """Ceilings for one launch reading `nbytes` (the headline's packed bytes):
    a plain and a non-temporal 16-byte stream over 12 rotating copies, and the
    same grid launched with nothing to read (the fixed cost of a launch)."""
    out = {}
    for name, nb, ntl in (("stream_read_%dB" % nbytes, nbytes, 0),
                          ("stream_read_%dB_nontemporal" % nbytes, nbytes, 1),
                          ("empty_launch_same_grid", 0, 0)):
        sb = StreamBench(dev, nb, ntl)
        us = sb.time(max(1, steps // (3 * GRAPH_LAUNCHES))) * 1e3
        out[name] = {"us_per_launch": round(us, 3)}
        if nb:
            out[name]["GB/s"] = round(nb / (us * 1e-6) / 1e9, 1)
            out[name]["frac_hbm_peak"] = round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
        sb.close()
    return out


def cpu_baseline(packed, x, n, k, seconds, threads=1):
    """Time the oracle (the C restatement of the reference CPU path) on the same
    workload: whole passes over the 14336 x 4096 matrix, repeated until at
    least `seconds` have elapsed."""
    from oracle import oracle as orc
    orc.lib()
    reps, t0 = 0, time.perf_counter()
    while True:
        orc.matvec(orc.Q4_K, packed, n, k, x, nthreads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return reps, el


def host_threads():
    """(threads, source) for the multi-threaded CPU baseline: OMP_NUM_THREADS
    when set (the share of the host's cores this process is given), else the
    CPUs in this process's affinity mask."""
    try:
        n = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        n = 0
    if n > 0:
        return n, "OMP_NUM_THREADS"
    return max(1, len(os.sched_getaffinity(0))), "affinity mask"


def decoder_bench(dev, distinct_layers, prompt=512, gen=128, cpu=True, graph=True):
    """Full Llama decoder of the 8B shape (32 layers, hidden 4096, 32/8 heads
    of 128, FFN 14336, vocab 32000), Q4_K weights with a Q6_K head: prefill of
    a `prompt`-token random prompt, then `gen` greedy decode steps replayed
    from one captured HIP graph.  Weights are random-init; `distinct_layers`
    layer sets are generated on the host and every layer gets its own copy in
    HBM, so each decode step streams all 32 layers' weights."""
    from aihost_amd import _native as nat
    from aihost_amd import llama
    cfg = llama.LLAMA_8B_SHAPE
    L, h = nat.lib(), dev.handle
    t0 = time.perf_counter()
    w = llama.synth_weights(cfg, seed=42, distinct_layers=distinct_layers)
    t_synth = time.perf_counter() - t0
    dw = llama.DeviceWeights(dev, w)
    dec = llama.LlamaDecoder(dev, cfg, dw, max_len=prompt + gen, max_prefill=prompt)
    ids = np.random.default_rng(43).integers(0, cfg.vocab, prompt).astype(np.int32)
    try:
        first = dec.prefill(ids)          # warm-up (GEMM workspace, code paths)
        dec.decode(4, use_graph=graph)    # captures the decode graph
        dev.synchronize()
        nat.check(L.aih_event_record(h, 2), "event")
        dec.prefill(ids, read=False)
        nat.check(L.aih_event_record(h, 3), "event")
        dec.decode(gen, use_graph=graph)
        nat.check(L.aih_event_record(h, 4), "event")
        dev.synchronize()
        ms = ctypes.c_float()
        nat.check(L.aih_event_elapsed(h, 2, 3, ctypes.byref(ms)), "event")
        t_pre = ms.value * 1e-3
        nat.check(L.aih_event_elapsed(h, 3, 4, ctypes.byref(ms)), "event")
        t_dec = ms.value * 1e-3
        toks = dec.tokens(gen + 1)
    finally:
        dec.dispose()
    wbytes = dw.nbytes() - w["token_embd"][1].nbytes + cfg.dim * 4 * 2   # one embedding row read per token
    dw.dispose()
    # KV cache reads per decode step (fp32 K and V rows 0..p of every layer), averaged over the steps
    avg_keys = prompt + (gen + 1) / 2.0
    kv_bytes = 2 * cfg.n_layers * avg_keys * cfg.kv_dim * 4
    per_tok = t_dec / gen
    flops_pre = 2.0 * prompt * sum(r * c for n_, (qt, a, r, c) in w.items()
                                   if n_.startswith("blk.") and qt != llama.F32)
    out = {
        "model": "Llama 8B shape, random init: 32 layers, hidden 4096, 32/8 heads x 128, FFN 14336, vocab 32000; "
                 "Q4_K weights, Q6_K head (%d distinct layer sets, one HBM copy per layer)" % distinct_layers,
        "prefill_tokens": prompt, "prefill_ms": round(t_pre * 1e3, 2),
        "prefill_tokens_per_s": round(prompt / t_pre, 1),
        "prefill_layer_matmul_TFLOP/s": round(flops_pre / t_pre / 1e12, 1),
        "decode_tokens": gen, "decode_steps": "graph replays" if graph else "eager launches",
        "decode_ms_per_token": round(per_tok * 1e3, 4),
        "decode_tokens_per_s": round(gen / t_dec, 1),
        "decode_GB/s": round((wbytes + kv_bytes) / per_tok / 1e9, 1),
        "decode_frac_hbm_peak": round((wbytes + kv_bytes) / per_tok / 1e9 / HBM_PEAK_GBS, 4),
        "decode_bytes_per_token": int(wbytes + kv_bytes),
        "first_tokens": [int(t) for t in toks[:8]], "first_token_check": int(first) == int(toks[0]),
        "host_weight_synthesis_s": round(t_synth, 1),
    }
    if cpu:
        # the oracle's single-thread matvec (the reference's scalar CPU path) on
        # one layer's seven matrices and the head, extrapolated to 32 layers
        from oracle import oracle as orc
        orc.lib()
        t_layer = 0.0
        x = np.random.default_rng(1).standard_normal((1, cfg.ffn)).astype(np.float32)
        for suf, qt, r, c in llama.layer_tensors(cfg):
            if qt == llama.F32:
                continue
            t1 = time.perf_counter()
            orc.matvec(qt, w["blk.0." + suf][1], r, c, x[:, :c], nthreads=1)
            t_layer += time.perf_counter() - t1
        qt, a, r, c = w["output"]
        t1 = time.perf_counter()
        orc.matvec(qt, a, r, c, x[:, :c], nthreads=1)
        t_head = time.perf_counter() - t1
        t_tok = cfg.n_layers * t_layer + t_head
        out["cpu_baseline_decode"] = {
            "value": round(1.0 / t_tok, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": "one layer's 7 Q4_K matvecs (%.2f s) and the Q6_K head (%.2f s) through the oracle's "
                      "single-thread row dequant + fp32 dot, extrapolated to 32 layers; attention and norms "
                      "not counted" % (t_layer, t_head)}
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3000)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary workloads")
    ap.add_argument("--no-decoder", action="store_true", help="skip the full-decoder prefill/decode leg")
    ap.add_argument("--decoder-distinct-layers", type=int, default=2)
    ap.add_argument("--only", choices=("ceilings", "gemm", "gemm-shapes", "decoder-eager", "small-batch"),
                    help="one leg alone, for profiling (one JSON line): the stream-read ceilings and the launch "
                         "floor; the prefill GEMM; the GEMM at the prefill shapes beside the vendor fp16 GEMM; "
                         "the decoder with eager decode steps (no graph); the Q6_K 4096x14336 matvec at 4 and "
                         "8 columns")
    ap.add_argument("--no-vendor", action="store_true",
                    help="with --only gemm-shapes: skip the vendor GEMM's child process (for profiler runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    from aihost_amd import _native as nat
    from aihost_amd import compute as C

    if args.steps < 1:
        print("--steps must be at least 1", file=sys.stderr)
        sys.exit(2)
    vendor = vendor_gemm() if args.only == "gemm-shapes" and not args.no_vendor else {}
    dev = C.HipComputeDevice(0)
    n, k = 14336, 4096
    if args.only == "ceilings":
        print(json.dumps(ceilings(dev, row_bytes_total(n, k), args.steps)))
        dev.dispose()
        return
    if args.only == "gemm":
        print(json.dumps(gemm_leg(dev)))
        dev.dispose()
        return
    if args.only == "gemm-shapes":
        print(json.dumps(gemm_shapes_leg(dev, vendor)))
        dev.dispose()
        return
    if args.only == "small-batch":
        print(json.dumps(small_batch_leg(dev)))
        dev.dispose()
        return
    if args.only == "decoder-eager":
        print(json.dumps(decoder_bench(dev, args.decoder_distinct_layers, gen=32, cpu=False, graph=False)))
        dev.dispose()
        return
    g_main = graph_size(args.steps)
    main_b = MatvecBench(dev, nat.Q4_K, n, k, 1, launches=g_main)
    # Untimed copy of one weight copy: a kernel of known traffic, so that a
    # counter run (FETCH_SIZE / WRITE_SIZE) over this script can be scaled by
    # what the counters read for it.
    probe = dev.create_buffer(main_b.packed.nbytes)
    nat.check(nat.lib().aih_memcpy_d2d(dev.handle, probe.get_pointer(), main_b.w[0].get_pointer(),
                                       main_b.packed.nbytes), "aih_memcpy_d2d")
    dev.synchronize()
    probe.dispose()
    ms_step, ms_kernel = main_b.time(args.steps, args.warmup)
    nbytes = algorithmic_bytes(nat.Q4_K, n, k, 1)
    gbs = nbytes / (ms_step * 1e-3) / 1e9
    achieved = nbytes / (ms_kernel * 1e-3) / 1e9
    y_check = main_b.output()
    packed, x_host = main_b.packed, main_b.x_host
    main_b.close()

    extra = {}
    if not args.no_extra:
        for name, qt, nn, kk, b in (("q4_0_14336x4096_b1", nat.Q4_0, 14336, 4096, 1),
                                    ("q8_0_4096x4096_b1", nat.Q8_0, 4096, 4096, 1),
                                    ("q6_k_4096x14336_b1", nat.Q6_K, 4096, 14336, 1),
                                    ("q6_k_4096x14336_b2", nat.Q6_K, 4096, 14336, 2),
                                    ("q6_k_4096x14336_b4", nat.Q6_K, 4096, 14336, 4),
                                    ("q6_k_4096x14336_b8", nat.Q6_K, 4096, 14336, 8),
                                    ("q4_k_4096x14336_b1", nat.Q4_K, 4096, 14336, 1)):
            mb = MatvecBench(dev, qt, nn, kk, b)
            s, kern = mb.time(GRAPH_LAUNCHES * max(1, args.steps // (3 * GRAPH_LAUNCHES)), args.warmup // 3)
            by = algorithmic_bytes(qt, nn, kk, b)
            extra[name] = {"GB/s": round(by / (s * 1e-3) / 1e9, 1),
                           "us_per_call": round(s * 1e3, 3),
                           "frac_hbm_peak": round(by / (kern * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            mb.close()
        extra.update(ceilings(dev, packed.nbytes, args.steps))
        # weight upload (host -> HBM through the pinned staging ring), a load-time
        # rate that crosses PCIe: reported beside the kernels, never as `value`
        ub = dev.create_buffer(packed.nbytes)
        src = np.ascontiguousarray(packed)
        nat.check(nat.lib().aih_upload_tensor(dev.handle, ub.get_pointer(), src.ctypes.data, src.nbytes), "upload")
        dev.synchronize()
        t0 = time.perf_counter()
        for _ in range(5):
            nat.check(nat.lib().aih_upload_tensor(dev.handle, ub.get_pointer(), src.ctypes.data, src.nbytes),
                      "upload")
        dev.synchronize()
        el = time.perf_counter() - t0
        extra["upload_q4_k_14336x4096"] = {"GB/s": round(5 * src.nbytes / el / 1e9, 2),
                                           "ms_per_call": round(el / 5 * 1e3, 3)}
        ub.dispose()
        extra.update(gemm_leg(dev))

    decode = None
    if not args.no_decoder:
        decode = decoder_bench(dev, args.decoder_distinct_layers, cpu=not args.no_cpu_baseline)

    cpu = cpu_mt = None
    if not args.no_cpu_baseline:
        reps, el = cpu_baseline(packed, x_host.reshape(1, k), n, k, args.cpu_seconds, threads=1)
        cpu = {"value": round(nbytes * reps / el / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": "%d full passes of the 14336x4096 Q4_K batch-1 matvec (row dequant + sequential fp32 dot, "
                         "oracle/oracle.c -O2 -ffp-contract=off) in %.1f s, one thread" % (reps, el)}
        # the same port with its rows split over the host cores (OpenMP, static schedule)
        nt, src = host_threads()
        reps, el = cpu_baseline(packed, x_host.reshape(1, k), n, k, args.cpu_seconds / 2, threads=nt)
        cpu_mt = {"value": round(nbytes * reps / el / 1e9, 3), "unit": "GB/s", "cores": nt, "kind": "port",
                  "host_nproc": os.cpu_count(), "threads_from": src,
                  "sample": "%d full passes of the same matvec in %.1f s, rows split over %d OpenMP threads "
                            "(the %s; the host has %d CPUs)" % (reps, el, nt, src, os.cpu_count())}
    dev.dispose()

    # the matvec's per-launch time over the faster of the two plain streams of
    # its bytes measured in this run (1.0 = as fast as the best stream)
    streams = [v["us_per_launch"] for key, v in extra.items() if key.startswith("stream_read_")]
    vs_stream = round(ms_kernel * 1e3 / min(streams), 4) if streams else None

    out = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i32+f32",
        "data": "synthetic: W ~ N(0,0.02) seed 42 quantized to Q4_K by the library's GGUF quantizer; x ~ N(0,1) seed 43",
        "config": {"workload": "Q4_K decode matvec, W 14336x4096 (GGUF dims [4096,14336]), batch 1",
                   "N": n, "K": k, "batch": 1, "weight_copies": COPIES,
                   "launch": "hipGraph of %d launches over the copies, replayed %d times (steps = %d)"
                             % (g_main, args.steps // g_main, args.steps),
                   "arithmetic": "weight codes x three int8 limbs of fixed-point x, v_dot4_i32_i8 (exact int32); "
                                 "scales, mins and limb weights in fp32",
                   "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "traffic_source": "committed counter summary %s (FETCH_SIZE + WRITE_SIZE per launch, scaled "
                                       "by a copy of known size), not this run" % os.path.relpath(TRAFFIC_PROFILE, ROOT),
                     "kernel_us": round(ms_kernel * 1e3, 3),
                     "timing": "kernel_us: HIP events around the timed graph replays on the library's stream, per "
                               "launch: back-to-back kernels, each with its launch's fixed cost, plus the start-up "
                               "of each replay (one replay at --steps <= 120: about 0.3 us per launch at 20)",
                     "bytes_per_launch": nbytes,
                     "vs_best_stream": vs_stream},
        "cpu_baseline": cpu,
        "cpu_baseline_threads": cpu_mt,
        "decode": decode,
        "also": extra,
        "y_checksum": float(np.sum(y_check.astype(np.float64))),
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
