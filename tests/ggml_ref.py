"""Independent numpy statement of the GGUF/ggml block formats (test helper).

Written from ggml's published loop structure (dequantize_row_q4_K / _q6_K /
_q8_0 / _q4_0 in ggml-quants.c, the format AIHost reads), NOT from AIHost's
per-element index arithmetic, so that agreement with the oracle pins the
element order of both.  fp16 fields are decoded with numpy's IEEE float16.
The arithmetic order matches ggml (d1 = d*sc; y = d1*q - m1), which is also
the reference's order, so results are compared bit for bit.
"""
import numpy as np

F32, Q4_0, Q8_0, Q4_K, Q6_K = 0, 2, 8, 12, 14
QK = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}
BB = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210}


def f16(b, off):
    return np.frombuffer(bytes(b[off:off + 2]), dtype=np.float16)[0].astype(np.float32)


def scale_min_k4(j, q):
    """ggml get_scale_min_k4."""
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def deq_q4_k(b):
    b = np.asarray(b, dtype=np.uint8)
    d, dmin = f16(b, 0), f16(b, 2)
    scales, q = b[4:16], b[16:144]
    y = np.empty(256, dtype=np.float32)
    pos, is_ = 0, 0
    for j in range(0, 256, 64):
        sc, m = scale_min_k4(is_, scales)
        d1, m1 = d * np.float32(sc), dmin * np.float32(m)
        sc, m = scale_min_k4(is_ + 1, scales)
        d2, m2 = d * np.float32(sc), dmin * np.float32(m)
        for l in range(32):
            y[pos] = d1 * np.float32(q[l] & 0xF) - m1
            pos += 1
        for l in range(32):
            y[pos] = d2 * np.float32(q[l] >> 4) - m2
            pos += 1
        q = q[32:]
        is_ += 2
    return y


def deq_q6_k(b):
    b = np.asarray(b, dtype=np.uint8)
    ql, qh, sc = b[0:128], b[128:192], b[192:208].view(np.int8)
    d = f16(b, 208)
    y = np.empty(256, dtype=np.float32)
    base = 0
    for n in range(0, 256, 128):
        for l in range(32):
            is_ = l // 16
            q1 = int((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32
            q2 = int((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32
            q3 = int((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32
            q4 = int((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32
            y[base + l + 0] = d * np.float32(sc[is_ + 0]) * np.float32(q1)
            y[base + l + 32] = d * np.float32(sc[is_ + 2]) * np.float32(q2)
            y[base + l + 64] = d * np.float32(sc[is_ + 4]) * np.float32(q3)
            y[base + l + 96] = d * np.float32(sc[is_ + 6]) * np.float32(q4)
        base += 128
        ql, qh, sc = ql[64:], qh[32:], sc[8:]
    return y


def deq_q8_0(b):
    b = np.asarray(b, dtype=np.uint8)
    d = f16(b, 0)
    return b[2:34].view(np.int8).astype(np.float32) * d


def deq_q4_0(b):
    b = np.asarray(b, dtype=np.uint8)
    d = f16(b, 0)
    qs = b[2:18]
    # ggml: x0 = (qs[j] & 0xF) - 8 -> y[j], x1 = (qs[j] >> 4) - 8 -> y[j+16]; y = x*d
    return (np.concatenate([(qs & 0xF).astype(np.int32) - 8, (qs >> 4).astype(np.int32) - 8])
            .astype(np.float32) * d)


DEQ = {Q4_K: deq_q4_k, Q6_K: deq_q6_k, Q8_0: deq_q8_0, Q4_0: deq_q4_0}


def dequantize(qtype, data):
    data = np.asarray(data, dtype=np.uint8)
    nb = data.size // BB[qtype]
    return np.concatenate([DEQ[qtype](data[i * BB[qtype]:(i + 1) * BB[qtype]]) for i in range(nb)])


def pack_scales_k4(sc, mn):
    """Pack 8 six-bit scales and 8 six-bit mins into 12 bytes, per the
    K-quant layout: bytes 0-3 low 6 bits = sc[0..3], top 2 bits = sc[4..7]>>4;
    bytes 4-7 low 6 bits = mn[0..3], top 2 bits = mn[4..7]>>4; bytes 8-11 low
    nibble = sc[4..7]&15, high nibble = mn[4..7]&15."""
    out = np.zeros(12, dtype=np.uint8)
    for j in range(4):
        out[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        out[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        out[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return out
