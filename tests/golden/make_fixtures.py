"""Write the seeded golden fixtures of the dequant and matvec path.

The reference holds no golden vectors for this path, so the expected outputs
come from the oracle (whose functions are pinned by the exhaustive, single-bit
and closed-form checks under tests/).  The fixtures freeze those outputs so
that a later change to the oracle or the kernels shows up as a diff.

    python tests/golden/make_fixtures.py      # rewrites tests/golden/fixtures.npz
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as orc  # noqa: E402

TYPES = {"q8_0": orc.Q8_0, "q4_0": orc.Q4_0, "q4_k": orc.Q4_K, "q6_k": orc.Q6_K}
SCALE_OFFSETS = {orc.Q8_0: (0,), orc.Q4_0: (0,), orc.Q4_K: (0, 2), orc.Q6_K: (208,)}


def blocks(qtype, nblocks, seed):
    """Random block bytes with finite fp16 scales: half normal (2^-14..2^-2),
    half subnormal, so both fp16 decoders are exercised."""
    rng = np.random.default_rng(seed)
    bb = orc.BLOCK_BYTES[qtype]
    data = rng.integers(0, 256, (nblocks, bb), dtype=np.uint8)
    for off in SCALE_OFFSETS[qtype]:
        h = np.where(np.arange(nblocks) % 2 == 0,
                     rng.integers(0x0400, 0x3400, nblocks), rng.integers(0x0001, 0x0400, nblocks))
        h = h.astype(np.uint16) | np.where(rng.integers(0, 2, nblocks) == 1, 0x8000, 0).astype(np.uint16)
        data[:, off:off + 2] = h.view(np.uint8).reshape(nblocks, 2)
    return data.reshape(-1)


def main():
    out = {}
    for name, qt in TYPES.items():
        nb = 8 if orc.BLOCK_ELEMS[qt] == 256 else 32
        data = blocks(qt, nb, seed=1000 + qt)
        n = nb * orc.BLOCK_ELEMS[qt]
        out[name + "_blocks"] = data
        out[name + "_ieee"] = orc.dequantize(qt, data, n, orc.F16_IEEE)
        out[name + "_refcpu"] = orc.dequantize(qt, data, n, orc.F16_REFCPU)
        # matvec: 8 rows of K = n/8, two activation columns
        k = n // 8
        x = np.random.default_rng(2000 + qt).standard_normal((2, k)).astype(np.float32)
        out[name + "_x"] = x
        out[name + "_y"] = orc.matvec(qt, data, 8, k, x)
    np.savez_compressed(os.path.join(HERE, "fixtures.npz"), **out)
    print("wrote", os.path.join(HERE, "fixtures.npz"), sum(v.nbytes for v in out.values()), "bytes raw")


if __name__ == "__main__":
    main()
