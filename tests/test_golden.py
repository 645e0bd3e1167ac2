"""Seeded golden fixtures (tests/golden/fixtures.npz, written by
tests/golden/make_fixtures.py): random blocks with normal and subnormal fp16
scales of every format, their dequantization in both fp16 modes, and an
8-row two-column matvec.  The CPU tests hold the oracle to the fixtures; the
GPU tests hold the HIP library to them (dequant bit-exact, matvec 1e-3)."""
import os

import numpy as np
import pytest

from aihost_amd import _native as nat

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.npz")
TYPES = {"q8_0": nat.Q8_0, "q4_0": nat.Q4_0, "q4_k": nat.Q4_K, "q6_k": nat.Q6_K}
TOL = 1e-3


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("name", sorted(TYPES))
def test_oracle_matches_fixtures(orc, fx, name):
    qt = TYPES[name]
    data = fx[name + "_blocks"]
    n = fx[name + "_ieee"].size
    for mode, key in ((orc.F16_IEEE, "_ieee"), (orc.F16_REFCPU, "_refcpu")):
        got = orc.dequantize(qt, data, n, mode)
        assert np.array_equal(got.view(np.uint32), fx[name + key].view(np.uint32)), (name, key)
    x = fx[name + "_x"]
    assert np.array_equal(orc.matvec(qt, data, 8, n // 8, x), fx[name + "_y"])


def test_fixtures_exercise_both_fp16_decoders(fx):
    # the two decoders differ only on subnormal scales; the fixtures hold some
    for name in TYPES:
        assert not np.array_equal(fx[name + "_ieee"], fx[name + "_refcpu"]), name


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(TYPES))
def test_gpu_matches_fixtures(device, fx, name):
    from gpu_util import assert_close, dequant, qmatvec
    qt = TYPES[name]
    data = fx[name + "_blocks"]
    n = fx[name + "_ieee"].size
    for mode, key in ((nat.F16_IEEE, "_ieee"), (nat.F16_REFCPU, "_refcpu")):
        got = dequant(device, qt, data, n, mode)
        assert np.array_equal(got.view(np.uint32), fx[name + key].view(np.uint32)), (name, key)
    y = qmatvec(device, qt, data, 8, n // 8, fx[name + "_x"])
    assert_close(y, fx[name + "_y"], TOL, name)
