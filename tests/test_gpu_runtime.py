"""Device/buffer/queue behaviour of the HIP device (the drop-in boundary)."""
import ctypes

import numpy as np
import pytest

from aihost_amd import _native as nat
from aihost_amd import compute as C

pytestmark = pytest.mark.gpu


def test_device_info(device):
    i = device.info()
    assert i.arch.decode().startswith("gfx950")
    assert i.compute_units >= 200 and i.wavefront_size == 64
    assert i.total_bytes > 200 * 2**30
    m = device.get_memory_info()
    assert m.total_bytes == i.total_bytes and m.available_bytes <= m.total_bytes


def test_alloc_free_and_double_free(device):
    L = nat.lib()
    before = device.info()
    p = ctypes.c_void_p()
    assert L.aih_malloc(device.handle, 1 << 20, ctypes.byref(p)) == nat.AIH_OK
    mid = device.info()
    assert mid.tracked_bytes == before.tracked_bytes + (1 << 20)
    assert mid.tracked_buffers == before.tracked_buffers + 1
    assert L.aih_free(device.handle, p) == nat.AIH_OK
    assert L.aih_free(device.handle, p) == nat.AIH_E_NOT_ALLOCATED
    assert device.info().tracked_bytes == before.tracked_bytes
    assert L.aih_malloc(device.handle, 0, ctypes.byref(p)) == nat.AIH_E_INVALID


def test_out_of_memory_maps_to_insufficient_vram(device):
    with pytest.raises(C.InsufficientVramException):
        device.create_buffer(1 << 52)
    # the device stays usable afterwards
    b = device.create_buffer(4096)
    b.write(np.arange(1024, dtype=np.float32))
    assert np.array_equal(b.read(), np.arange(1024, dtype=np.float32))
    b.dispose()


def test_staged_round_trip_large(device):
    rng = np.random.default_rng(0)
    data = rng.integers(0, 256, 40 * 2**20 + 123).astype(np.uint8)   # spans several staging slots
    b = device.create_buffer(data.nbytes)
    b.write(data)
    assert np.array_equal(b.read(np.uint8), data)
    assert np.array_equal(b.read_range(7 * 2**20 + 5, 1000, np.uint8), data[7 * 2**20 + 5:7 * 2**20 + 1005])
    c = device.create_buffer(data.nbytes)
    assert nat.lib().aih_memcpy_d2d(device.handle, c.get_pointer(), b.get_pointer(), data.nbytes) == 0
    assert nat.lib().aih_memset(device.handle, b.get_pointer(), 0, 4096) == 0
    assert np.array_equal(c.read(np.uint8), data)
    assert not b.read_range(0, 4096, np.uint8).any()
    b.dispose()
    c.dispose()


def test_upload_tensor_verbatim(device):
    packed = np.random.default_rng(1).integers(0, 256, 9 * 2304).astype(np.uint8)
    t = C.Tensor.from_quantized(device, packed, 4096, 9, C.DataType.Q4_K)
    assert t.shape == (4096, 9)
    assert np.array_equal(t.buffer.read(np.uint8), packed)
    with pytest.raises(ValueError):
        C.Tensor.from_quantized(device, packed[:-1], 4096, 9, C.DataType.Q4_K)
    t.dispose()


def test_large_upload_verbatim(device):
    """A transfer of several staging slots, each filled by the host copy
    threads (slot fills of 2 MiB or more are split over them), arrives byte
    for byte; so does a second one of another length through the same pool."""
    rng = np.random.default_rng(7)
    for n in ((40 << 20) + 12345, (3 << 20) + 7):
        data = rng.integers(0, 256, n, dtype=np.uint8)
        b = device.create_buffer(n)
        assert nat.lib().aih_upload_tensor(device.handle, b.get_pointer(), data.ctypes.data, n) == 0
        assert np.array_equal(b.read(np.uint8), data)
        b.dispose()


def test_events_time_the_stream(device):
    L = nat.lib()
    b = device.create_buffer(64 << 20)
    assert L.aih_event_record(device.handle, 0) == 0
    for _ in range(4):
        assert L.aih_memset(device.handle, b.get_pointer(), 1, 64 << 20) == 0
    assert L.aih_event_record(device.handle, 1) == 0
    ms = ctypes.c_float()
    assert L.aih_event_elapsed(device.handle, 0, 1, ctypes.byref(ms)) == 0
    assert ms.value > 0.0
    assert L.aih_event_record(device.handle, 16) == nat.AIH_E_INVALID
    assert L.aih_stream(device.handle) is not None
    b.dispose()


def test_second_context_is_independent(device):
    d2 = C.HipComputeDevice(0)
    b = d2.create_buffer(1024)
    p = b.get_pointer()
    # a pointer owned by one context is not freeable through another
    assert nat.lib().aih_free(device.handle, p) == nat.AIH_E_NOT_ALLOCATED
    d2.dispose()   # frees b as well


def test_probe_stream_read_folds_every_byte(device):
    """The bandwidth probe reads every 16-byte piece once: the XOR of the
    per-wave words equals the XOR of the whole buffer's 32-bit words."""
    from aihost_amd import _native as nat
    L = nat.lib()
    data = np.random.default_rng(5).integers(0, 2**32, (1 << 20) // 4, dtype=np.uint32)
    src = device.create_buffer(data.nbytes)
    out = device.create_buffer(8192 * 4)
    try:
        src.write(data)
        for nt in (0, 1):
            nat.check(L.aih_memset(device.handle, out.get_pointer(), 0, 8192 * 4), "memset")
            nat.check(L.aih_probe_stream_read(device.handle, src.get_pointer(), data.nbytes, nt, out.get_pointer()),
                      "probe")
            device.synchronize()
            words = out.read_range(0, 8192, np.uint32)
            assert np.bitwise_xor.reduce(words) == np.bitwise_xor.reduce(data)
        nat.check(L.aih_probe_stream_read(device.handle, None, 0, 0, out.get_pointer()), "empty launch")
        assert L.aih_probe_stream_read(device.handle, src.get_pointer(), 17, 0, out.get_pointer()) == nat.AIH_E_INVALID
        assert L.aih_probe_stream_read(device.handle, src.get_pointer(), 16, 0, None) == nat.AIH_E_INVALID
    finally:
        src.dispose()
        out.dispose()
