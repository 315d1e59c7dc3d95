"""Error paths that need a device, each forced from the host (no kernel is made to fail).

* an output too large for the device raises OutOfMemoryError after the cache has been returned and
  the allocation retried, and the library keeps working afterwards;
* a device index past the device count, the host device or a malformed device string raises
  DeviceError.
"""
import gc

import numpy as np
import pytest

import musapy_amd as ms
from tests.conftest import assert_bits_equal

pytestmark = pytest.mark.gpu


def test_out_of_memory_is_reported_and_recoverable():
    a = ms.from_numpy(np.ones((100_000, 1), np.float32))
    b = ms.from_numpy(np.ones((1, 1_000_000), np.float32))  # the (100000, 1000000) f32 result is 400 GB
    ms.synchronize()
    live = ms.mem_stats()["live_bytes"]
    with pytest.raises(ms.OutOfMemoryError):
        ms.add(a, b)
    gc.collect()
    ms.synchronize()
    assert ms.mem_stats()["live_bytes"] == live
    x = np.arange(4096, dtype=np.float32)
    assert_bits_equal(ms.add(ms.from_numpy(x), ms.from_numpy(x)).numpy(), x + x, "add after the failed allocation")
    assert ms.sum(a).item() == 100_000.0


def test_invalid_devices():
    x = np.ones(8, np.float32)
    with pytest.raises(ms.DeviceError):
        ms.from_numpy(x, device=f"hip:{ms.device_count()}")
    with pytest.raises(ms.DeviceError):
        ms.from_numpy(x, device="cpu")
    with pytest.raises(ms.DeviceError):
        ms.from_numpy(x, device="cuda:zero")
    assert ms.from_numpy(x, device="musa:0").device == "hip:0"
    assert ms.sum(ms.from_numpy(x, device="hip:0")).item() == 8.0
