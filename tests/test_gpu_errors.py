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


def test_rank_limit():
    """32 dimensions is the kernels' limit (the reference's MUSAPY_MAX_NDIM): a 33-dimensional array
    is refused when it is created; a 32-dimensional one works."""
    with pytest.raises(ms.ShapeError):
        ms.from_numpy(np.ones((1,) * 33, np.float32))
    x = np.arange(6, dtype=np.float32).reshape((1,) * 30 + (2, 3))
    X = ms.from_numpy(x)
    assert_bits_equal(ms.add(X, X).numpy(), x + x, "32-d add")
    assert ms.sum(X).item() == 15.0
    assert ms.sum(X, axis=31).numpy().reshape(-1).tolist() == [3.0, 12.0]


def test_c_abi_rejects_bad_rank_and_axis():
    """A C-ABI wrapper given ndim outside [0, 32] or an axis outside [0, ndim) launches nothing and
    reports wrapper error 3 (also as -3 through mpy_rt_check_launch)."""
    import ctypes
    import os

    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "musapy_amd",
                                   "libmusapy_hip.so"))
    lib.musapy_kernels_take_error.restype = ctypes.c_int
    lib.mpy_rt_check_launch.restype = ctypes.c_int
    P, I, SZ, SS = ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_ssize_t)
    lib.musapy_add_f32_v2.argtypes = [P, P, P, I, SZ, SS, SS, P]
    lib.musapy_sum_f32_v2.argtypes = [P, P, I, SZ, SS, I, ctypes.c_size_t, ctypes.c_size_t, P]
    lib.musapy_cumsum_f32_v3.argtypes = [P, P, P, I, SZ, SS, I, ctypes.c_size_t, ctypes.c_size_t, P]
    x = np.arange(8, dtype=np.float32)
    X = ms.from_numpy(x)
    Y = ms.from_numpy(np.full(8, -1.0, np.float32))
    ms.synchronize()
    lib.musapy_kernels_take_error()  # start clean
    shape = (ctypes.c_size_t * 40)(*([1] * 39 + [8]))
    st = (ctypes.c_ssize_t * 40)(*([0] * 39 + [1]))
    lib.musapy_add_f32_v2(X.data_ptr, X.data_ptr, Y.data_ptr, 40, shape, st, st, X.stream_ptr)
    assert lib.musapy_kernels_take_error() == 3
    one = (ctypes.c_size_t * 1)(8)
    s1 = (ctypes.c_ssize_t * 1)(1)
    lib.musapy_sum_f32_v2(X.data_ptr, Y.data_ptr, 1, one, s1, 1, 8, 1, X.stream_ptr)  # axis 1 of a 1-d array
    assert lib.mpy_rt_check_launch() == -3
    lib.musapy_cumsum_f32_v3(X.data_ptr, Y.data_ptr, None, 1, one, s1, -1, 8, 1, X.stream_ptr)
    assert lib.musapy_kernels_take_error() == 3
    ms.synchronize()
    assert Y.numpy().tolist() == [-1.0] * 8  # nothing was written
    lib.musapy_add_f32_v2(X.data_ptr, X.data_ptr, Y.data_ptr, 1, one, s1, s1, X.stream_ptr)
    assert lib.mpy_rt_check_launch() == 0
    ms.synchronize()
    assert_bits_equal(Y.numpy(), x + x, "valid call after the refused ones")
