"""Arrays past the 32-bit element limits, on the GPU (they need about 30 GB of device memory).

Row counts and row lengths of 2^31 or more send the elementwise planner to its 64-bit kernels, and
whole-array reductions carry 64-bit element indices; planted values past 2^31 / 2^32 check both.
The data is mostly zeros with a few planted values, so every expected result is exact.
"""
import gc

import numpy as np
import pytest

import musapy_amd as ms

pytestmark = pytest.mark.gpu


def test_reductions_past_2_31_elements():
    n = (1 << 31) + 7
    x = np.zeros(n, np.float32)
    x[123] = 4.0
    x[(1 << 31) + 1] = 5.0
    x[n - 3] = 5.0  # a tie: the lower index wins
    X = ms.from_numpy(x)
    del x
    assert ms.argmax(X).item() == (1 << 31) + 1
    assert ms.max(X).item() == 5.0
    assert ms.sum(X).item() == 14.0
    assert ms.argmin(X).item() == 0
    Y = ms.add(X, X)  # 1-D contiguous: the flat kernel over 2^31 + 7 elements
    assert ms.sum(Y).item() == 28.0
    assert ms.argmax(Y).item() == (1 << 31) + 1
    del X, Y
    gc.collect()
    ms.synchronize()
    ms.empty_cache()


def test_reversed_copy_past_2_32_elements():
    n = (1 << 32) + 1000
    x = np.zeros(n, np.uint8)
    x[n - 1] = 7
    x[(1 << 32) + 3] = 9
    x[5] = 11
    X = ms.from_numpy(x)
    del x
    Y = ms.contiguous(ms.flip(X, 0))  # one row of 2^32 + 1000 reversed bytes: the 64-bit path
    y = Y.numpy()
    assert y[0] == 7 and y[n - 1 - ((1 << 32) + 3)] == 9 and y[n - 1 - 5] == 11
    assert int(np.count_nonzero(y)) == 3
    del X, Y, y
    gc.collect()
    ms.synchronize()
    ms.empty_cache()


def test_zero_ties_past_2_31_elements():
    """The whole-array reduction's packed 64-bit wave keys (value, ~index) hold indices below
    2^32 - 1: a zero tie past 2^31 must still go to the lower index and keep that zero's sign."""
    n = (1 << 31) + (1 << 20)
    x = np.full(n, -1.0, np.float32)
    lo, hi = (1 << 31) + 123, (1 << 31) + 456
    x[lo], x[hi] = -0.0, 0.0
    X = ms.from_numpy(x)
    del x
    assert ms.argmax(X).item() == lo
    assert np.signbit(ms.max(X).numpy())  # the first zero is -0
    del X
    gc.collect()
    y = np.full(n, 1.0, np.float32)
    y[lo], y[hi] = 0.0, -0.0
    Y = ms.from_numpy(y)
    del y
    assert ms.argmin(Y).item() == lo
    assert not np.signbit(ms.min(Y).numpy())  # the first zero is +0
    del Y
    gc.collect()
    ms.synchronize()
    ms.empty_cache()
