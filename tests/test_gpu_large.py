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
