"""pytest configuration: the `gpu` marker and shared helpers.

`-m "not gpu"` runs on any host (oracle pinning, host-side logic, C-ABI exports).
`-m gpu` needs an MI355X; those tests call the HIP path and compare with the CPU oracle.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); compares the GPU path with the oracle")


def ulp_diff_f32(a, b):
    """Distance in units in the last place between float32 arrays (NaN == NaN counts as 0)."""
    a = np.ascontiguousarray(a, dtype=np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, dtype=np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def ulp_diff_f64(a, b):
    """Same for float64; exact integer arithmetic only where the bits differ."""
    a = np.ascontiguousarray(a, dtype=np.float64).view(np.int64).ravel()
    b = np.ascontiguousarray(b, dtype=np.float64).view(np.int64).ravel()
    out = np.zeros(a.shape, dtype=np.float64)
    for i in np.nonzero(a != b)[0]:
        x, y = int(a[i]), int(b[i])
        x = -(x & 0x7FFFFFFFFFFFFFFF) if x < 0 else x
        y = -(y & 0x7FFFFFFFFFFFFFFF) if y < 0 else y
        out[i] = float(abs(x - y))
    return out


def assert_bits_equal(got, want, what="", nan_bits=False):
    """Bit-exact comparison.  A NaN produced by an invalid operation (inf - inf, 0 * inf, ...)
    has a platform-defined sign and payload -- x86 SSE returns the negative "default NaN",
    CDNA the positive canonical quiet NaN -- so unless `nan_bits` is set, a NaN component
    matches any NaN component; every other value must agree in every bit."""
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert got.dtype == want.dtype, (what, got.dtype, want.dtype)
    if not nan_bits and (np.issubdtype(got.dtype, np.floating) or np.issubdtype(got.dtype, np.complexfloating)):
        comp = np.float32 if got.dtype in (np.float32, np.complex64) else (
            np.float64 if got.dtype in (np.float64, np.complex128) else got.dtype)
        gc = np.ascontiguousarray(got).reshape(-1).view(comp)
        wc = np.ascontiguousarray(want).reshape(-1).view(comp)
        both_nan = np.isnan(gc) & np.isnan(wc)
        if both_nan.any():
            gc, wc = gc.copy(), wc.copy()
            gc[both_nan] = 0
            wc[both_nan] = 0
            got = gc.view(got.dtype).reshape(got.shape)
            want = wc.view(want.dtype).reshape(want.shape)
    size = got.dtype.itemsize
    word = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64, 16: np.uint64}[size]
    per = 2 if size == 16 else 1
    g = np.ascontiguousarray(got).reshape(-1).view(word).reshape(-1, per)
    w = np.ascontiguousarray(want).reshape(-1).view(word).reshape(-1, per)
    diff = np.any(g != w, axis=1)
    if diff.any():
        bad = np.nonzero(diff)[0]
        i = bad[0]
        fg, fw = got.reshape(-1), want.reshape(-1)
        raise AssertionError(f"{what}: {len(bad)} of {fg.size} elements differ in bits; first at {i}: "
                             f"got {fg[i]!r} ({g[i]}) want {fw[i]!r} ({w[i]})")
