"""musapy_reduce_fused_noalloc_v1: the single-launch reduction with the library's static scratch.

Called through the C ABI and compared with musapy_reduce_fused_v1 given its own workspace (the
same kernels, so the results must agree bit for bit) and with the CPU oracle (the reduction
bars: bit-exact for max/min/arg and int64, tol * sum|x| for sums and means).  Two calls in a row,
the second on a smaller input, check that each call leaves the shared scratch clean for the next.
"""
import ctypes
import os

import numpy as np
import pytest

import musapy_amd as ms
from oracle import reference as R
from tests.conftest import assert_bits_equal

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "musapy_amd", "libmusapy_hip.so")
RNG = np.random.default_rng(7)
P, I, U = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
SZ, SS = ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_ssize_t)
OPS = {"sum": 0, "prod": 1, "max": 2, "min": 3, "mean": 4, "argmax": 5, "argmin": 6}
DT = {np.int64: 4, np.float32: 10, np.float64: 11, np.complex64: 13, np.complex128: 14}
SCRATCH_BYTES = (1 << 20) + 256  # as the library's scratch: 1 MiB of slots, then a line ending in its fault word


def lib():
    L = ctypes.CDLL(LIB)
    L.musapy_reduce_fused_v1.restype = ctypes.c_int
    L.musapy_reduce_fused_v1.argtypes = [I, I, P, P, I, SZ, SS, I, U, U, U, P, U, P]
    L.musapy_reduce_fused_noalloc_v1.restype = ctypes.c_int
    L.musapy_reduce_fused_noalloc_v1.argtypes = [I, I, P, P, I, SZ, SS, I, U, U, U, P]
    L.musapy_kernels_take_error.restype = ctypes.c_int
    L.musapy_kernels_take_fault.restype = ctypes.c_int
    L.musapy_kernels_take_fault.argtypes = [ctypes.c_int]
    L.musapy_kernels_set_spin_limit.restype = ctypes.c_uint32
    L.musapy_kernels_set_spin_limit.argtypes = [ctypes.c_uint32]
    return L


def data(kind, dt, shape):
    if dt == np.int64:
        return RNG.integers(-1000, 1001, shape, dtype=np.int64)
    if kind == "prod":
        x = RNG.uniform(0.999, 1.001, shape)
    else:
        x = RNG.standard_normal(shape)
    if dt in (np.complex64, np.complex128):
        x = x + 1j * RNG.standard_normal(shape) * (1e-3 if kind == "prod" else 1)
    return x.astype(dt)


def reduce_both(L, kind, dt, x, tiles):
    """(noalloc result, workspace result) of reducing the last axis of contiguous `x`."""
    rows, n = (1, x.size) if x.ndim == 1 else x.shape
    out_dt = np.int64 if kind.startswith("arg") else dt
    X = ms.from_numpy(x)
    C1 = ms.from_numpy(np.zeros(rows, out_dt))
    C2 = ms.from_numpy(np.zeros(rows, out_dt))
    WS = ms.from_numpy(np.zeros(SCRATCH_BYTES // 8, np.uint64))
    shape = (ctypes.c_size_t * x.ndim)(*x.shape)
    strides = (ctypes.c_ssize_t * x.ndim)(*[s // x.itemsize for s in x.strides])
    ms.synchronize()
    args = (OPS[kind], DT[dt], X.data_ptr)
    tail = (x.ndim, shape, strides, x.ndim - 1, n, rows, tiles)
    r1 = L.musapy_reduce_fused_noalloc_v1(*args, C1.data_ptr, *tail, X.stream_ptr)
    r2 = L.musapy_reduce_fused_v1(*args, C2.data_ptr, *tail, WS.data_ptr, SCRATCH_BYTES, X.stream_ptr)
    assert (r1, r2) == (0, 0), (kind, dt, x.shape, tiles, r1, r2)
    ms.synchronize()
    assert L.musapy_kernels_take_fault(0) == 0
    shape_out = () if x.ndim == 1 else (rows,)
    return C1.numpy().reshape(shape_out), C2.numpy().reshape(shape_out)


def check_oracle(kind, got, x):
    want = R.reduce(x, kind, x.ndim - 1)
    what = f"noalloc {kind} {x.dtype} {x.shape}"
    if kind in ("max", "min", "argmax", "argmin") or want.dtype == np.int64:
        assert_bits_equal(got, want, what)
        return
    if kind == "prod":
        err = np.abs(got.astype(np.complex128) - want) / np.abs(want)
        eps = 1.2e-7 if want.dtype in (np.float32, np.complex64) else 2.3e-16
        assert np.all(err <= 20 * eps * np.sqrt(x.shape[-1]) + 4 * eps), what
        return
    tol = 1e-5 if want.dtype in (np.float32, np.complex64) else 1e-12
    scale = np.sum(np.abs(x.astype(np.complex128)), axis=-1)
    if kind == "mean":
        scale = scale / x.shape[-1]
    assert np.all(np.abs(got.astype(np.complex128) - want) <= tol * scale + 1e-30), what


CASES = [(k, d) for d in (np.float32, np.float64, np.int64) for k in OPS if not (k == "mean" and d == np.int64)]
CASES += [(k, d) for d in (np.complex64, np.complex128) for k in ("sum", "prod", "mean")]


@pytest.mark.parametrize("kind,dt", CASES, ids=[f"{k}-{np.dtype(d).name}" for k, d in CASES])
def test_noalloc_matches_the_workspace_entry_point(kind, dt):
    L = lib()
    # whole array (persistent grid) then a smaller one; rows split into tiles then fewer rows
    for shape, tiles in (((1 << 21) + 333,), 512), (((1 << 19) + 5,), 64), ((48, 1 << 16), 8), ((5, 40_000), 8):
        x = data(kind, dt, shape)
        got, ref = reduce_both(L, kind, dt, x, tiles)
        assert_bits_equal(got, ref, f"noalloc vs workspace {kind} {np.dtype(dt).name} {shape} tiles={tiles}",
                          nan_bits=True)
        check_oracle(kind, got, x)


COL_CASES = [(k, d) for d in (np.float32, np.float64, np.int64, np.complex64) for k in ("sum", "mean", "prod")
             if not (k == "mean" and d == np.int64)]


@pytest.mark.parametrize("kind,dt", COL_CASES, ids=[f"{k}-{np.dtype(d).name}" for k, d in COL_CASES])
def test_noalloc_column_reductions(kind, dt):
    """Column sums, means and products (axis 0: a strided axis, unit-stride outputs) run in one
    launch through the static scratch too (the column kernel's last block per group folds): two
    calls in a row, the second smaller, agree bit for bit with the workspace entry point."""
    L = lib()
    for (rows, cols), tiles in (((1024, 2048), 8), ((300, 700), 4)):
        x = data(kind, dt, (rows, cols))
        X = ms.from_numpy(x)
        C1 = ms.from_numpy(np.zeros(cols, dt))
        C2 = ms.from_numpy(np.zeros(cols, dt))
        WS = ms.from_numpy(np.zeros(SCRATCH_BYTES // 8, np.uint64))
        shape = (ctypes.c_size_t * 2)(rows, cols)
        strides = (ctypes.c_ssize_t * 2)(cols, 1)
        ms.synchronize()
        args = (OPS[kind], DT[dt], X.data_ptr)
        tail = (2, shape, strides, 0, rows, cols, tiles)
        r1 = L.musapy_reduce_fused_noalloc_v1(*args, C1.data_ptr, *tail, X.stream_ptr)
        r2 = L.musapy_reduce_fused_v1(*args, C2.data_ptr, *tail, WS.data_ptr, SCRATCH_BYTES, X.stream_ptr)
        assert (r1, r2) == (0, 0), (kind, dt, rows, cols, tiles, r1, r2)
        ms.synchronize()
        assert L.musapy_kernels_take_fault(0) == 0
        got, ref = C1.numpy(), C2.numpy()
        what = f"noalloc columns {kind} {np.dtype(dt).name} ({rows}, {cols}) tiles={tiles}"
        assert_bits_equal(got, ref, what, nan_bits=True)
        want = R.reduce(x, kind, 0)
        if want.dtype == np.int64:
            assert_bits_equal(got, want, what)
        elif kind == "prod":
            eps = 1.2e-7 if want.dtype in (np.float32, np.complex64) else 2.3e-16
            err = np.abs(got.astype(np.complex128) - want) / np.abs(want)
            assert np.all(err <= 20 * eps * np.sqrt(rows) + 4 * eps), what
        else:
            tol = 1e-5 if want.dtype in (np.float32, np.complex64) else 1e-12
            scale = np.sum(np.abs(x.astype(np.complex128)), axis=0) / (rows if kind == "mean" else 1)
            assert np.all(np.abs(got.astype(np.complex128) - want) <= tol * scale + 1e-30), what


def test_noalloc_refuses_more_slots_than_the_scratch_holds():
    """64 outputs x 513 tiles of f64 max need 64*513*4 = 131,328 words, more than the 131,072 of
    the 1 MiB scratch: refused with -2 and wrapper error 5, nothing launched; the next call,
    with 256 tiles, fits and works."""
    L = lib()
    n = 513 * 2048
    x = RNG.standard_normal((64, n))
    X = ms.from_numpy(x)
    C = ms.from_numpy(np.full(64, -1.0))
    shape = (ctypes.c_size_t * 2)(64, n)
    strides = (ctypes.c_ssize_t * 2)(n, 1)
    ms.synchronize()
    L.musapy_kernels_take_error()
    r = L.musapy_reduce_fused_noalloc_v1(OPS["max"], DT[np.float64], X.data_ptr, C.data_ptr, 2, shape, strides, 1,
                                         n, 64, 513, X.stream_ptr)
    assert r == -2
    assert L.musapy_kernels_take_error() == 5
    ms.synchronize()
    assert C.numpy().tolist() == [-1.0] * 64  # nothing was written
    r = L.musapy_reduce_fused_noalloc_v1(OPS["max"], DT[np.float64], X.data_ptr, C.data_ptr, 2, shape, strides, 1,
                                         n, 64, 256, X.stream_ptr)
    assert r == 0
    ms.synchronize()
    assert_bits_equal(C.numpy(), R.reduce(x, "max", 1), "noalloc max after the refused call")


def test_noalloc_fault_is_taken_once_and_the_next_call_starts_clean():
    """A no-alloc reduction whose combiner gives up (no polls allowed) reports through the
    scratch's fault word, once; the next no-alloc call zeroes the scratch on its own stream first
    and matches the workspace entry point bit for bit, twice in a row (the second smaller)."""
    L = lib()
    x = data("sum", np.float32, (1 << 21) + 333)
    X = ms.from_numpy(x)
    C = ms.from_numpy(np.zeros(1, np.float32))
    shape = (ctypes.c_size_t * 1)(x.size)
    strides = (ctypes.c_ssize_t * 1)(1)
    ms.synchronize()
    assert L.musapy_kernels_take_fault(0) == 0
    prev = L.musapy_kernels_set_spin_limit(0)
    try:
        r = L.musapy_reduce_fused_noalloc_v1(OPS["sum"], DT[np.float32], X.data_ptr, C.data_ptr, 1, shape, strides, 0,
                                             x.size, 1, 512, X.stream_ptr)
    finally:
        L.musapy_kernels_set_spin_limit(prev)
    assert r == 0
    ms.synchronize()
    assert L.musapy_kernels_take_fault(0) == 1
    assert L.musapy_kernels_take_fault(0) == 0  # reported once
    for n, tiles in ((1 << 21) + 333, 512), ((1 << 19) + 5, 64):
        got, ref = reduce_both(L, "sum", np.float32, x[:n], tiles)
        assert_bits_equal(got, ref, f"noalloc after a fault, n={n}", nan_bits=True)
        check_oracle("sum", got, x[:n])
