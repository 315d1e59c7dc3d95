"""Bounded device waits that run out are reported, not folded into a wrong result.

The combiner of a single-launch reduction and the look-back of a tiled row scan wait for other
workgroups.  Each wait polls a bounded number of times; `musapy_kernels_set_spin_limit(0)` makes
every such wait give up before its first poll, so the error path runs while every kernel still
exits normally (nothing here makes the GPU fault or hang).  Expected behaviour, as the reference
surfaces execution errors at stream synchronisation (rust/musapy-core/src/stream.rs:311-377):
the synchronize that covers the work raises KernelError and poisons the stream, and the next
reduction on that stream is correct again.
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
RNG = np.random.default_rng(41)


def _lib():
    lib = ctypes.CDLL(LIB)
    lib.musapy_kernels_set_spin_limit.restype = ctypes.c_uint32
    lib.musapy_kernels_set_spin_limit.argtypes = [ctypes.c_uint32]
    lib.musapy_kernels_take_fault.restype = ctypes.c_int
    lib.musapy_kernels_take_fault.argtypes = [ctypes.c_int]
    return lib


class _NoPolls:
    """Every bounded wait gives up at once while inside the block."""

    def __init__(self, lib):
        self.lib = lib

    def __enter__(self):
        self.prev = self.lib.musapy_kernels_set_spin_limit(0)
        return self

    def __exit__(self, *exc):
        self.lib.musapy_kernels_set_spin_limit(self.prev)


def _fresh_stream_case(make, run, check):
    """Runs `run` on its own stream with no polls allowed, expects KernelError at the readback,
    then runs it again with the default limit and checks the result."""
    lib = _lib()
    s = ms.Stream()
    with ms.stream(s):
        inputs = make()
        good = run(*inputs).numpy()  # the normal path first
        check(good, "before the forced fault")
        with _NoPolls(lib):
            bad = run(*inputs)
            with pytest.raises(ms.KernelError, match="device wait expired"):
                bad.numpy()
        assert s.is_poisoned
        again = run(*inputs).numpy()  # same stream, default limit again
        check(again, "after the forced fault")
        assert_bits_equal(again, good, "rerun on the recovered stream")
    assert lib.musapy_kernels_take_fault(0) == 0  # the fault was consumed by the readback


def test_whole_array_reduction_gives_up_and_recovers():
    x = RNG.standard_normal(1 << 22).astype(np.float32)
    want = R.reduce(x, "sum", None)

    def check(got, what):
        assert abs(float(got) - float(want)) <= 1e-5 * np.abs(x).sum(), what

    _fresh_stream_case(lambda: (ms.from_numpy(x),), lambda X: ms.sum(X), check)
    _fresh_stream_case(lambda: (ms.from_numpy(x),), lambda X: ms.argmax(X),
                       lambda got, what: assert_bits_equal(got, R.reduce(x, "argmax", None), what))


def test_row_reduction_gives_up_and_recovers():
    x = RNG.standard_normal((8, 1 << 20)).astype(np.float32)
    _fresh_stream_case(lambda: (ms.from_numpy(x),), lambda X: ms.argmax(X, axis=1),
                       lambda got, what: assert_bits_equal(got, R.reduce(x, "argmax", 1), what))
    _fresh_stream_case(lambda: (ms.from_numpy(x),), lambda X: ms.max(X, axis=1),
                       lambda got, what: assert_bits_equal(got, R.reduce(x, "max", 1), what))


def test_column_reduction_gives_up_and_recovers():
    """Column sums and means in one launch: the group's last block finds no tile published."""
    x = RNG.standard_normal((4096, 2048)).astype(np.float32)
    for op in ("sum", "mean"):
        want = R.reduce(x, op, 0)

        def check(got, what, want=want):
            assert np.all(np.abs(got - want) <= 1e-5 * np.abs(x).sum(axis=0)), what

        _fresh_stream_case(lambda: (ms.from_numpy(x),), lambda X, op=op: getattr(ms, op)(X, axis=0), check)


def test_two_axis_reduction_gives_up_and_recovers():
    """max / min over (0, 1) in one launch (row-keyed kernel, 3000 rows; chunked kernel, 600 rows of
    8192): the combiner finds no key published, and the blocks that wait for row 0's flags find none
    and fold their rows masked instead (always right).  Row 0 with and without a NaN head."""
    x = RNG.standard_normal((3000, 2048)).astype(np.float32)
    y = x.copy()
    y[0, 3] = np.nan  # drops column 3, whatever it holds below
    y[2999, 3] = 1e30
    # rows of whole 8192-element chunks: the chunked kernel (its row-0 flags and keys time out)
    u = RNG.standard_normal((600, 8192)).astype(np.float32)
    v = u.copy()
    v[0, 8000] = np.nan
    v[599, 8000] = 1e30
    for arr in (x, y, u, v):
        for op in ("max", "min"):
            _fresh_stream_case(lambda arr=arr: (ms.from_numpy(arr),), lambda X, op=op: getattr(ms, op)(X, axis=(0, 1)),
                               lambda got, what, arr=arr, op=op: assert_bits_equal(got, R.reduce(arr, op, (0, 1)), what))


def test_row_scan_look_back_gives_up_and_recovers():
    y = RNG.random((4, 100_000))
    want = R.cumsum(y, 1)

    def check(got, what):
        assert np.all(np.abs(got - want) <= 1e-12 * np.abs(want)), what

    _fresh_stream_case(lambda: (ms.from_numpy(y),), lambda Y: ms.cumsum(Y, axis=1), check)


def test_chained_row_scan_gives_up_and_recovers():
    y = RNG.random((520, 20_000))
    want = R.cumsum(y, 1)

    def check(got, what):
        assert np.all(np.abs(got - want) <= 1e-12 * np.cumsum(np.abs(y), axis=1)), what

    _fresh_stream_case(lambda: (ms.from_numpy(y),), lambda Y: ms.cumsum(Y, axis=1), check)


def _fused_lib():
    lib = _lib()
    P, I, SZ, SS = ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_ssize_t)
    lib.musapy_reduce_fused_v1.restype = ctypes.c_int
    lib.musapy_reduce_fused_v1.argtypes = [I, I, P, P, I, SZ, SS, I, ctypes.c_size_t, ctypes.c_size_t,
                                           ctypes.c_size_t, P, ctypes.c_size_t, P]
    lib.musapy_kernels_take_fault_ws.restype = ctypes.c_int
    lib.musapy_kernels_take_fault_ws.argtypes = [P, ctypes.c_size_t, P]
    return lib


def test_c_abi_fault_word_and_workspace_reuse():
    """A caller of musapy_reduce_fused_v1 reads the fault in its own workspace's last word with
    musapy_kernels_take_fault_ws after its synchronize; taking it zeroes the workspace, so the
    next call on the same workspace is correct."""
    lib = _fused_lib()
    RED_SUM, DT_F64 = 0, 11
    x = RNG.standard_normal((4, 1 << 18))
    X = ms.from_numpy(x)
    C = ms.from_numpy(np.zeros(4))
    ws_words = 4 * 64 * 2 + 1  # the slots, then the fault word
    WS = ms.from_numpy(np.zeros(ws_words, np.uint64))
    shape = (ctypes.c_size_t * 2)(4, 1 << 18)
    strides = (ctypes.c_ssize_t * 2)(1 << 18, 1)
    ms.synchronize()
    st = X.stream_ptr
    assert lib.musapy_kernels_take_fault_ws(WS.data_ptr, ws_words * 8, st) == 0

    def call():
        return lib.musapy_reduce_fused_v1(RED_SUM, DT_F64, X.data_ptr, C.data_ptr, 2, shape, strides, 1, 1 << 18, 4,
                                          64, WS.data_ptr, ws_words * 8, st)

    # one word short of the slots and the fault word: refused, nothing launched
    assert lib.musapy_reduce_fused_v1(RED_SUM, DT_F64, X.data_ptr, C.data_ptr, 2, shape, strides, 1, 1 << 18, 4, 64,
                                      WS.data_ptr, (ws_words - 1) * 8, st) == -1
    with _NoPolls(lib):
        assert call() == 0
        ms.synchronize()
    assert lib.musapy_kernels_take_fault(0) == 0  # the no-alloc scratch's word is not this one
    assert lib.musapy_kernels_take_fault_ws(WS.data_ptr, ws_words * 8, st) == 1
    assert not WS.numpy().any(), "taking the fault zeroes the workspace"
    assert lib.musapy_kernels_take_fault_ws(WS.data_ptr, ws_words * 8, st) == 0
    assert call() == 0
    ms.synchronize()
    assert lib.musapy_kernels_take_fault_ws(WS.data_ptr, ws_words * 8, st) == 0
    got = C.numpy()
    want = R.reduce(x, "sum", 1)
    assert np.all(np.abs(got - want) <= 1e-12 * np.abs(x).sum(axis=1))
    assert not WS.numpy().any(), "the workspace is left zero"


def test_fault_is_reported_to_the_stream_whose_wait_expired():
    """Stream A queues a reduction that gives up (no polls), stream B one with the default limit.
    B's synchronize is clean and B is not poisoned; A's synchronize raises KernelError and poisons
    A; the next reduction on A is exact again (rust/musapy-core/src/stream.rs:311-377 poisons the
    stream whose synchronize failed)."""
    lib = _lib()
    x = RNG.standard_normal(1 << 22).astype(np.float32)
    y = RNG.standard_normal((8, 1 << 20)).astype(np.float32)
    a_s, b_s = ms.Stream(), ms.Stream()
    with ms.stream(a_s):
        X = ms.from_numpy(x)
    with ms.stream(b_s):
        Y = ms.from_numpy(y)
    ms.synchronize()
    with ms.stream(a_s):
        with _NoPolls(lib):
            bad = ms.argmax(X)
    with ms.stream(b_s):
        good = ms.argmax(Y, axis=1)
    b_s.synchronize()
    assert not b_s.is_poisoned
    assert_bits_equal(good.numpy(), R.reduce(y, "argmax", 1), "stream B's reduction")
    with pytest.raises(ms.KernelError, match="device wait expired"):
        a_s.synchronize()
    assert a_s.is_poisoned and not b_s.is_poisoned
    del bad
    with ms.stream(a_s):
        again = ms.argmax(X).numpy()
    assert_bits_equal(again, R.reduce(x, "argmax", None), "stream A after the fault")
    assert not b_s.is_poisoned


def test_device_synchronize_poisons_only_the_faulting_stream():
    """ms.synchronize() checks every stream with bounded waits queued: the one whose scan gave up
    raises and is poisoned, the other stream's results are exact and it stays clean."""
    lib = _lib()
    y = RNG.random((520, 20_000))
    x = RNG.standard_normal((4096, 2048)).astype(np.float32)
    a_s, b_s = ms.Stream(), ms.Stream()
    with ms.stream(a_s):
        Y = ms.from_numpy(y)
    with ms.stream(b_s):
        X = ms.from_numpy(x)
    ms.synchronize()
    with ms.stream(a_s):
        with _NoPolls(lib):
            ms.cumsum(Y, axis=1)
    with ms.stream(b_s):
        s0 = ms.sum(X, axis=0)
    with pytest.raises(ms.KernelError, match="device wait expired in a cumsum"):
        ms.synchronize()
    assert a_s.is_poisoned and not b_s.is_poisoned
    want = R.reduce(x, "sum", 0)
    assert np.all(np.abs(s0.numpy() - want) <= 1e-5 * np.abs(x).sum(axis=0))
    ms.synchronize()  # nothing left to report


def test_reference_signature_scan_reports_in_its_scratch():
    """musapy_cumsum_f64_v3 (the reference's signature) keeps its fault word in the last 8 bytes
    of the scratch capacity the reference's formula gives (op_builder.rs:3315-3321)."""
    lib = _lib()
    P, I, SZ, SS, U = (ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t),
                       ctypes.POINTER(ctypes.c_ssize_t), ctypes.c_size_t)
    lib.musapy_cumsum_f64_v3.restype = None
    lib.musapy_cumsum_f64_v3.argtypes = [P, P, P, I, SZ, SS, I, U, U, P]
    lib.musapy_kernels_take_fault_ws.restype = ctypes.c_int
    lib.musapy_kernels_take_fault_ws.argtypes = [P, U, P]
    rows, L = 4, 100_000
    y = RNG.random((rows, L))
    bpr = (L + 255) // 256
    cap = rows * (bpr + (bpr + 255) // 256 if bpr > 256 else bpr)
    Y = ms.from_numpy(y)
    O = ms.from_numpy(np.zeros_like(y))
    T = ms.from_numpy(np.full(cap, 7.0))  # garbage: the launch clears what it uses
    shape = (ctypes.c_size_t * 2)(rows, L)
    strides = (ctypes.c_ssize_t * 2)(L, 1)
    ms.synchronize()
    st = Y.stream_ptr
    with _NoPolls(lib):
        lib.musapy_cumsum_f64_v3(Y.data_ptr, O.data_ptr, T.data_ptr, 2, shape, strides, 1, L, rows * L, st)
        ms.synchronize()
    assert lib.musapy_kernels_take_fault_ws(T.data_ptr, cap * 8, st) == 2
    lib.musapy_cumsum_f64_v3(Y.data_ptr, O.data_ptr, T.data_ptr, 2, shape, strides, 1, L, rows * L, st)
    ms.synchronize()
    assert lib.musapy_kernels_take_fault_ws(T.data_ptr, cap * 8, st) == 0
    want = R.cumsum(y, 1)
    assert np.all(np.abs(O.numpy() - want) <= 1e-12 * np.abs(want))
