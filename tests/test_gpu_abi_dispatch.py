"""The reference's own call sequences through the C ABI, checked against the oracle.

A Rust musapy that links this library in place of its MUSA kernels does not go through this
repository's op layer: it follows rust/musapy-ops/src/op_builder.rs, which picks the entry point
and the tiling itself.  This file replays that dispatch with ctypes on device pointers:

* reductions (op_builder.rs:2511-3098):
  - axis_len > 1024: `_partial_` with tiles = ceil(axis_len / 1024) (2523); while tiles > 32768
    the partials are fed back, as an [out_size, tiles] array, to the same op's `_partial_`
    (sum partial for mean, 2797-2816 and 2238-2266) or, for argmax/argmin, to `_mid_`
    (2275-2301, 2594); then `_final_` (complex finals and the mean final take axis_len);
  - 16 < axis_len <= 1024 (not arg): `_small_axis_` with group_size 32/64/128/256 (3024-3036);
  - otherwise the one-pass entry point (arg reductions up to 1024);
  - axis=None reduces the materialised 1-D array (2464-2473);
* cumsum (3288-3326): `tmp` sized by the reference's formula, NULL when one block covers a row.

Bars: max/min/argmax/argmin and int64 results bit-exact; sums and means within
tol * sum|x| (tol 1e-5 f32/c64, 1e-12 f64/c128); products within 20 eps sqrt(n) relative; cumsum
within 1e-12 of each prefix's magnitude (f64 on U(0,1)), bit-exact for int64.
"""
import ctypes
import math
import os

import numpy as np
import pytest

import musapy_amd as ms
from oracle import reference as R
from tests.conftest import assert_bits_equal

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "musapy_amd", "libmusapy_hip.so")
RNG = np.random.default_rng(2523)
P, I, U = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
SZ, SS = ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_ssize_t)
SFX = {np.int64: "i64", np.float32: "f32", np.float64: "f64", np.complex64: "c64", np.complex128: "c128"}
TOL = {np.float32: 1e-5, np.float64: 1e-12, np.complex64: 1e-5, np.complex128: 1e-12}
_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = ctypes.CDLL(LIB)
        _lib.mpy_rt_check_launch.restype = ctypes.c_int
    return _lib


def fn(name, argtypes):
    f = getattr(lib(), name)
    f.argtypes = argtypes
    f.restype = None
    return f


class Calls:
    """Counts the entry points a dispatch used, so each test can show what it covered."""

    def __init__(self):
        self.names = []

    def __call__(self, name, argtypes, *args):
        fn(name, argtypes)(*args)
        assert lib().mpy_rt_check_launch() == 0, name
        self.names.append(name)


def dev_zeros(n, dt):
    return ms.from_numpy(np.zeros(max(int(n), 1), dt))


def view_args(base_dev, base, view):
    """Device pointer, shape and element strides of a numpy view of `base`, on the device copy."""
    es = base.itemsize
    off = (view.__array_interface__["data"][0] - base.__array_interface__["data"][0]) // es
    shape = (ctypes.c_size_t * max(view.ndim, 1))(*view.shape)
    strides = (ctypes.c_ssize_t * max(view.ndim, 1))(*[s // es for s in view.strides])
    return base_dev.data_ptr + off * es, shape, strides


RED_ARGS = [I, SZ, SS, I, U, U]


def reduce_like_op_builder(kind, x_ptr, ndim, shape, strides, axis, axis_len, out_size, out_ptr, dt, stream,
                           calls):
    """op_builder.rs reduction_axis, Device::Musa branch, for compute dtype `dt`."""
    sfx = SFX[dt]
    arg = kind in ("argmax", "argmin")
    cplx = sfx in ("c64", "c128")
    if axis_len > 1024:
        tiles = (axis_len + 1023) // 1024
        if arg:
            pv, pi = dev_zeros(out_size * tiles, dt), dev_zeros(out_size * tiles, np.int64)
            keep = [pv, pi]
            calls(f"musapy_{kind}_partial_{sfx}_v2", [P, P, P] + RED_ARGS + [U, P], x_ptr, pv.data_ptr, pi.data_ptr,
                  ndim, shape, strides, axis, axis_len, out_size, tiles, stream)
            sv, si = pv.data_ptr, pi.data_ptr
            while tiles > 32768:
                nt = (tiles + 1023) // 1024
                dv, di = dev_zeros(out_size * nt, dt), dev_zeros(out_size * nt, np.int64)
                keep += [dv, di]
                calls(f"musapy_{kind}_mid_{sfx}_v2", [P, P, P, P, U, U, U, P], sv, si, dv.data_ptr, di.data_ptr,
                      out_size, nt, tiles, stream)
                sv, si, tiles = dv.data_ptr, di.data_ptr, nt
            calls(f"musapy_{kind}_final_{sfx}_v2", [P, P, P, U, U, P], sv, si, out_ptr, tiles, out_size, stream)
            return keep
        pp = dev_zeros(out_size * tiles, dt)
        keep = [pp]
        calls(f"musapy_{kind}_partial_{sfx}_v2", [P, P] + RED_ARGS + [U, P], x_ptr, pp.data_ptr, ndim, shape, strides,
              axis, axis_len, out_size, tiles, stream)
        src = pp.data_ptr
        mid = "sum" if kind == "mean" else kind
        while tiles > 32768:
            nt = (tiles + 1023) // 1024
            dst = dev_zeros(out_size * nt, dt)
            keep.append(dst)
            sh = (ctypes.c_size_t * 2)(out_size, tiles)
            st = (ctypes.c_ssize_t * 2)(tiles, 1)
            calls(f"musapy_{mid}_partial_{sfx}_v2", [P, P] + RED_ARGS + [U, P], src, dst.data_ptr, 2, sh, st, 1, tiles,
                  out_size, nt, stream)
            src, tiles = dst.data_ptr, nt
        if kind == "mean" or cplx:
            calls(f"musapy_{kind}_final_{sfx}_v2", [P, P, U, U, U, P], src, out_ptr, tiles, out_size, axis_len, stream)
        else:
            calls(f"musapy_{kind}_final_{sfx}_v2", [P, P, U, U, P], src, out_ptr, tiles, out_size, stream)
        return keep
    if axis_len > 16 and not arg:
        gs = 32 if axis_len <= 32 else 64 if axis_len <= 64 else 128 if axis_len <= 128 else 256
        calls(f"musapy_{kind}_small_axis_{sfx}_v2", [P, P] + RED_ARGS + [I, P], x_ptr, out_ptr, ndim, shape, strides,
              axis, axis_len, out_size, gs, stream)
        return []
    calls(f"musapy_{kind}_{sfx}_v2", [P, P] + RED_ARGS + [P], x_ptr, out_ptr, ndim, shape, strides, axis, axis_len,
          out_size, stream)
    return []


def data(kind, dt, shape):
    if dt == np.int64:
        return RNG.integers(-1000, 1001, shape, dtype=np.int64)
    if kind == "prod":
        x = RNG.uniform(0.999, 1.001, shape)
        if dt in (np.complex64, np.complex128):
            x = x + 1j * RNG.uniform(-1e-3, 1e-3, shape)
        return x.astype(dt)
    x = RNG.standard_normal(shape)
    if dt in (np.complex64, np.complex128):
        x = x + 1j * RNG.standard_normal(shape)
    return x.astype(dt)


def check(kind, got, want, xv, axis, what):
    if kind in ("max", "min", "argmax", "argmin") or want.dtype == np.int64:
        assert_bits_equal(got, want, what)
        return
    assert got.shape == want.shape and got.dtype == want.dtype, what
    n = xv.size // max(want.size, 1)
    if kind == "prod":
        eps = 1.2e-7 if want.dtype in (np.float32, np.complex64) else 2.3e-16
        err = np.abs(got.astype(np.complex128) - want) / np.maximum(np.abs(want), 1e-300)
        assert np.all(err <= 20 * eps * math.sqrt(n) + 4 * eps), f"{what}: max rel err {err.max()}"
        return
    ax = None if axis is None else (axis,)
    scale = np.sum(np.abs(xv.astype(np.complex128)), axis=ax)
    if kind == "mean":
        scale = scale / max(n, 1)
    err = np.abs(got.astype(np.complex128) - want.astype(np.complex128))
    assert np.all(err <= TOL[want.dtype.type] * scale + 1e-30), f"{what}: max err {err.max()}"


def run_case(kind, dt, base, view, axis, calls):
    """Reduce `view` (a numpy view of `base`) over `axis` (None: the whole array) through the ABI."""
    B = ms.from_numpy(base)
    out_dt = np.int64 if kind in ("argmax", "argmin") else dt
    if axis is None:
        flat = np.ascontiguousarray(view).reshape(-1)
        F = ms.from_numpy(flat)  # the reference materialises axis=None inputs (op_builder.rs:2464-2473)
        x_ptr, ndim = F.data_ptr, 1
        shape = (ctypes.c_size_t * 1)(flat.size)
        strides = (ctypes.c_ssize_t * 1)(1)
        kaxis, axis_len, out_size, stream = 0, flat.size, 1, F.stream_ptr
        out_shape = ()
    else:
        x_ptr, shape, strides = view_args(B, base, view)
        ndim, kaxis, axis_len = view.ndim, axis, view.shape[axis]
        out_shape = tuple(d for i, d in enumerate(view.shape) if i != axis)
        out_size = max(int(np.prod(out_shape)), 1)
        stream = B.stream_ptr
    O = dev_zeros(out_size, out_dt)
    ms.synchronize()
    keep = reduce_like_op_builder(kind, x_ptr, ndim, shape, strides, kaxis, axis_len, out_size, O.data_ptr, dt,
                                  stream, calls)
    ms.synchronize()
    got = O.numpy()[:out_size].reshape(out_shape)
    want = R.reduction_axis(np.ascontiguousarray(view) if axis is None else view, axis, False, kind)
    check(kind, got, want, view, axis, f"{kind} {np.dtype(dt).name} view {view.shape} {view.strides} axis={axis}")
    del keep


VALUE_KINDS = ["sum", "prod", "max", "min", "mean"]


# (kind, dtype) of the real entry points: there is no integer mean (integer means reduce in float64,
# reduction_compute_dtype), so that pair is not a case
REAL_CASES = [(k, d) for k in VALUE_KINDS + ["argmax", "argmin"] for d in (np.int64, np.float32, np.float64)
              if not (k == "mean" and d == np.int64)]
REAL_IDS = [f"{k}-{np.dtype(d).name}" for k, d in REAL_CASES]


def layouts(shape, dt, kind):
    """C-contiguous, transposed and reversed/stepped views of a 2-D base."""
    base = data(kind, dt, shape)
    yield base, base
    yield base, base.T
    yield base, base[::-1, ::2] if shape[1] > 1 else base[::-1]


@pytest.mark.parametrize("kind,dt", REAL_CASES, ids=REAL_IDS)
def test_one_pass_and_small_axis(kind, dt):
    """axis_len <= 16: one pass; 16 < axis_len <= 1024: `_small_axis_` with each group size (arg
    reductions take the one-pass entry point up to 1024)."""
    calls = Calls()
    for shape in ((37, 11), (300, 17), (96, 33), (100, 64), (64, 100), (40, 129), (20, 1000), (5, 1024)):
        for base, view in layouts(shape, dt, kind):
            for axis in range(view.ndim):
                run_case(kind, dt, base, view, axis, calls)
    used = set(calls.names)
    if kind in ("argmax", "argmin"):
        assert used == {f"musapy_{kind}_{SFX[dt]}_v2"}, used
    else:
        assert {f"musapy_{kind}_small_axis_{SFX[dt]}_v2", f"musapy_{kind}_{SFX[dt]}_v2"} <= used, used


@pytest.mark.parametrize("dt", [np.complex64, np.complex128])
@pytest.mark.parametrize("kind", ["sum", "prod", "mean"])
def test_complex_entry_points(kind, dt):
    """Complex sum/prod/mean through the one-pass, small-axis and partial + final entry points."""
    calls = Calls()
    for shape in ((37, 11), (50, 200), (8, 3000)):
        for base, view in layouts(shape, dt, kind):
            for axis in range(view.ndim):
                run_case(kind, dt, base, view, axis, calls)
    s = SFX[dt]
    assert {f"musapy_{kind}_{s}_v2", f"musapy_{kind}_small_axis_{s}_v2", f"musapy_{kind}_partial_{s}_v2",
            f"musapy_{kind}_final_{s}_v2"} <= set(calls.names)


@pytest.mark.parametrize("kind,dt", REAL_CASES, ids=REAL_IDS)
def test_partial_then_final(kind, dt):
    """axis_len > 1024: partial with ceil(axis_len / 1024) tiles, then final (no re-feed)."""
    calls = Calls()
    for shape in ((16, 5000), (3, 70000), (1025, 8)):
        for base, view in layouts(shape, dt, kind):
            for axis in range(view.ndim):
                run_case(kind, dt, base, view, axis, calls)
    x = data(kind, dt, (4, 3000, 5))
    for axis in (0, 1, 2, None):
        run_case(kind, dt, x, x, axis, calls)
        run_case(kind, dt, x, x.transpose(2, 0, 1), axis, calls)
    s = SFX[dt]
    assert {f"musapy_{kind}_partial_{s}_v2", f"musapy_{kind}_final_{s}_v2"} <= set(calls.names)


# (kind, compute dtype) pairs of the multi-stage re-feed: one per `_mid_` symbol plus the value ops
MULTI = [("argmax", np.float32), ("argmin", np.float32), ("argmax", np.float64), ("argmin", np.float64),
         ("argmax", np.int64), ("argmin", np.int64), ("sum", np.float32), ("mean", np.float32),
         ("max", np.float32), ("min", np.float64), ("sum", np.int64), ("prod", np.float64)]


@pytest.mark.parametrize("kind,dt", MULTI, ids=[f"{k}-{np.dtype(d).name}" for k, d in MULTI])
def test_multi_stage_refeed(kind, dt):
    """axis_len > 32M: tiles = ceil(axis_len / 1024) > 32768, so the partials are reduced once more
    (arg: `_mid_`; others: the partial entry point over [out_size, tiles]) before the final."""
    n = 33_600_000 + 777  # 32,814 tiles -> 33 -> final
    x = data(kind, dt, (n,))
    if kind in ("argmax", "argmin", "max", "min"):
        # plant ties across tiles and stages: the first occurrence (lowest index) must win
        v = x.max() if kind in ("argmax", "max") else x.min()
        for k in (5_000_123, 17_000_000, 33_000_001):
            x[k] = v + (1 if kind in ("argmax", "max") else -1) * (1 if dt == np.int64 else 0.5)
    calls = Calls()
    run_case(kind, dt, x, x, 0, calls)
    s = SFX[dt]
    if kind in ("argmax", "argmin"):
        assert calls.names == [f"musapy_{kind}_partial_{s}_v2", f"musapy_{kind}_mid_{s}_v2",
                               f"musapy_{kind}_final_{s}_v2"]
    else:
        mid = "sum" if kind == "mean" else kind
        assert calls.names == [f"musapy_{kind}_partial_{s}_v2", f"musapy_{mid}_partial_{s}_v2",
                               f"musapy_{kind}_final_{s}_v2"]


def test_multi_stage_nan_rules():
    """The NaN-at-position-0 rule and skipped later NaNs survive the partial -> mid -> final chain."""
    n = 33_600_000 + 777
    x = RNG.standard_normal(n).astype(np.float32)
    x[[3, 9_000_000, 33_000_000]] = np.nan
    calls = Calls()
    for kind in ("argmax", "argmin", "max", "min"):
        run_case(kind, np.float32, x, x, 0, calls)
    x[0] = np.nan
    for kind in ("argmax", "max"):
        run_case(kind, np.float32, x, x, 0, calls)


@pytest.mark.parametrize("dt", [np.int64, np.float32, np.float64])
def test_cumsum_with_reference_scratch(dt):
    """musapy_cumsum_<T>_v3 with `tmp` of num_rows * (bpr [+ ceil(bpr/256)]) elements, bpr =
    ceil(axis_len / 256), and tmp = NULL when bpr == 1 (op_builder.rs:3288-3326)."""
    cs = fn(f"musapy_cumsum_{SFX[dt]}_v3", [P, P, P, I, SZ, SS, I, U, U, P])
    for shape, axis in (((7, 200), 1), ((3, 256), 1), ((3, 257), 1), ((5, 4096), 1), ((4, 65536), 1),
                        ((2, 65537), 1), ((600, 3000), 1), ((3000, 70), 0), ((9, 40, 11), 1), ((1, 300_000), 1)):
        base = RNG.integers(-1000, 1001, shape, dtype=np.int64) if dt == np.int64 else RNG.random(shape).astype(dt)
        for view in (base, base[:, ::-1] if base.ndim == 2 else base.transpose(0, 2, 1)):
            ax = axis if view is base or view.ndim == 2 else (2 if axis == 1 else axis)
            B = ms.from_numpy(base)
            x_ptr, sh, st = view_args(B, base, view)
            L = view.shape[ax]
            total = view.size
            bpr = (L + 255) // 256
            rows = total // L
            scratch = rows * (bpr + (bpr + 255) // 256) if bpr > 256 else rows * bpr
            T = dev_zeros(scratch, dt) if bpr > 1 else None
            O = dev_zeros(total, dt)
            ms.synchronize()
            cs(x_ptr, O.data_ptr, T.data_ptr if T is not None else None, view.ndim, sh, st, ax, L, total, B.stream_ptr)
            assert lib().mpy_rt_check_launch() == 0
            ms.synchronize()
            got = O.numpy()[:total].reshape(view.shape)
            want = R.cumsum(view, ax)
            what = f"cumsum {np.dtype(dt).name} {view.shape} {view.strides} axis={ax}"
            if dt == np.int64:
                assert_bits_equal(got, want, what)
                continue
            tol = 1e-5 if dt == np.float32 else 1e-12
            bound = tol * np.cumsum(np.abs(view.astype(np.float64)), axis=ax)
            if dt == np.float32 and L > 65536:
                # The reference's sequential f32 running sum itself drifts by about sqrt(L) * eps
                # * sum|x| (3e-5 relative at L = 300,000 on U(0,1) data), more than the bound, and a
                # tiled scan cannot follow that drift: the bound is widened by the reference's own
                # distance from the exact prefix sums (the sequential column/strided kernel still
                # matches it exactly; a tiled row scan is held to the exact sums).
                bound = bound + np.abs(want - np.cumsum(view.astype(np.float64), axis=ax))
            assert np.all(np.abs(got.astype(np.float64) - want) <= bound + 1e-30), what


@pytest.mark.parametrize("dt", [np.int64, np.float32, np.float64])
def test_cumsum_workspace_entry_matches_scratch_entry(dt):
    """musapy_cumsum_ws_v1 (new; the chained scan on a zeroed workspace, no clearing launch) gives
    the bits of musapy_cumsum_<T>_v3 on the same rows, leaves the workspace zero for the next call
    (two calls in a row, the second smaller), and declines (-1, nothing launched) the shapes that
    do not take the chained path."""
    DT = {np.int64: 4, np.float32: 10, np.float64: 11}[dt]  # MUSAPY_DT_I64 / _F32 / _F64
    ws_fn = getattr(lib(), "musapy_cumsum_ws_v1")
    ws_fn.argtypes = [I, P, P, I, SZ, SS, I, U, U, P, U, P]
    ws_fn.restype = ctypes.c_int
    cs = fn(f"musapy_cumsum_{SFX[dt]}_v3", [P, P, P, I, SZ, SS, I, U, U, P])
    WS = dev_zeros(1 << 17, np.uint64)  # 1 MiB
    # 16 KB tiles, then the same on a smaller call, then 64 KB tiles (rows of at least two of them)
    for shape in ((1030, 9000), (520, 4097), (520, 33000)):
        base = RNG.integers(-1000, 1001, shape, dtype=np.int64) if dt == np.int64 else RNG.random(shape).astype(dt)
        B = ms.from_numpy(base)
        x_ptr, sh, st = view_args(B, base, base)
        L, total = shape[1], base.size
        O1, O2 = dev_zeros(total, dt), dev_zeros(total, dt)
        bpr = (L + 255) // 256
        T = dev_zeros(shape[0] * (bpr + (bpr + 255) // 256 if bpr > 256 else bpr), dt)
        ms.synchronize()
        assert ws_fn(DT, x_ptr, O1.data_ptr, 2, sh, st, 1, L, total, WS.data_ptr, 1 << 20, B.stream_ptr) == 0
        assert lib().mpy_rt_check_launch() == 0
        cs(x_ptr, O2.data_ptr, T.data_ptr, 2, sh, st, 1, L, total, B.stream_ptr)
        assert lib().mpy_rt_check_launch() == 0
        ms.synchronize()
        got = O1.numpy()[:total].reshape(shape)
        assert_bits_equal(got, O2.numpy()[:total].reshape(shape), f"ws vs scratch entry {shape}")
        if dt == np.int64:
            assert_bits_equal(got, R.cumsum(base, 1), f"ws entry {shape}")
        else:
            want = R.cumsum(base, 1)
            bound = TOL[dt] * np.cumsum(np.abs(base.astype(np.float64)), axis=1) + np.abs(
                want - np.cumsum(base.astype(np.float64), axis=1))
            assert np.all(np.abs(got.astype(np.float64) - want) <= bound), f"ws entry {shape}"
        assert not WS.numpy().any(), "the workspace is left zero"
    # not the chained path: few rows, a strided axis, a workspace too small
    x = RNG.random((8, 9000)).astype(dt) if dt != np.int64 else RNG.integers(0, 9, (8, 9000))
    X = ms.from_numpy(x)
    x_ptr, sh, st = view_args(X, x, x)
    O = dev_zeros(x.size, dt)
    assert ws_fn(DT, x_ptr, O.data_ptr, 2, sh, st, 1, 9000, x.size, WS.data_ptr, 1 << 20, X.stream_ptr) == -1
    y = RNG.random((1030, 9000)).astype(dt) if dt != np.int64 else RNG.integers(0, 9, (1030, 9000))
    Y = ms.from_numpy(y)
    y_ptr, sh, st = view_args(Y, y, y)
    assert ws_fn(DT, y_ptr, O.data_ptr, 2, sh, st, 0, 1030, y.size, WS.data_ptr, 1 << 20, Y.stream_ptr) == -1
    assert ws_fn(DT, y_ptr, O.data_ptr, 2, sh, st, 1, 9000, y.size, WS.data_ptr, 1024, Y.stream_ptr) == -1
    assert lib().mpy_rt_check_launch() == 0
