"""GPU parity of contiguous() materialisation against the CPU oracle (bit-exact, NaN payloads too).

Covers every element size the copy kernels take (1, 2, 4, 8 and 16 bytes), the reference's
transpose2d dispatch (the transposed view of a C-contiguous 2-D array) and the general stride
walk (flips, stepped slices, offsets, 3-D permutes), the reference's known answers
(tests/python/test_indexing.py TestContiguous / GPU tiled-transpose shapes), and the
musapy_copy_transpose2d_* and musapy_copy_* entry points called directly through the C ABI.
"""
import ctypes
import os

import numpy as np
import pytest

import musapy_amd as ms
from oracle import reference as R
from tests.conftest import assert_bits_equal, ulp_diff_f32

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(4242)
LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "musapy_amd", "libmusapy_hip.so")
DTYPES = [np.bool_, np.int8, np.uint8, np.int16, np.float16, np.int32, np.float32, np.int64, np.float64,
          np.complex64, np.complex128]


def rand(shape, dt):
    n = int(np.prod(shape)) * np.dtype(dt).itemsize
    raw = RNG.integers(0, 256, n, dtype=np.uint8)
    if dt == np.bool_:
        raw = raw & 1
    return raw.view(dt).reshape(shape)


def check(got_arr, want, what):
    assert got_arr.is_contiguous(), what
    assert_bits_equal(got_arr.numpy(), want, what, nan_bits=True)


@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: np.dtype(d).name)
def test_contiguous_views(dt):
    x = rand((6, 10, 36), dt)
    X = ms.from_numpy(x)
    views = [
        ("T", lambda a: ms.transpose(a), lambda v: v.T),
        ("permute102", lambda a: ms.permute(a, [1, 0, 2]), lambda v: v.transpose(1, 0, 2)),
        ("permute201", lambda a: ms.permute(a, [2, 0, 1]), lambda v: v.transpose(2, 0, 1)),
        ("flip2", lambda a: ms.flip(a, 2), lambda v: v[:, :, ::-1]),
        ("flip0", lambda a: ms.flip(a, 0), lambda v: v[::-1]),
        ("sliced", lambda a: ms.slice(a, [(1, 6, 2), (0, 10, 3), (5, 35, 1)]), lambda v: v[1:6:2, ::3, 5:35]),
        ("offset", lambda a: ms.slice(a, [(0, 6, 1), (0, 10, 1), (1, 36, 1)]), lambda v: v[:, :, 1:]),
        ("select", lambda a: ms.index_select(a, 1, 7), lambda v: v[:, 7, :]),
        ("getitem", lambda a: a[2:, 1, ::5], lambda v: v[2:, 1, ::5]),
        ("empty", lambda a: ms.slice(a, [(0, 6, 1), (3, 3, 1), (0, 36, 1)]), lambda v: v[:, 3:3, :]),
    ]
    for name, df, nf in views:
        check(ms.contiguous(df(X)), R.contiguous(nf(x)), f"{np.dtype(dt).name} {name}")
    # the 2-D transposed view (transpose2d dispatch) and a contiguous no-op
    y = rand((37, 1000), dt)
    Y = ms.from_numpy(y)
    check(ms.contiguous(ms.transpose(Y)), R.contiguous(y.T), f"{np.dtype(dt).name} 2-D transpose")
    same = ms.contiguous(Y)
    assert same.data_ptr == Y.data_ptr
    check(same, y, "no-op")


def test_contiguous_tiled_transpose_reference_shapes():
    """tests/python/test_indexing.py::test_gpu_contig_transpose_tiled(_dtypes) shapes."""
    for r, c in [(1024, 1024), (1000, 37), (37, 1000), (31, 33), (33, 31), (32, 32), (5, 5), (1, 100), (100, 1),
                 (2, 1025)]:
        data = RNG.random((r, c), dtype=np.float32)
        got = ms.contiguous(ms.transpose(ms.from_numpy(data)))
        assert got.shape == (c, r)
        check(got, R.contiguous(data.T), f"f32 {r}x{c}")
    d64 = RNG.random((257, 63))
    check(ms.contiguous(ms.transpose(ms.from_numpy(d64))), R.contiguous(d64.T), "f64 257x63")
    di = RNG.integers(-1000, 1000, (63, 257))
    for dtype in (np.int64, np.int32):
        a = ms.from_numpy(di.astype(dtype))
        assert ms.contiguous(ms.transpose(a)).tolist() == di.T.tolist()


def test_contiguous_reference_known_answers():
    """tests/python/test_indexing.py TestContiguous."""
    a = ms.array([[1.0, 2.0], [3.0, 4.0]])
    assert ms.contiguous(a).tolist() == [[1.0, 2.0], [3.0, 4.0]]
    c = ms.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]])
    m = ms.contiguous(ms.transpose(c))
    assert m.shape == (3, 2) and m.tolist() == [[1.0, 4.0], [2.0, 5.0], [3.0, 6.0]]
    assert ms.contiguous(ms.flip(c, 1)).tolist() == [[3.0, 2.0, 1.0], [6.0, 5.0, 4.0]]
    s = ms.array(np.arange(10, dtype=np.float32))[3:7]
    assert ms.contiguous(s).tolist() == [3.0, 4.0, 5.0, 6.0]


@pytest.mark.parametrize("shape", [(300, 517), (1030, 70), (70, 1030), (5, 4099), (4099, 5)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_transposed_casts_every_tile_shape(shape):
    """Casts and unary ops of transposed views go through the LDS tile: 128 rows in 1024 lanes for
    casts (halved until the tile fits, 32 rows for a 1-byte input widened to 8 bytes), 64 rows in
    512 lanes for other functors, 8 or 16 lanes along a short P, 64 x 64 tiles for 16-byte copies.
    Ragged edges on both dims."""
    casts = [(np.uint8, "f64"), (np.int8, "f32"), (np.int16, "i64"), (np.uint32, "f64"), (np.float32, "f64"),
             (np.float64, "f32"), (np.int64, "f32"), (np.float32, "c64"), (np.float64, "c128")]
    for src, dst in casts:
        x = rand(shape, src) if np.dtype(src).kind in "iu" else RNG.standard_normal(shape).astype(src)
        got = ms.astype(ms.transpose(ms.from_numpy(x)), dst)
        assert_bits_equal(got.numpy(), R.cast(x.T, dst), f"{np.dtype(src).name}->{dst} T {shape}", nan_bits=True)
    x = RNG.uniform(-3, 3, shape).astype(np.float32)
    e = ms.exp(ms.transpose(ms.from_numpy(x))).numpy()  # expf: within 2 ulp of the oracle, as in C2's test
    assert e.shape == x.T.shape and ulp_diff_f32(e, R.unary("exp", x.T)).max() <= 2, f"exp T {shape}"
    h = rand(shape, np.float16)
    check(ms.contiguous(ms.transpose(ms.from_numpy(h))), R.contiguous(h.T), f"f16 T {shape}")
    # 16-byte elements take 64 x 64 tiles once P reaches 64, in both tile orders (L > P: (1030, 70))
    for dt in (np.complex64, np.complex128):
        z = rand(shape, dt)
        check(ms.contiguous(ms.transpose(ms.from_numpy(z))), R.contiguous(z.T), f"{np.dtype(dt).name} T {shape}")


def test_contiguous_large_transpose_and_sizes():
    x = RNG.standard_normal((8192, 4096), dtype=np.float32)
    check(ms.contiguous(ms.transpose(ms.from_numpy(x))), R.contiguous(x.T), "f32 (8192,4096)^T")
    for n in (1, 2, 3, 15, 17, 1023, 1025, 65537):
        v = rand((n, 3), np.float64)
        check(ms.contiguous(ms.transpose(ms.from_numpy(v))), R.contiguous(v.T), f"f64 ({n},3)^T")
        check(ms.contiguous(ms.flip(ms.from_numpy(v), 0)), R.contiguous(v[::-1]), f"f64 flip n={n}")


def _abi():
    lib = ctypes.CDLL(LIB)
    for name in ("f32", "f64", "i32", "i64"):
        f = getattr(lib, f"musapy_copy_transpose2d_{name}")
        f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_void_p]
        f.restype = None
        g = getattr(lib, f"musapy_copy_{name}")
        g.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t),
                      ctypes.POINTER(ctypes.c_ssize_t), ctypes.c_void_p]
        g.restype = None
    return lib


@pytest.mark.parametrize("name,dt", [("f32", np.float32), ("f64", np.float64), ("i32", np.int32),
                                     ("i64", np.int64)])
def test_copy_entry_points_through_the_c_abi(name, dt):
    """musapy_copy_transpose2d_<T>(src, dst, rows, cols, stream): src is a C-contiguous (cols, rows)
    array and dst[r*cols + c] = src[c*rows + r] (kernels.rs:327-330); musapy_copy_<T> with
    explicit shape/strides (kernels.rs:321-324)."""
    lib = _abi()
    for rows, cols in ((1, 1), (33, 31), (1000, 37), (4096, 2048)):
        src = rand((cols, rows), dt)
        S = ms.from_numpy(src)
        D = ms.from_numpy(np.zeros((rows, cols), dt))
        ms.synchronize()
        getattr(lib, f"musapy_copy_transpose2d_{name}")(S.data_ptr, D.data_ptr, rows, cols, S.stream_ptr)
        ms.synchronize()
        assert_bits_equal(D.numpy(), np.ascontiguousarray(src.T), f"transpose2d {name} {rows}x{cols}", nan_bits=True)
    x = rand((5, 8, 9), dt)
    X = ms.from_numpy(x)
    D = ms.from_numpy(np.zeros((9, 3, 8), dt))
    shape = (ctypes.c_size_t * 3)(9, 3, 8)
    strides = (ctypes.c_ssize_t * 3)(-1, 2 * 72, 9)  # view x[::2].transpose(2, 0, 1)[::-1]
    base = X.data_ptr + 8 * x.itemsize  # element (0, 0, 8): the reversed axis starts at its end
    ms.synchronize()
    getattr(lib, f"musapy_copy_{name}")(base, D.data_ptr, 3, shape, strides, X.stream_ptr)
    ms.synchronize()
    want = np.ascontiguousarray(x[::2].transpose(2, 0, 1)[::-1])
    assert_bits_equal(D.numpy(), want, f"copy {name} strided", nan_bits=True)


@pytest.mark.parametrize("dt", [np.uint8, np.float16, np.float32, np.float64, np.complex128],
                         ids=lambda d: np.dtype(d).name)
def test_reversed_rows(dt):
    """Flips of the innermost dim (stride -1) read whole vectors and reverse them in registers
    when each row's items line up; ragged and misaligned rows take the element path."""
    for shape in ((1 << 16,), (1000,), (7, 256), (33, 48), (5, 37), (64, 1024)):
        x = rand(shape, dt)
        X = ms.from_numpy(x)
        check(ms.contiguous(ms.flip(X, len(shape) - 1)), R.contiguous(np.flip(x, -1)), f"flip {shape}")
        if len(shape) == 2:  # offset rows: the first item no longer ends on a vector boundary
            v = ms.slice(X, [(0, shape[0], 1), (1, shape[1], 1)])
            check(ms.contiguous(ms.flip(v, 1)), R.contiguous(x[:, 1:][:, ::-1]), f"flip offset {shape}")
    if dt in (np.float32, np.float64):
        a = RNG.standard_normal((64, 1024)).astype(dt)
        b = RNG.standard_normal((64, 1024)).astype(dt)
        A, B = ms.from_numpy(a), ms.from_numpy(b)
        got = ms.sub(ms.flip(A, 1), B).numpy()
        assert_bits_equal(got, R.binary("sub", a[:, ::-1], b), "sub(flip(a), b)")
        got = ms.exp(ms.flip(A, 1)).numpy()
        want = R.unary("exp", a[:, ::-1])
        assert np.array_equal(np.isnan(got), np.isnan(want))
        assert np.all(np.abs(got - want) <= 4 * np.spacing(np.abs(want)))
