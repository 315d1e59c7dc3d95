"""GPU parity of reductions and cumsum against the CPU oracle.

max/min/argmax/argmin and every int64 result are bit-exact (ties -> lowest index, a NaN at
position 0 absorbs, later NaNs are skipped -- op_builder.rs:3543-3578).  Floating sums and means
use the condition-aware bound of BASELINE.json: |gpu - cpu| <= tol * sum|x| over the reduced
elements, tol = 1e-5 (f32) / 1e-12 (f64); the sequential CPU sum itself is that far from the
exact sum, so an elementwise relative bound would reject every correct parallel order.
"""
import numpy as np
import pytest

import musapy_amd as ms
from oracle import reference as R
from tests.conftest import assert_bits_equal

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(77)
TOL = {np.float32: 1e-5, np.float64: 1e-12, np.complex64: 1e-5, np.complex128: 1e-12}


def dev(x):
    return ms.from_numpy(np.ascontiguousarray(x))


def abs_sum(x, axis, keepdims):
    ax = axis if axis is None or isinstance(axis, tuple) else (axis,)
    return np.sum(np.abs(x.astype(np.complex128 if np.iscomplexobj(x) else np.float64)), axis=ax, keepdims=keepdims)


def check_reduce(kind, x, axis=None, keepdims=False, gpu_x=None):
    gx = dev(x) if gpu_x is None else gpu_x
    got = getattr(ms, kind)(gx, axis=axis, keepdims=keepdims).numpy()
    want = R.reduce(x, kind, axis, keepdims)
    what = f"{kind} {x.dtype} {x.shape} axis={axis} keepdims={keepdims}"
    if kind in ("max", "min", "argmax", "argmin") or want.dtype == np.int64:
        assert_bits_equal(got, want, what)
        return
    assert got.shape == want.shape and got.dtype == want.dtype, what
    tol = TOL[want.dtype.type]
    if kind == "prod":
        # products have no bound in BASELINE.json; compare relatively, allowing sqrt(n) roundings
        n = x.size // max(want.size, 1)
        eps = 1.2e-7 if want.dtype in (np.float32, np.complex64) else 2.3e-16
        err = np.abs(got.astype(np.complex128) - want) / np.maximum(np.abs(want), 1e-300)
        assert np.all(err <= 20 * eps * np.sqrt(n) + 4 * eps), f"{what}: max rel err {err.max()}"
        return
    scale = abs_sum(x, axis, keepdims)
    if kind == "mean":
        n = x.size // max(want.size, 1)
        scale = scale / max(n, 1)
    err = np.abs(got.astype(np.complex128) - want.astype(np.complex128))
    assert np.all(err <= tol * scale + 1e-30), f"{what}: max err {err.max()} vs bound {tol * scale.max()}"


SHAPES_AXES = [
    ((257,), [None, 0]),
    ((4, 1000), [0, 1, None, -1]),
    ((1000, 4), [0, 1]),
    ((33, 65, 7), [0, 1, 2, None]),
    ((5000, 3), [0, 1]),
    ((3, 1, 4096), [2, 1, 0]),
    ((2, 300000), [1]),
]


@pytest.mark.parametrize("kind", ["sum", "prod", "max", "min", "mean", "argmax", "argmin"])
@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int64])
def test_reduce_shapes(kind, dt):
    for shape, axes in SHAPES_AXES:
        if dt == np.int64:
            x = RNG.integers(-1000, 1000, shape).astype(np.int64)
        elif kind == "prod":
            # keep the product O(1): a product that underflows compares the CPU's stuck denormal
            # with a tree's exact zero, which says nothing about either
            x = RNG.uniform(0.999, 1.001, shape).astype(dt)
        else:
            x = RNG.standard_normal(shape).astype(dt)
        for ax in axes:
            check_reduce(kind, x, ax)
        check_reduce(kind, x, axes[0], keepdims=True)


@pytest.mark.parametrize("kind", ["max", "min", "argmax", "argmin"])
def test_ordered_semantics_planted(kind):
    # ties, +-0 and NaN at k=0 / later, spread over tiles of the parallel paths
    for shape, axis in (((64, 3000), 1), ((3000, 64), 0), ((1, 1 << 20), 1), ((16, 37), 1)):
        x = RNG.integers(-2, 3, shape).astype(np.float32)
        flat_axis_len = shape[axis]
        idx = [slice(None)] * 2
        idx[axis] = 0
        x[tuple(idx)][::5] = np.nan           # NaN at k = 0 in every 5th output
        idx[axis] = flat_axis_len // 2
        x[tuple(idx)][1::3] = np.nan          # a later NaN
        x[tuple(idx)][2::7] = -0.0
        check_reduce(kind, x, axis)
        check_reduce(kind, x.astype(np.float64), axis)
    z = np.zeros((8, 5000), np.float32)
    z[:, ::2] = -0.0
    check_reduce(kind, z, 1)
    check_reduce(kind, z.T.copy(), 0)


@pytest.mark.parametrize("kind", ["max", "min", "argmax", "argmin"])
@pytest.mark.parametrize("n", [300, 8192, 20000])
def test_f32_row_combine_edge_values(kind, n):
    """Unit-stride f32 rows, whose lanes combine (value, index) through one packed 64-bit key per
    step: infinities, all-NaN rows, subnormals, +-0 ties in both orders and ties spread over lanes
    and waves, each row also negated (min sees the mirror case)."""
    rows = np.empty((12, n), np.float32)
    rows[0] = -np.inf                                        # every element -inf
    rows[1] = np.nan
    rows[1, n - 1] = -np.inf                                 # one element, the last
    rows[2] = -1.0
    rows[2, 100], rows[2, n // 2] = -0.0, 0.0                # -0 first, then +0
    rows[3] = -1.0
    rows[3, 100], rows[3, n // 2] = 0.0, -0.0                # +0 first, then -0
    rows[4] = np.where(RNG.random(n) < 0.5, -0.0, 0.0)
    rows[4, 7] = -0.0
    rows[5] = RNG.uniform(-1, 1, n)
    rows[5, [n - 5, 200, n // 3]] = 3.0                      # ties in different lanes and waves
    rows[6] = -0.0
    rows[6, 50] = np.float32(1e-45)                          # the smallest subnormal
    rows[6, n - 50] = np.float32(-1e-45)
    rows[7] = RNG.uniform(-1, 1, n)
    rows[7, [n - 1, n - 100]] = np.inf
    rows[8] = RNG.uniform(-1, 1, n)
    rows[8, 0] = np.nan                                      # NaN at position 0 absorbs
    rows[9] = np.nan                                         # all NaN
    rows[10] = RNG.standard_normal(n)
    rows[10, ::3] = np.nan
    rows[11] = np.float32(2.5)                               # one value everywhere: index 0
    check_reduce(kind, rows, 1)
    check_reduce(kind, -rows, 1)


@pytest.mark.parametrize("kind", ["max", "min"])
@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int64])
def test_two_axis_max_min_semantics(kind, dt):
    """max/min over (0, 1) of a 2-D array run as the axis-0 partial plus one fused final (or, when
    the axis-0 pass is not split, as two passes); either way the result is the reference's
    axis-0-then-axis-1 one: a NaN heading column 0 absorbs everything, a NaN heading another
    column drops that column from the second pass, later NaNs are skipped, +-0 ties keep the first."""
    for shape in ((3000, 64), (64, 3000), (4096, 1000), (70000, 3)):
        if dt == np.int64:
            check_reduce(kind, RNG.integers(-5, 6, shape).astype(np.int64), (0, 1))
            continue
        x = RNG.integers(-2, 3, shape).astype(dt)
        x[0, 1] = np.nan          # drops column 1 from the second pass
        x[7, ::3] = np.nan        # later NaNs are skipped
        x[:, 2] = -0.0
        check_reduce(kind, x, (0, 1))
        y = x.copy()
        y[0, 0] = np.nan          # absorbs everything
        check_reduce(kind, y, (0, 1))
        z = np.full(shape, np.nan, dt)
        z[0, 1], z[5, 1], z[9, 2] = 1.0, 3.0, 7.0  # column 2's head is NaN: its 7.0 is dropped
        check_reduce(kind, z, (0, 1))
        w = np.zeros(shape, dt)
        w[:, ::2] = -0.0          # the first column's zero decides the bits
        check_reduce(kind, w, (0, 1))
        check_reduce(kind, np.ascontiguousarray(w[:, ::-1]), (0, 1))


@pytest.mark.parametrize("kind", ["sum", "max", "argmax", "mean"])
def test_reduce_views(kind):
    base = RNG.standard_normal((64, 96)).astype(np.float32)
    B = dev(base)
    for nv, dv in ((lambda x: x[:, ::-1], lambda a: ms.flip(a, 1)),
                   (lambda x: x.T, lambda a: ms.transpose(a)),
                   (lambda x: x[3:60:2, 5:90], lambda a: ms.slice(a, [(3, 60, 2), (5, 90, 1)]))):
        for ax in (0, 1, None):
            check_reduce(kind, np.ascontiguousarray(nv(base)), ax, gpu_x=dv(B))


@pytest.mark.parametrize("kind", ["sum", "mean", "prod", "max", "min", "argmax", "argmin"])
def test_multi_axis(kind):
    x = RNG.standard_normal((6, 7, 8)).astype(np.float32)
    if kind == "prod":
        x = RNG.uniform(0.9, 1.1, (6, 7, 8)).astype(np.float32)
    for axes in ((0, 1), (1, 2), (0, 2), (0, 1, 2), (-1, 0)):
        for keep in (False, True):
            check_reduce(kind, x, axes, keep)


@pytest.mark.parametrize("kind", ["sum", "mean", "prod"])
@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int64])
def test_multi_axis_merged(kind, dt):
    """Adjacent reduced axes that are stride-contiguous are reduced in one pass; the result
    must stay within the bound of the reference's axis-by-axis order."""
    shape = (24, 96, 130)
    if kind == "prod":
        x = RNG.uniform(0.999, 1.001, shape) if dt != np.int64 else RNG.integers(-1, 2, shape)
    else:
        x = RNG.standard_normal(shape) * 100 if dt != np.int64 else RNG.integers(-(2**40), 2**40, shape)
    x = x.astype(dt)
    if kind == "mean" and dt == np.int64:
        x = x.astype(np.float64)
    for axes in ((1, 2), (0, 1), (0, 1, 2), (-2, -1)):
        for keep in (False, True):
            check_reduce(kind, x, axes, keep)
    # a permuted view: reduced axes no longer stride-contiguous, reduced one at a time
    xt = np.ascontiguousarray(np.transpose(x, (2, 0, 1)))
    gx = ms.permute(dev(x), (2, 0, 1))
    for axes in ((0, 1), (1, 2)):
        check_reduce(kind, xt, axes, gpu_x=gx)


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int64])
def test_single_launch_tiled_reductions(dt):
    """Reductions large enough to be split into tiles (> 256 KB with few outputs) run as one
    launch that hands tile results over through the stream's workspace; the workspace must be
    left clean, so the cases run back to back with changing shapes and repeats."""
    n = 3_000_001
    if dt == np.int64:
        x = RNG.integers(-(2**40), 2**40, n).astype(np.int64)
    else:
        x = RNG.standard_normal(n).astype(dt)
    X = dev(x)
    for kind in ("sum", "max", "min", "argmax", "argmin", "mean", "sum"):
        if kind == "mean" and dt == np.int64:
            continue
        check_reduce(kind, x, None, gpu_x=X)
    m = x[: 7 * 400_000].reshape(7, 400_000)  # few outputs, several tiles each
    M = dev(m)
    for kind in ("argmax", "sum", "min", "argmin"):
        check_reduce(kind, m, 1, gpu_x=M)
        check_reduce(kind, m, 1, gpu_x=M)
    if dt != np.int64:
        # NaN at position 0 absorbs; a NaN elsewhere is skipped; ties go to the lowest index
        y = x.copy()
        y[0] = np.nan
        for kind in ("max", "argmax", "min", "argmin"):
            check_reduce(kind, y, None)
        z = x.copy()
        z[1_234_567] = np.nan
        z[2_500_000] = z[2_900_000] = np.abs(z).max() + 1
        for kind in ("max", "argmax"):
            check_reduce(kind, z, None)
    t = np.zeros(2_000_000, dt)
    t[[5, 1_999_999]] = 3
    for kind in ("argmax", "argmin"):
        check_reduce(kind, t, None)
    if dt != np.int64:
        # blocks whose whole share is NaN publish "no element"; an all-NaN array keeps index 0
        u = np.full(2_000_003, np.nan, dt)
        u[1_777_777] = -5.0
        for kind in ("max", "argmax", "min", "argmin"):
            check_reduce(kind, u, None)
            check_reduce(kind, np.full(2_000_003, np.nan, dt), None)
        v = np.full(2_000_003, -np.inf, dt)
        v[[3, 1_500_000]] = -1e30
        for kind in ("max", "argmax", "min", "argmin"):
            check_reduce(kind, v, None)


@pytest.mark.parametrize("dt", [np.complex64, np.complex128])
def test_complex_reductions(dt):
    for shape, axes in (((3, 4), [None, 0, 1, (0, 1), -1]), ((16, 64, 64), [(1, 2), 0, 2]), ((4, 200000), [1])):
        z = (RNG.standard_normal(shape) + 1j * RNG.standard_normal(shape)).astype(dt)
        for ax in axes:
            check_reduce("sum", z, ax)
            check_reduce("mean", z, ax)
        zp = (np.exp(1j * RNG.uniform(-0.1, 0.1, shape[-1:]))).astype(dt)
        check_reduce("prod", zp, None)
    with pytest.raises(ms.DtypeError):
        ms.max(dev(np.array([1 + 2j], np.complex128)))


@pytest.mark.parametrize("dt", [np.complex64, np.complex128])
def test_single_launch_complex_reductions(dt):
    """Complex sum/mean/prod split into tiles also run as one launch (four workspace words per
    slot); back-to-back calls check that the workspace is left clean."""
    z = (RNG.standard_normal((5, 400_000)) + 1j * RNG.standard_normal((5, 400_000))).astype(dt)
    Z = dev(z)
    for kind in ("sum", "mean", "sum"):
        check_reduce(kind, z, 1, gpu_x=Z)
        check_reduce(kind, z, None, gpu_x=Z)
    zp = np.exp(1j * RNG.uniform(-1e-3, 1e-3, (3, 300_000))).astype(dt)
    check_reduce("prod", zp, 1)
    check_reduce("prod", np.ascontiguousarray(zp[0]), None)


def test_reduce_errors_and_edges():
    x = dev(np.ones((2, 3), np.float32))
    with pytest.raises(ms.ShapeError):
        ms.sum(x, axis=5)
    with pytest.raises(ms.ShapeError):
        ms.sum(x, axis=(0, 0))
    with pytest.raises(ms.ShapeError):
        ms.sum(x, axis=(0, 1), out=dev(np.zeros(2, np.float32)))
    with pytest.raises(Exception):
        ms.sum(x, axis=0, out=dev(np.zeros(2, np.int64)))
    r = ms.sum(dev(np.array([5.0], np.float32)))
    assert r.shape == () and r.item() == 5.0
    assert ms.sum(dev(np.array([1, 2, 3], np.int8))).dtype == "i64"
    e = ms.sum(dev(np.zeros((3, 0), np.float32)), axis=1)
    assert e.numpy().tolist() == [0.0, 0.0, 0.0]
    with pytest.raises(ms.ShapeError):
        ms.max(dev(np.zeros((3, 0), np.float32)), axis=1)
    out = dev(np.zeros(3, np.float32))
    ms.sum(dev(np.ones((3, 4), np.float32)), axis=1, out=out)
    assert out.tolist() == [4.0, 4.0, 4.0]


# ---------------------------------------------------------------------------------------------
# cumsum
@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int64])
def test_cumsum_shapes(dt):
    cases = [((1300,), 0), ((1537,), 0), ((3, 70000), 1), ((65536,), 0), ((65537,), 0), ((5, 7), 1),
             ((64, 4097), 1), ((2000, 3), 0), ((7, 300, 5), 1), ((4, 12288), 1)]
    for shape, ax in cases:
        x = RNG.integers(-50, 50, shape).astype(dt) if dt == np.int64 else RNG.random(shape).astype(dt)
        got = ms.cumsum(dev(x), axis=ax).numpy()
        want = R.cumsum(x, ax)
        if dt == np.int64:
            assert_bits_equal(got, want, f"cumsum {shape}")
        else:
            scale = np.cumsum(np.abs(x.astype(np.float64)), axis=ax)
            assert np.all(np.abs(got - want) <= TOL[dt] * scale), f"cumsum {dt} {shape} axis {ax}"


def test_cumsum_reference_cases():
    # tests/python/test_reduction.py:337-423 (cumsum of ones, capacity limit)
    for n in (65536, 65537, 1_000_000):
        r = ms.cumsum(ms.ones(n, dtype="i64"), axis=0)
        assert ms.sum(r).item() == n * (n + 1) // 2
        v = r.numpy()
        assert v[-1] == n and v[min(65535, n - 1)] == min(65536, n)
    x = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    assert ms.cumsum(dev(x)).tolist() == [1.0, 3.0, 6.0, 10.0]
    assert ms.cumsum(dev(x), axis=0).tolist() == [[1.0, 2.0], [4.0, 6.0]]
    assert ms.cumsum(dev(np.array([1, 2, 3], np.int64)), axis=0).dtype == "i64"
    with pytest.raises(ms.ShapeError):
        ms.cumsum(ms.ones(256**3 + 1, dtype="f32"), axis=0)


def test_cumsum_views_and_exact_orders():
    base = RNG.random((300, 200)).astype(np.float64)
    B = dev(base)
    # column and strided scans add in the CPU's order: bit-exact
    assert_bits_equal(ms.cumsum(B, axis=0).numpy(), R.cumsum(base, 0), "column scan")
    assert_bits_equal(ms.cumsum(ms.transpose(B), axis=1).numpy(), R.cumsum(base.T, 1), "transposed scan")
    flat = ms.cumsum(ms.transpose(B)).numpy()
    want = R.cumsum(base.T, None)
    assert np.all(np.abs(flat - want) <= 1e-12 * np.cumsum(np.abs(base.T.reshape(-1))))


def test_cumsum_deterministic():
    x = RNG.random((8, 1 << 18)).astype(np.float32)
    X = dev(x)
    a = ms.cumsum(X, axis=1).numpy()
    for _ in range(3):
        assert_bits_equal(ms.cumsum(X, axis=1).numpy(), a, "cumsum run-to-run")
    s = ms.sum(X, axis=1).numpy()
    for _ in range(3):
        assert_bits_equal(ms.sum(X, axis=1).numpy(), s, "sum run-to-run")
    # many rows: the chained scan (tile-major over the rows, each tile waits for its predecessor)
    y = RNG.random((600, 40000))
    Y = dev(y)
    b = ms.cumsum(Y, axis=1).numpy()
    for _ in range(2):
        assert_bits_equal(ms.cumsum(Y, axis=1).numpy(), b, "chained cumsum run-to-run")
    want = R.cumsum(y[:4], 1)
    assert np.all(np.abs(b[:4] - want) <= 1e-12 * np.abs(want))


@pytest.mark.parametrize("kind", ["sum", "prod", "max", "min", "mean", "argmax", "argmin"])
@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int64])
def test_column_reductions_split_into_row_tiles(kind, dt):
    """Column reductions split into 8-64 row tiles (partial + final): ragged column groups,
    unaligned rows, outer dims, NaN in row 0 and later rows, and argmax ties."""
    cases = [((1024, 4096), 0), ((2048, 4096), 0), ((3, 512, 1000), 1), ((640, 2056), 0), ((4096, 260), 0)]
    for shape, ax in cases:
        if dt == np.int64:
            x = RNG.integers(-50, 50, shape).astype(np.int64)
        elif kind == "prod":
            x = RNG.uniform(0.999, 1.001, shape).astype(dt)
        else:
            x = RNG.standard_normal(shape).astype(dt)
            if kind in ("max", "min", "argmax", "argmin"):
                x = np.round(x * 4) / 4  # plenty of ties
                flat = np.moveaxis(x, ax, 0)
                flat[0, ::7] = np.nan   # NaN at axis position 0 absorbs those columns
                flat[3, 1::5] = np.nan  # later NaNs are skipped
        check_reduce(kind, x, ax)


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int64, np.complex64, np.complex128])
def test_single_launch_column_reductions(dt):
    """Column sums, means and products in one launch (the last block of each column group folds
    the group's tiles): ragged column groups, outer dims, back-to-back calls on one workspace, and
    the same bits run to run."""
    cases = [((4096, 2048), 0), ((2000, 1030), 0), ((6, 1500, 300), 1), ((8192, 70), 0)]
    for shape, ax in cases:
        if dt == np.int64:
            x = RNG.integers(-1000, 1000, shape).astype(np.int64)
        elif np.dtype(dt).kind == "c":
            x = (RNG.standard_normal(shape) + 1j * RNG.standard_normal(shape)).astype(dt)
        else:
            x = RNG.standard_normal(shape).astype(dt)
        X = dev(x)
        kinds = ("sum", "mean") if dt != np.int64 else ("sum",)
        for kind in kinds:
            first = getattr(ms, kind)(X, axis=ax).numpy()
            check_reduce(kind, x, ax, gpu_x=X)
            assert_bits_equal(getattr(ms, kind)(X, axis=ax).numpy(), first, f"{kind} {dt.__name__} {shape} rerun")
    xp = RNG.uniform(0.999, 1.001, (3000, 520)).astype(np.float64 if dt == np.int64 else dt)
    check_reduce("prod", xp, 0)


def test_cumsum_look_back_long_rows():
    """Few long rows take the decoupled look-back over tiles claimed in memory order: a row of
    2^24 f64 is 4096 tiles, so most tiles find their predecessor's prefix beyond the 64-tile window
    and wait for it to move; int64 is exact, floats within the prefix bound of the oracle and the
    same bits on every run."""
    for shape, dt in (((1, 1 << 24), np.float64), ((3, 5_000_001), np.int64), ((7, 300_001), np.float32),
                      ((64, 65536), np.float64), ((2, 4097), np.float64), ((5, 8193), np.float32)):
        x = RNG.integers(-1000, 1000, shape) if dt == np.int64 else RNG.random(shape)
        x = x.astype(dt)
        X = dev(x)
        got = ms.cumsum(X, axis=1).numpy()
        want = R.cumsum(x, 1)
        what = f"look-back cumsum {np.dtype(dt).name} {shape}"
        if dt == np.int64:
            assert_bits_equal(got, want, what)
        else:
            exact = np.cumsum(x.astype(np.float64), axis=1)
            bound = TOL[dt] * np.cumsum(np.abs(x.astype(np.float64)), axis=1)
            if dt == np.float32:  # the sequential f32 reference drifts past the bound on long rows
                bound = bound + np.abs(want - exact)
            assert np.all(np.abs(got.astype(np.float64) - want) <= bound), what
        assert_bits_equal(ms.cumsum(X, axis=1).numpy(), got, what + " run-to-run")


@pytest.mark.parametrize("kind", ["max", "min"])
@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int64])
def test_two_axis_single_launch(kind, dt):
    """max/min over (0, 1) of a C-contiguous matrix run as one launch (musapy_reduce_2d_ordered_v1)
    that must give the per-axis passes' bits: the first extreme in COLUMN-major order.  A zero of
    one sign that comes first row-major and of the other sign first column-major tells the two
    orders apart; rows span several blocks of the persistent grid; keepdims keeps (1, 1).  f32 rows of
    2048 or more elements (a multiple of 4) take the row-keyed kernel: odd row counts, rows of
    several block rounds with a ragged end, and row 0 with and without NaN heads (the refold)."""
    sign = 1 if kind == "max" else -1
    for shape in ((8192, 8192), (3000, 2048), (2500, 4096), (5, 8), (1, 12), (1500, 8188), (2501, 4096),
                  (300, 20000), (7, 2052)):
        if dt == np.int64:
            x = RNG.integers(-10**6, 10**6, shape).astype(np.int64)
        else:
            x = RNG.standard_normal(shape).astype(dt)
        check_reduce(kind, x, (0, 1))
        check_reduce(kind, x, (0, 1), keepdims=True)
        if dt == np.int64:
            continue
        z = np.full(shape, -sign, dt)
        z[0, shape[1] - 1] = -0.0          # first extreme in row-major order
        z[shape[0] - 1, 0 if shape[1] == 1 else 1] = 0.0  # first in column-major order: its bits win
        check_reduce(kind, z, (0, 1))
        y = x.copy()
        y[0, 3] = np.nan                   # drops column 3, whatever it holds below
        y[shape[0] - 1, 3] = sign * 1e30
        y[shape[0] // 2, 5] = np.nan       # skipped
        check_reduce(kind, y, (0, 1))
        y[0, 0] = np.nan                   # absorbs everything
        check_reduce(kind, y, (0, 1))


@pytest.mark.parametrize("kind", ["max", "min"])
def test_two_axis_chunked_rows(kind):
    """f32 rows of whole 8192-element chunks take the chunked two-axis kernel (one round of up to
    1024 blocks, chunk c = row c / chunks-per-row): grids smaller than the chunk count and larger,
    several chunks per row, row 0's NaN in a later chunk (its block masks every block's refold),
    ties across rows and columns resolved in column-major order, infinities, a column of NaNs
    below row 0."""
    sign = 1 if kind == "max" else -1
    for shape in ((1, 8192), (3, 8192), (100, 16384), (2049, 8192), (64, 32768), (1031, 16384)):
        R, C = shape
        x = RNG.standard_normal(shape).astype(np.float32)
        check_reduce(kind, x, (0, 1))
        t = x.copy()                       # the extreme twice: column-major order picks the left one
        t[R - 1, 7] = sign * 50.0
        t[0, 8] = sign * 50.0
        check_reduce(kind, t, (0, 1))
        if R > 1:
            t[R // 2, 7] = sign * 50.0     # same column, earlier row
            check_reduce(kind, t, (0, 1))
        y = x.copy()
        y[0, C - 3] = np.nan               # row 0's NaN in its last chunk drops column C - 3 ...
        y[R - 1, C - 3] = sign * np.inf    # ... and the infinity below it
        y[R // 2, 1:9] = np.nan            # skipped
        check_reduce(kind, y, (0, 1))
        y[R - 1, 2] = sign * np.inf        # an eligible infinity wins
        check_reduce(kind, y, (0, 1))
        z = np.full(shape, -sign, np.float32)
        z[0, C - 1] = -0.0
        z[R - 1, 1] = 0.0
        check_reduce(kind, z, (0, 1))


@pytest.mark.parametrize("m", [3, 4, 5])
def test_whole_array_chunk_walk(m):
    """Whole-array f32 reductions whose 1024 streaming blocks take m or m + 1 chunks of 8192
    elements each (the chunk walker's steady loop and both of its tails), with and without whole
    chunks left over and a partial last chunk: sums within the bound, exact arg results, with
    the extreme planted in the partial chunk and tied in an earlier block; and max / min over
    both axes of m * 1024 + 5 rows of one chunk (the chunked two-axis kernel)."""
    chunk, grid = 8192, 1024
    for extra in (0, 517 * chunk + 1234, (grid - 1) * chunk + 8191):
        n = m * grid * chunk + extra
        x = RNG.standard_normal(n).astype(np.float32)
        gx = dev(x)
        for kind in ("sum", "argmax", "min"):
            check_reduce(kind, x, None, gpu_x=gx)
        y = x.copy()
        y[n - 1] = 40.0                        # the partial chunk (or the last block's last chunk)
        y[(m - 1) * grid * chunk + 3 * chunk + 5] = 40.0  # a tie in block 3's m-th chunk: the lower index wins
        check_reduce("argmax", y, None)
        check_reduce("max", y, None)
    # the chunked two-axis kernel walks its chunks the same way: m * 1024 + 5 rows of one chunk
    x2 = RNG.standard_normal((m * grid + 5, chunk)).astype(np.float32)
    x2[m * grid + 4, 17] = 40.0  # in the last row: a block with m + 1 chunks
    for kind in ("max", "min"):
        check_reduce(kind, x2, (0, 1))


@pytest.mark.parametrize("kind", ["max", "min", "argmax", "argmin"])
def test_whole_array_signed_zero_ties(kind):
    """Whole-array f32 reductions of 3M+ elements (the persistent grid with its packed-key wave
    combine, in the streaming blocks and in the combiner): when the extreme is a zero, the first
    zero decides the index and the sign, whether -0 or +0 comes first, with the first zero in a
    late block."""
    n = 3_000_000 + 77
    fill = np.float32(-1.0 if kind in ("max", "argmax") else 1.0)
    for first, second in ((-0.0, 0.0), (0.0, -0.0)):
        x = np.full(n, fill, np.float32)
        x[2_500_001], x[2_900_000] = first, second
        check_reduce(kind, x, None)
        x[1_000_003] = second  # now the first zero sits in an earlier block
        check_reduce(kind, x, None)
    x = np.full(n, fill, np.float32)
    idx = RNG.choice(np.arange(1_000_000, n), 5000, replace=False)
    x[idx] = np.where(RNG.random(5000) < 0.5, -0.0, 0.0).astype(np.float32)
    check_reduce(kind, x, None)


def test_cumsum_chained_rows():
    """Many rows of several tiles take the chained scan, in 64 KB tiles (rows of at least two) or
    16 KB tiles: row counts that are not a multiple of 8 (the grid pads the row pitch to one),
    ragged last tiles, rows that are not 16-byte aligned (a sliced view), int64 exact, floats
    within the prefix bound of the oracle, and the same bits on every run."""
    cases = [((515, 70001), np.float64), ((777, 20000), np.int64), ((513, 33333), np.float32),
             ((600, 4097), np.float64), ((1030, 8192), np.float32)]
    for shape, dt in cases:
        x = RNG.integers(-1000, 1000, shape) if dt == np.int64 else RNG.random(shape)
        x = x.astype(dt)
        X = dev(x)
        got = ms.cumsum(X, axis=1).numpy()
        want = R.cumsum(x, 1)
        what = f"chained cumsum {np.dtype(dt).name} {shape}"
        if dt == np.int64:
            assert_bits_equal(got, want, what)
        else:
            exact = np.cumsum(x.astype(np.float64), axis=1)
            bound = TOL[dt] * np.cumsum(np.abs(x.astype(np.float64)), axis=1) + np.abs(want - exact)
            assert np.all(np.abs(got - want) <= bound), what
        assert_bits_equal(ms.cumsum(X, axis=1).numpy(), got, what + " run-to-run")
    # views whose rows start 8 bytes past 16-byte alignment: the element-wise load path, in 16 KB
    # tiles (rows shorter than two 64 KB tiles) and in 64 KB tiles
    for cols in (9001, 20001):
        base = RNG.random((520, cols))
        V = ms.slice(dev(base), [(0, 520, 1), (1, cols, 1)])
        got = ms.cumsum(V, axis=1).numpy()
        want = R.cumsum(base[:, 1:], 1)
        assert np.all(np.abs(got - want) <= 1e-12 * np.cumsum(np.abs(base[:, 1:]), axis=1)), f"unaligned rows {cols}"
