"""Seeded random layouts against the CPU oracle, through the public API.

Every case builds its operands as views of random arrays -- permutations, flips, stepped slices,
size-1 (broadcast) dims, empty dims, and long innermost rows that reach the row-piece and tiled
kernels -- identically on the device and in NumPy, then holds the device result to the same bar
as the fixed-layout tests: bit-exact for IEEE add/sub/mul/div, neg/abs, casts, comparisons and
max/argmax; |gpu - cpu| <= tol * sum|x| for sums.  Each case prints its seed-derived index in the
failure message, so a failure names the layout that produced it.
"""
import numpy as np
import pytest

import musapy_amd as ms
from oracle import reference as R
from tests.conftest import assert_bits_equal

pytestmark = pytest.mark.gpu
TOL = {np.float32: 1e-5, np.float64: 1e-12}


def rand_shape(rng, ndim):
    dims = []
    for _ in range(ndim):
        r = rng.random()
        dims.append(0 if r < 0.03 else 1 if r < 0.15 else int(rng.integers(2, 24)))
    if ndim and rng.random() < 0.25:
        dims[-1] = int(rng.integers(500, 1400))  # long rows
    while int(np.prod(dims)) > 400_000:  # keep every case small
        i = int(np.argmax(dims[:-1])) if ndim > 1 else 0
        dims[i] = max(1, dims[i] // 2)
    return tuple(dims)


def rand_data(rng, shape, dt):
    x = rng.uniform(-2, 2, shape)
    if np.dtype(dt).kind == "c":
        x = x + 1j * rng.uniform(-2, 2, shape)
    return x.astype(dt)


def random_view(rng, x, X, max_ops=3):
    """Apply the same 0..max_ops random view operations to a NumPy array and its device copy."""
    for _ in range(int(rng.integers(0, max_ops + 1))):
        op = int(rng.integers(0, 3))
        if op == 0 and x.ndim >= 2:
            perm = [int(p) for p in rng.permutation(x.ndim)]
            x, X = np.transpose(x, perm), ms.permute(X, perm)
        elif op == 1 and x.ndim >= 1:
            ax = int(rng.integers(0, x.ndim))
            x, X = np.flip(x, ax), ms.flip(X, ax)
        elif op == 2 and x.ndim >= 1:
            ranges = []
            for n in x.shape:
                if n <= 1:
                    ranges.append((0, n, 1))
                else:
                    ranges.append((int(rng.integers(0, max(1, n // 3))), n, int(rng.integers(1, 4))))
            x = x[tuple(slice(a, b, c) for a, b, c in ranges)]
            X = ms.slice(X, ranges)
    return x, X


def operand(rng, shape, dt):
    """A device view of exactly `shape` (built through a permuted or flipped base at random),
    and the same values as a contiguous NumPy array."""
    k = int(rng.integers(0, 3))
    if k == 0 or len(shape) < 2:
        base = rand_data(rng, shape, dt)
        x, X = base, ms.from_numpy(base)
        if len(shape) and rng.random() < 0.5:
            ax = int(rng.integers(0, len(shape)))
            base = rand_data(rng, shape, dt)
            x, X = np.flip(base, ax), ms.flip(ms.from_numpy(base), ax)
    else:
        perm = [int(p) for p in rng.permutation(len(shape))]
        inv = [perm.index(i) for i in range(len(shape))]
        base = rand_data(rng, tuple(shape[p] for p in perm), dt)
        x, X = np.transpose(base, inv), ms.permute(ms.from_numpy(base), inv)
    assert x.shape == tuple(shape) and X.shape == tuple(shape)
    return np.ascontiguousarray(x), X


def broadcast_partner(rng, shape):
    s = [1 if (d and rng.random() < 0.3) else d for d in shape]
    drop = int(rng.integers(0, len(s) + 1)) if rng.random() < 0.3 else 0
    return tuple(s[drop:])


@pytest.mark.parametrize("chunk", range(4))
def test_binary_and_compare_random_layouts(chunk):
    rng = np.random.default_rng(1000 + chunk)
    for case in range(120):
        dt = [np.float32, np.float64, np.complex64][int(rng.integers(0, 3)) if case % 4 == 3 else case % 2]
        shape_a = rand_shape(rng, int(rng.integers(1, 5)))
        a, A = operand(rng, shape_a, dt)
        shape_b = broadcast_partner(rng, shape_a)
        b, B = operand(rng, shape_b, dt)
        if rng.random() < 0.5:
            a, A, b, B = b, B, a, A
        what = f"chunk {chunk} case {case}: {np.dtype(dt).name} {a.shape} . {b.shape}"
        ops = ("add", "sub", "mul", "div") if np.dtype(dt).kind != "c" else ("add", "mul")
        op = ops[case % len(ops)]
        got = getattr(ms, op)(A, B).numpy()
        assert_bits_equal(got, R.binary(op, a, b), f"{op} {what}")
        if np.dtype(dt).kind != "c":
            cop = ("lt", "ge", "eq", "ne")[case % 4]
            assert_bits_equal(getattr(ms, cop)(A, B).numpy(), R.compare(cop, a, b), f"{cop} {what}")


@pytest.mark.parametrize("chunk", range(3))
def test_unary_and_cast_random_views(chunk):
    rng = np.random.default_rng(2000 + chunk)
    for case in range(120):
        dt = (np.float32, np.float64)[case % 2]
        base = rand_data(rng, rand_shape(rng, int(rng.integers(1, 5))), dt)
        x, X = random_view(rng, base, ms.from_numpy(base))
        x = np.ascontiguousarray(x)
        what = f"chunk {chunk} case {case}: {np.dtype(dt).name} {x.shape}"
        op = ("neg", "abs", "sign")[case % 3]
        assert_bits_equal(getattr(ms, op)(X).numpy(), R.unary(op, x), f"{op} {what}", nan_bits=True)
        dst = "f64" if dt == np.float32 else "f32"
        assert_bits_equal(ms.astype(X, dst).numpy(), R.cast(x, dst), f"astype {dst} {what}", nan_bits=True)
        assert_bits_equal(ms.contiguous(X).numpy(), x, f"contiguous {what}", nan_bits=True)


@pytest.mark.parametrize("chunk", range(3))
def test_reductions_random_views(chunk):
    rng = np.random.default_rng(3000 + chunk)
    for case in range(100):
        dt = (np.float32, np.float64)[case % 2]
        shape = tuple(d if d else 3 for d in rand_shape(rng, int(rng.integers(1, 4))))  # no empty axes
        base = rand_data(rng, shape, dt)
        x, X = random_view(rng, base, ms.from_numpy(base))
        x = np.ascontiguousarray(x)
        if x.size == 0:
            continue
        r = rng.random()
        if r < 0.25 or x.ndim == 1:
            axis = None if r < 0.1 else int(rng.integers(-x.ndim, x.ndim))
        else:
            k = int(rng.integers(1, x.ndim + 1))
            axis = tuple(int(v) for v in rng.choice(x.ndim, size=k, replace=False))
        keep = bool(rng.random() < 0.3)
        what = f"chunk {chunk} case {case}: {np.dtype(dt).name} {x.shape} axis={axis} keepdims={keep}"
        for kind in ("max", "argmax", "min"):
            got = getattr(ms, kind)(X, axis=axis, keepdims=keep).numpy()
            assert_bits_equal(got, R.reduce(x, kind, axis, keep), f"{kind} {what}")
        got = ms.sum(X, axis=axis, keepdims=keep).numpy()
        want = R.reduce(x, "sum", axis, keep)
        ax = axis if axis is None or isinstance(axis, tuple) else (axis,)
        scale = np.sum(np.abs(x.astype(np.float64)), axis=ax, keepdims=keep)
        assert got.shape == want.shape, what
        assert np.all(np.abs(got.astype(np.float64) - want) <= TOL[dt] * scale + 1e-30), f"sum {what}"


def rand_mixed(rng, shape, dt):
    if np.dtype(dt).kind == "i":
        return rng.integers(-1000, 1001, shape).astype(dt)
    return rand_data(rng, shape, dt)


@pytest.mark.parametrize("chunk", range(2))
def test_mixed_dtype_random_layouts(chunk):
    """Operands of different dtypes (promotion fused into the op, or cast first) in random views."""
    rng = np.random.default_rng(4000 + chunk)
    pairs = [(np.int64, np.float64), (np.int64, np.float32), (np.int32, np.float64), (np.float32, np.float64),
             (np.int32, np.float32), (np.float32, np.complex64), (np.float64, np.complex64)]
    for case in range(100):
        ta, tb = pairs[case % len(pairs)]
        if rng.random() < 0.5:
            ta, tb = tb, ta
        shape_a = rand_shape(rng, int(rng.integers(1, 4)))
        base = rand_mixed(rng, shape_a, ta)
        a, A = random_view(rng, base, ms.from_numpy(base), max_ops=2)
        a = np.ascontiguousarray(a)
        shape_b = broadcast_partner(rng, a.shape)
        b = rand_mixed(rng, shape_b, tb)
        B = ms.from_numpy(b)
        op = ("add", "sub", "mul")[case % 3]
        what = f"chunk {chunk} case {case}: {np.dtype(ta).name}{a.shape} {op} {np.dtype(tb).name}{b.shape}"
        assert_bits_equal(getattr(ms, op)(A, B).numpy(), R.binary(op, a, b), what)


@pytest.mark.parametrize("chunk", range(2))
def test_cumsum_random_views(chunk):
    """cumsum over a random axis (or flattened) of random views: f32/f64 to the sum bound, i64 exact."""
    rng = np.random.default_rng(5000 + chunk)
    for case in range(60):
        dt = (np.float32, np.float64, np.int64)[case % 3]
        shape = tuple(d if d else 2 for d in rand_shape(rng, int(rng.integers(1, 4))))
        base = rand_mixed(rng, shape, dt)
        x, X = random_view(rng, base, ms.from_numpy(base))
        x = np.ascontiguousarray(x)
        axis = None if rng.random() < 0.2 else int(rng.integers(-x.ndim, x.ndim))
        what = f"chunk {chunk} case {case}: {np.dtype(dt).name} {x.shape} axis={axis}"
        got = ms.cumsum(X, axis=axis).numpy()
        want = R.cumsum(x, axis=axis)
        assert got.shape == want.shape and got.dtype == want.dtype, what
        if dt == np.int64:
            assert np.array_equal(got, want), what
            continue
        # each prefix is a sum: bound it by tol * (running sum of |x|) along the same axis
        ax = 0 if axis is None else axis
        xa = np.abs(x.reshape(-1) if axis is None else x).astype(np.float64)
        scale = np.cumsum(xa, axis=ax)
        assert np.all(np.abs(got.astype(np.float64) - want) <= TOL[dt] * scale + 1e-30), what
