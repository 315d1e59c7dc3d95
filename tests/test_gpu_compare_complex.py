"""GPU parity of comparisons and complex elementwise ops against the CPU oracle (bit-exact).

Comparisons: eq/ne/lt/gt/le/ge over f32/f64 (0/1 bytes, bool dtype) and complex eq/ne, on every
layout the binary kernels specialise (contiguous with aligned and misaligned starts, transposed,
flipped, sliced, broadcast, 0-d, empty), with NaN / +-0 / +-inf salted inputs, mixed-dtype
promotion, out=, dunders and the reference's error cases and known answers
(tests/python/test_comparison.py, tests/python/test_complex.py).

Complex: add/sub/mul/div/neg/abs over c64/c128 and the real -> complex and c64 -> c128 casts.
"""
import numpy as np
import pytest

import musapy_amd as ms
from oracle import reference as R
from tests.conftest import assert_bits_equal

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(31337)
CMPS = ["eq", "ne", "lt", "gt", "le", "ge"]


def dev(x):
    return ms.from_numpy(x)


def salted(shape, dt):
    x = RNG.standard_normal(shape).astype(dt)
    flat = x.reshape(-1)
    if flat.size:
        idx = RNG.choice(flat.size, size=max(1, flat.size // 6), replace=False)
        flat[idx] = np.resize(np.array([np.nan, 0.0, -0.0, np.inf, -np.inf], dtype=dt), idx.size)
    return x


def cplx(shape, dt):
    return (RNG.standard_normal(shape) + 1j * RNG.standard_normal(shape)).astype(dt)


def check_bool(got_arr, want, what):
    assert got_arr.dtype == "b1", what
    got = got_arr.numpy()
    assert got.dtype == np.bool_, what
    assert_bits_equal(got.view(np.uint8), want.view(np.uint8), what)


def _views():
    return [
        ("contig", lambda x: x, lambda a: a),
        ("transposed", lambda x: x.T, lambda a: ms.transpose(a)),
        ("flipped", lambda x: x[:, ::-1], lambda a: ms.flip(a, 1)),
        ("sliced", lambda x: x[1:11:2, 3:19], lambda a: ms.slice(a, [(1, 11, 2), (3, 19, 1)])),
    ]


@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("op", CMPS)
def test_compare_layouts(op, dt):
    base_a, base_b = salted((12, 20), dt), salted((12, 20), dt)
    base_b[::2] = base_a[::2]
    A, B = dev(base_a), dev(base_b)
    for name, nf, df in _views():
        check_bool(getattr(ms, op)(df(A), df(B)), R.compare(op, nf(base_a), nf(base_b)), f"{op} {name}")
    # misaligned start (offset 1 element) on both sides
    fa, fb = base_a.reshape(-1), base_b.reshape(-1)
    got = getattr(ms, op)(ms.slice(dev(fa), [(1, 240, 1)]), ms.slice(dev(fb), [(0, 239, 1)]))
    check_bool(got, R.compare(op, fa[1:], fb[:-1]), f"{op} offset")


@pytest.mark.parametrize("sa,sb", [((4096, 1), (8192,)), ((1,), (1000,)), ((), (33, 7)), ((5, 1, 3), (4, 1)),
                                   ((7, 1), (1, 9)), ((3,), ()), ((), ()), ((0, 4), (4,)), ((2, 0), (1, 1))])
def test_compare_broadcast_and_edge_shapes(sa, sb):
    a, b = salted(sa, np.float32), salted(sb, np.float32)
    for op in ("lt", "eq"):
        got = getattr(ms, op)(dev(a), dev(b))
        want = R.compare(op, a, b)
        assert got.shape == want.shape
        check_bool(got, want, f"{op} {sa} vs {sb}")


def test_compare_sizes_and_tails():
    for n in (1, 3, 15, 16, 17, 255, 1023, 1025, 4097, 65537, 1 << 20, (1 << 20) + 13):
        a, b = salted(n, np.float32), salted(n, np.float32)
        b[::5] = a[::5]
        check_bool(ms.le(dev(a), dev(b)), R.compare("le", a, b), f"le n={n}")
        a64, b64 = a.astype(np.float64), b.astype(np.float64)
        check_bool(ms.ne(dev(a64), dev(b64)), R.compare("ne", a64, b64), f"ne f64 n={n}")


def test_compare_mixed_dtypes_promote_then_compare():
    f32, f64 = salted((300,), np.float32), salted((300,), np.float64)
    f64[::3] = f32[::3]
    i64 = RNG.integers(-5, 5, 300).astype(np.int64)
    i32 = RNG.integers(-5, 5, 300).astype(np.int32)
    cases = [(f32, f64), (f64, f32), (i64, f64), (f32, i64), (i32, f32), (i64, i32.astype(np.float64))]
    for a, b in cases:
        for op in ("eq", "lt", "ge"):
            check_bool(getattr(ms, op)(dev(a), dev(b)), R.compare(op, a, b), f"{op} {a.dtype} vs {b.dtype}")


def test_compare_out_param_and_errors():
    a, b = dev(np.array([1.0, 2.0, 3.0], np.float32)), dev(np.array([3.0, 2.0, 1.0], np.float32))
    out = ms.array([False, False, False], dtype="b1")
    r = ms.gt(a, b, out=out)
    assert r.tolist() == [False, False, True]
    assert out.tolist() == [False, False, True]
    with pytest.raises(ms.DtypeError):
        ms.gt(a, b, out=ms.array([0.0, 0.0, 0.0]))
    with pytest.raises(ms.ShapeError):
        ms.gt(a, b, out=ms.array([False, False], dtype="b1"))
    with pytest.raises(ms.ShapeError):
        ms.eq(a, dev(np.array([1.0, 2.0], np.float32)))
    with pytest.raises(ms.DtypeError):  # promoted dtype int64 is outside the compute whitelist
        ms.eq(dev(np.array([1, 2], np.int64)), dev(np.array([1, 2], np.int64)))
    with pytest.raises(ms.DtypeError):
        ms.lt(dev(cplx(3, np.complex64)), dev(cplx(3, np.complex64)))


def test_compare_reference_known_answers_and_dunders():
    """tests/python/test_comparison.py values (TestComparison, TestComparisonDunders, TestComparisonMusa)."""
    a = ms.array([1.0, 2.0, 3.0])
    b = ms.array([1.0, 5.0, 3.0])
    c = ms.eq(a, b)
    assert c.dtype == "b1" and c.dtype == "bool" and c.dtype == ms.bool_
    assert c.tolist() == [True, False, True]
    assert ms.ne(a, b).tolist() == [False, True, False]
    a, b = ms.array([1.0, 2.0, 3.0]), ms.array([3.0, 2.0, 1.0])
    assert ms.lt(a, b).tolist() == [True, False, False]
    assert ms.gt(a, b).tolist() == [False, False, True]
    assert ms.le(a, b).tolist() == [True, True, False]
    assert ms.ge(a, b).tolist() == [False, True, True]
    assert (a == b).tolist() == [False, True, False]
    assert (a != b).tolist() == [True, False, True]
    assert (a < b).tolist() == [True, False, False]
    assert (a > b).tolist() == [False, False, True]
    assert (a <= b).tolist() == [True, True, False]
    assert (a >= b).tolist() == [False, True, True]
    assert (a >= b).dtype == "b1"
    c = ms.eq(ms.array([[1.0], [2.0], [3.0]]), ms.array([1.0, 2.0, 3.0, 4.0]))
    assert c.shape == (3, 4)
    assert c.tolist() == [[True, False, False, False], [False, True, False, False], [False, False, True, False]]
    assert ms.lt(ms.array([[1.0], [2.0], [3.0]]), ms.array([1.0, 2.0, 3.0, 4.0])).tolist()[0] == [False, True, True,
                                                                                                 True]
    c = ms.eq(ms.array([1, 2, 3], dtype="i64"), ms.array([1.0, 2.5, 3.0], dtype="f64"))
    assert c.dtype == "b1" and c.tolist() == [True, False, True]
    c = ms.gt(ms.array([[1.0, 2.0], [3.0, 4.0]]), ms.array([[1.0, 0.0], [3.0, 0.0]]))
    assert c.tolist() == [[False, True], [False, True]]
    assert (ms.array([[1.0], [2.0]]) == ms.array([1.0, 2.0, 3.0])).tolist() == [[True, False, False],
                                                                               [False, True, False]]


@pytest.mark.parametrize("dt", [np.complex64, np.complex128])
def test_complex_compare(dt):
    x, y = cplx((9, 31), dt), cplx((9, 31), dt)
    y[::2] = x[::2]
    y[1, :5] = x[1, :5].real + 1j * x[1, :5].imag * -1  # same real part only
    x[2, 0] = complex(np.nan, 0)
    y[2, 0] = complex(np.nan, 0)
    x[2, 1], y[2, 1] = complex(0.0, -0.0), complex(-0.0, 0.0)
    X, Y = dev(x), dev(y)
    for op in ("eq", "ne"):
        check_bool(getattr(ms, op)(X, Y), R.compare(op, x, y), f"{op} {dt}")
        check_bool(getattr(ms, op)(ms.transpose(X), ms.flip(ms.transpose(Y), 0)),
                   R.compare(op, x.T, y.T[::-1]), f"{op} {dt} views")
        check_bool(getattr(ms, op)(X, ms.slice(Y, [(0, 1, 1), (0, 31, 1)])), R.compare(op, x, y[:1]),
                   f"{op} {dt} broadcast")
    # reference known answers (tests/python/test_complex.py::test_eq_ne)
    a = ms.array([1 + 2j, 3 + 4j, 5 + 0j], dtype=np.dtype(dt).name)
    b = ms.array([1 + 2j, 3 - 4j, 5 + 0j], dtype=np.dtype(dt).name)
    assert ms.eq(a, b).dtype == "b1" and ms.eq(a, b).tolist() == [True, False, True]
    assert ms.ne(a, b).tolist() == [False, True, False]


def test_mixed_real_complex_compare():
    a = np.array([1.0, 2.0, 3.0, np.nan], np.float32)
    z = np.array([1 + 0j, 2 + 1j, 3 - 0j, complex(np.nan, 0)], np.complex64)
    for op in ("eq", "ne"):
        check_bool(getattr(ms, op)(dev(a), dev(z)), R.compare(op, a, z), f"{op} f32 vs c64")
        check_bool(getattr(ms, op)(dev(a.astype(np.float64)), dev(z)), R.compare(op, a.astype(np.float64), z),
                   f"{op} f64 vs c64")
    with pytest.raises(ms.DtypeError):  # c64 vs c128 narrows to c64, and c128 -> c64 has no cast
        ms.eq(dev(z), dev(z.astype(np.complex128)))


# ---- complex arithmetic -----------------------------------------------------------------------
@pytest.mark.parametrize("dt", [np.complex64, np.complex128])
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_complex_binary_layouts(op, dt):
    base_a, base_b = cplx((12, 20), dt), cplx((12, 20), dt)
    base_a[0, :3] = [complex(np.inf, 1), complex(np.nan, 0), complex(1e30, -1e30)]
    base_b[0, :3] = [complex(0.5, 0), complex(1, 1), complex(1e-30, 3e30)]
    A, B = dev(base_a), dev(base_b)
    for name, nf, df in _views():
        got = getattr(ms, op)(df(A), df(B)).numpy()
        assert_bits_equal(got, R.binary(op, nf(base_a), nf(base_b)), f"{op} {dt} {name}")
    fa, fb = base_a.reshape(-1), base_b.reshape(-1)
    got = getattr(ms, op)(ms.slice(dev(fa), [(1, 240, 1)]), ms.slice(dev(fb), [(0, 239, 1)])).numpy()
    assert_bits_equal(got, R.binary(op, fa[1:], fb[:-1]), f"{op} {dt} offset")
    col, row = base_a[:, :1], base_b[:1, :]
    assert_bits_equal(getattr(ms, op)(dev(col), dev(row)).numpy(), R.binary(op, col, row), f"{op} {dt} bcast")


@pytest.mark.parametrize("dt", [np.complex64, np.complex128])
def test_complex_binary_sizes(dt):
    for n in (1, 2, 3, 7, 8, 9, 255, 1025, 65537, (1 << 20) + 3):
        a, b = cplx(n, dt), cplx(n, dt)
        for op in ("mul", "div"):
            assert_bits_equal(getattr(ms, op)(dev(a), dev(b)).numpy(), R.binary(op, a, b), f"{op} {dt} n={n}")


@pytest.mark.parametrize("dt", [np.complex64, np.complex128])
def test_complex_unary(dt):
    z = cplx((40, 33), dt) * 4
    z[0, :6] = [3 + 4j, -5 - 12j, complex(0.0, -0.0), complex(-0.0, 0.0), complex(np.inf, 1), complex(np.nan, 2)]
    Z = dev(z)
    for op in ("neg", "abs"):
        want = R.unary(op, z)
        got = getattr(ms, op)(Z)
        assert got.dtype == want.dtype.name
        assert_bits_equal(got.numpy(), want, f"{op} {dt}")
        assert_bits_equal(getattr(ms, op)(ms.transpose(Z)).numpy(), R.unary(op, z.T), f"{op} {dt} T")
        sl = ms.slice(Z, [(1, 40, 3), (2, 33, 2)])
        assert_bits_equal(getattr(ms, op)(sl).numpy(), R.unary(op, z[1:40:3, 2:33:2]), f"{op} {dt} sliced")
    assert_bits_equal((-Z).numpy(), R.unary("neg", z), "dunder neg", nan_bits=True)
    assert_bits_equal(abs(Z).numpy(), R.unary("abs", z), "dunder abs")
    out = ms.from_numpy(np.zeros(z.shape, np.float32 if dt == np.complex64 else np.float64))
    ms.abs(Z, out=out)
    assert_bits_equal(out.numpy(), R.unary("abs", z), "abs out=")
    for op in ("sin", "exp", "sign"):
        with pytest.raises(ms.DtypeError):
            getattr(ms, op)(Z)
    with pytest.raises(ms.DtypeError):
        ms.pow(Z, Z)


def test_casts_to_complex():
    x32 = salted((37, 29), np.float32)
    x64 = salted((37, 29), np.float64)
    for x in (x32, x64):
        for dst in ("c64", "c128"):
            X = dev(x)
            assert_bits_equal(ms.astype(X, dst).numpy(), R.cast(x, dst), f"{x.dtype}->{dst}", nan_bits=True)
            assert_bits_equal(ms.astype(ms.transpose(X), dst).numpy(), R.cast(x.T, dst), f"{x.dtype}->{dst} T",
                              nan_bits=True)
    z = cplx((37, 29), np.complex64)
    Z = dev(z)
    assert_bits_equal(Z.astype("c128").numpy(), R.cast(z, "c128"), "c64->c128")
    assert_bits_equal(ms.astype(ms.flip(Z, 0), ms.complex128).numpy(), R.cast(z[::-1], "c128"), "c64->c128 flip")
    with pytest.raises(ms.DtypeError):
        ms.astype(Z, "f32")
    with pytest.raises(ms.DtypeError):
        ms.astype(dev(z.astype(np.complex128)), "c64")
    with pytest.raises(ms.DtypeError):
        ms.astype(dev(np.arange(4)), "c64")


def test_mixed_real_complex_binary():
    """tests/python/test_complex.py TestMixedPromotion."""
    r = ms.add(ms.array([1.0, 2.0], dtype="f64"), ms.array([1 + 1j, 2 - 2j], dtype="c64"))
    assert r.dtype == "c128" and np.allclose(np.array(r.tolist()), [2 + 1j, 4 - 2j])
    r = ms.add(ms.array([1.0, 2.0], dtype="f32"), ms.array([1 + 1j, 2 - 2j], dtype="c64"))
    assert r.dtype == "c64"
    r = ms.add(ms.array([1.0, 2.0], dtype="f32"), ms.array([1 + 1j, 2 - 2j], dtype="c128"))
    assert r.dtype == "c128"
    r = ms.add(ms.array([1 + 1j, 2 + 2j]), ms.array([1.0, 2.0]))
    assert r.dtype == "c128" and r.tolist() == [2 + 1j, 4 + 2j]
    assert ms.add(ms.array([1 + 1j], dtype="c64"), ms.array([2 + 2j], dtype="c64")).dtype == "c64"
    a, z = salted((64,), np.float32), cplx((64,), np.complex128)
    for op in ("add", "sub", "mul", "div"):
        assert_bits_equal(getattr(ms, op)(dev(a), dev(z)).numpy(), R.binary(op, a, z), f"{op} f32 c128")
        assert_bits_equal(getattr(ms, op)(dev(z), dev(a)).numpy(), R.binary(op, z, a), f"{op} c128 f32")


def test_reference_complex_known_answers():
    """tests/python/test_complex.py TestComplexOps / TestComplexCreation values."""
    a = ms.array([1 + 2j, 3 - 4j])
    assert a.dtype == "c128" and a.tolist() == [1 + 2j, 3 - 4j]
    assert ms.array([1.0, 2.0, 3.0], dtype="c64").tolist() == [1 + 0j, 2 + 0j, 3 + 0j]
    for dtype, tol in (("c64", 1e-5), ("c128", 1e-12)):
        x = ms.array([1 + 2j, 3 + 4j, -1 + 0.5j], dtype=dtype)
        y = ms.array([1 - 1j, 0 + 2j, 2 - 2j], dtype=dtype)
        xn, yn = np.array([1 + 2j, 3 + 4j, -1 + 0.5j]), np.array([1 - 1j, 0 + 2j, 2 - 2j])
        for name, got, exp in (("add", ms.add(x, y), xn + yn), ("sub", ms.sub(x, y), xn - yn),
                               ("mul", ms.mul(x, y), xn * yn), ("div", ms.div(x, y), xn / yn)):
            assert np.allclose(np.array(got.tolist()), exp, rtol=tol, atol=tol), name
        x = ms.array([1 + 2j, 3 - 4j, -0.5 + 0.25j], dtype=dtype)
        ab = ms.abs(x)
        assert ab.dtype == ("f32" if dtype == "c64" else "f64")
        assert np.allclose(np.array(ab.tolist()), np.abs([1 + 2j, 3 - 4j, -0.5 + 0.25j]), rtol=tol)
    arr = ms.array([[1 + 1j, 2 + 2j], [3 + 3j, 4 + 4j]])
    view = arr[:, 0]
    assert view.tolist() == [1 + 1j, 3 + 3j]
    assert ms.neg(view).tolist() == [-1 - 1j, -3 - 3j]
