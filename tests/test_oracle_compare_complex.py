"""Pins the oracle's comparison and complex restatements (CPU only, no GPU).

Comparisons (oracle_compare, op_builder.rs:1765-1864) are checked against numpy's IEEE
comparison ufuncs, an independent implementation, on data salted with NaN, +-0 and +-inf, under
broadcasting and strided views; and against the known answers of the reference's own tests
(tests/python/test_comparison.py, tests/python/test_complex.py).

Complex arithmetic (oracle_binary_cplx / oracle_unary_cplx, op_builder.rs:1652-1969) is checked
against exact rational arithmetic (fractions.Fraction) rounded once to f64, and for c64 then once
more to f32 -- the rounding the reference's CplxScalar round trip specifies -- and against
identities that hold exactly in IEEE arithmetic (z * 1, z * i, z * conj(z), z / z).  abs is
checked against the correctly rounded sqrt of the correctly rounded sum of squares.  Casts to
complex are checked against numpy's astype.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import reference as R

RNG = np.random.default_rng(77)
NP_CMP = {"eq": np.equal, "ne": np.not_equal, "lt": np.less, "gt": np.greater, "le": np.less_equal,
          "ge": np.greater_equal}


def salted(shape, dt):
    x = RNG.standard_normal(shape).astype(dt)
    flat = x.reshape(-1)
    k = max(1, flat.size // 8)
    idx = RNG.choice(flat.size, size=min(flat.size, 5 * k), replace=False)
    specials = np.array([np.nan, 0.0, -0.0, np.inf, -np.inf], dtype=dt)
    flat[idx] = np.resize(specials, idx.size)
    return x


@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("op", list(NP_CMP))
def test_compare_matches_numpy_ieee(op, dt):
    a, b = salted((17, 23), dt), salted((17, 23), dt)
    b[::3] = a[::3]  # equal pairs, including NaN == NaN (false) and +0 == -0 (true)
    got = R.compare(op, a, b)
    assert got.dtype == np.bool_
    assert np.array_equal(got, NP_CMP[op](a, b))
    # strided / transposed views and broadcasting go through the stride walk
    assert np.array_equal(R.compare(op, a.T, b.T), NP_CMP[op](a.T, b.T))
    assert np.array_equal(R.compare(op, a[::-2, 1::3], b[::2, ::3]), NP_CMP[op](a[::-2, 1::3], b[::2, ::3]))
    col, row = a[:, :1], b[:1, :]
    assert np.array_equal(R.compare(op, col, row), NP_CMP[op](col, row))


def test_compare_signed_zero_and_nan_cases():
    a = np.array([0.0, -0.0, np.nan, np.nan, 1.0, np.inf], np.float32)
    b = np.array([-0.0, 0.0, np.nan, 1.0, np.nan, np.inf], np.float32)
    assert R.compare("eq", a, b).tolist() == [True, True, False, False, False, True]
    assert R.compare("ne", a, b).tolist() == [False, False, True, True, True, False]
    assert R.compare("le", a, b).tolist() == [True, True, False, False, False, True]
    assert R.compare("lt", a, b).tolist() == [False] * 6


def test_compare_reference_known_answers():
    """Values of tests/python/test_comparison.py (TestComparison / TestComparisonDunders)."""
    f = lambda v: np.array(v, np.float32)  # noqa: E731 - musapy's default float dtype
    assert R.compare("eq", f([1, 2, 3]), f([1, 5, 3])).tolist() == [True, False, True]
    assert R.compare("ne", f([1, 2, 3]), f([1, 5, 3])).tolist() == [False, True, False]
    a, b = f([1, 2, 3]), f([3, 2, 1])
    assert R.compare("lt", a, b).tolist() == [True, False, False]
    assert R.compare("gt", a, b).tolist() == [False, False, True]
    assert R.compare("le", a, b).tolist() == [True, True, False]
    assert R.compare("ge", a, b).tolist() == [False, True, True]
    c = R.compare("eq", f([[1], [2], [3]]), f([1, 2, 3, 4]))
    assert c.shape == (3, 4)
    assert c.tolist() == [[True, False, False, False], [False, True, False, False], [False, False, True, False]]
    c = R.compare("lt", f([[1], [2], [3]]), f([1, 2, 3, 4]))
    assert c.tolist()[0] == [False, True, True, True]
    i64 = np.array([1, 2, 3], np.int64)
    assert R.compare("eq", i64, np.array([1.0, 2.5, 3.0])).tolist() == [True, False, True]
    assert R.compare("gt", f([[1, 2], [3, 4]]), f([[1, 0], [3, 0]])).tolist() == [[False, True], [False, True]]
    assert R.compare("eq", f([[1], [2]]), f([1, 2, 3])).tolist() == [[True, False, False], [False, True, False]]
    with pytest.raises(R.OracleError):
        R.compare("eq", f([1, 2, 3]), f([1, 2]))


@pytest.mark.parametrize("dt", [np.complex64, np.complex128])
def test_complex_compare_reference_known_answers(dt):
    """tests/python/test_complex.py::test_eq_ne and ::test_ordering_rejected."""
    x = np.array([1 + 2j, 3 + 4j, 5 + 0j], dt)
    y = np.array([1 + 2j, 3 - 4j, 5 + 0j], dt)
    assert R.compare("eq", x, y).tolist() == [True, False, True]
    assert R.compare("ne", x, y).tolist() == [False, True, False]
    for op in ("lt", "gt", "le", "ge"):
        with pytest.raises(R.OracleError):
            R.compare(op, x, y)
    z = np.array([complex(np.nan, 0), complex(0, -0.0), complex(1, np.nan)], dt)
    w = np.array([complex(np.nan, 0), complex(-0.0, 0), complex(1, 2)], dt)
    assert R.compare("eq", z, w).tolist() == [False, True, False]
    assert R.compare("ne", z, w).tolist() == [True, False, True]


def test_mixed_real_complex_compare_casts_first():
    a = np.array([1.0, 2.0, 3.0], np.float32)
    z = np.array([1 + 0j, 2 + 1j, 3 - 0j], np.complex64)
    assert R.compare("eq", a, z).tolist() == [True, False, True]
    with pytest.raises(R.OracleError):  # c64 vs c128 narrows to c64: c128 -> c64 has no cast
        R.compare("eq", z, z.astype(np.complex128))


# ---- complex arithmetic ----------------------------------------------------------------------
def _exact(op, a, b):
    ar, ai, br, bi = (Fraction(float(v)) for v in (a.real, a.imag, b.real, b.imag))
    if op == "add":
        return ar + br, ai + bi
    if op == "sub":
        return ar - br, ai - bi
    if op == "mul":
        return ar * br - ai * bi, ar * bi + ai * br
    den = br * br + bi * bi
    return (ar * br + ai * bi) / den, (ai * br - ar * bi) / den


@pytest.mark.parametrize("dt", [np.complex64, np.complex128])
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_complex_binary_exact_on_small_integers(op, dt):
    """Components are small integers, so every product and sum is exact in f64 and the only
    roundings are the final quotient's (to f64, then to f32 for c64)."""
    n = 300
    a = (RNG.integers(-512, 512, n) + 1j * RNG.integers(-512, 512, n)).astype(dt)
    b = (RNG.integers(-512, 512, n) + 1j * RNG.integers(-512, 512, n)).astype(dt)
    b[b == 0] = 1 + 1j
    got = R.binary(op, a, b)
    assert got.dtype == dt
    for g, x, y in zip(got, a, b):
        re, im = _exact(op, x, y)
        want_re, want_im = float(re), float(im)  # Fraction -> float rounds to nearest even
        if dt == np.complex64:
            want_re, want_im = np.float32(want_re), np.float32(want_im)
        assert g.real == want_re and g.imag == want_im, (op, x, y, g, want_re, want_im)


@pytest.mark.parametrize("dt", [np.complex64, np.complex128])
def test_complex_binary_identities(dt):
    z = (RNG.standard_normal(500) + 1j * RNG.standard_normal(500)).astype(dt)
    one = np.ones_like(z)
    i = np.full_like(z, 1j)
    assert np.array_equal(R.binary("mul", z, one), z)
    rot = R.binary("mul", z, i)  # (a + bi) * i = -b + ai, exact
    assert np.array_equal(rot.real, -z.imag) and np.array_equal(rot.imag, z.real)
    zz = R.binary("mul", z, np.conj(z))
    assert np.all(zz.imag == 0)
    q = R.binary("div", z, z)
    assert np.all(q.real == 1) and np.all(q.imag == 0)
    # close to numpy's own complex arithmetic (a different algorithm for division)
    w = (RNG.standard_normal(500) + 1j * RNG.standard_normal(500)).astype(dt)
    tol = 1e-5 if dt == np.complex64 else 1e-13
    for op, f in (("add", np.add), ("sub", np.subtract), ("mul", np.multiply), ("div", np.divide)):
        assert np.allclose(R.binary(op, z, w), f(z, w), rtol=tol, atol=tol), op
    with pytest.raises(R.OracleError):
        R.binary("pow", z, w)


@pytest.mark.parametrize("dt", [np.complex64, np.complex128])
def test_complex_unary_neg_abs(dt):
    z = (RNG.standard_normal(400) * 8 + 1j * RNG.standard_normal(400) * 8).astype(dt)
    z[:4] = np.array([3 + 4j, -5 - 12j, complex(0.0, -0.0), complex(-0.0, 0.0)], dt)
    neg = R.unary("neg", z)
    assert neg.dtype == dt
    assert np.array_equal(np.signbit(neg.real), ~np.signbit(z.real))
    assert np.array_equal(neg, -z)
    ab = R.unary("abs", z)
    rdt = np.float32 if dt == np.complex64 else np.float64
    assert ab.dtype == rdt
    assert ab[0] == 5 and ab[1] == 13 and ab[2] == 0 and ab[3] == 0
    for g, v in zip(ab, z):
        re, im = float(v.real), float(v.imag)
        if dt == np.complex64:  # squares of f32 values are exact in f64; one rounding in the sum
            want = np.float32(math.sqrt(float(Fraction(re) ** 2 + Fraction(im) ** 2)))
        else:
            want = math.sqrt(re * re + im * im)
        assert g == want, (v, g, want)
    for op in ("sin", "exp", "sign"):
        with pytest.raises(R.OracleError):
            R.unary(op, z)


def test_casts_to_complex_match_numpy():
    x32 = salted((50,), np.float32)
    x64 = salted((50,), np.float64)
    for x, dst, ndt in ((x32, "c64", np.complex64), (x32, "c128", np.complex128), (x64, "c64", np.complex64),
                        (x64, "c128", np.complex128)):
        got = R.cast(x, dst)
        want = x.astype(ndt)
        assert got.dtype == ndt
        assert np.array_equal(got.real.view(got.real.dtype), want.real, equal_nan=True)
        assert np.all(got.imag == 0) and not np.any(np.signbit(got.imag))
    z = (RNG.standard_normal(40) + 1j * RNG.standard_normal(40)).astype(np.complex64)
    assert np.array_equal(R.cast(z, "c128"), z.astype(np.complex128))
    assert np.array_equal(R.cast(z.T[::-1], "c128"), z[::-1].astype(np.complex128))
    for src, dst in (("c128", "c64"), ("c64", "f32"), ("i64", "c64"), ("u8", "c128")):
        with pytest.raises(R.OracleError):
            R.validate_cast(src, dst)


def test_mixed_real_complex_binary_promotion():
    """tests/python/test_complex.py TestMixedPromotion: result dtypes and values."""
    f64 = np.array([1.0, 2.0])
    c64 = np.array([1 + 1j, 2 - 2j], np.complex64)
    r = R.binary("add", f64, c64)
    assert r.dtype == np.complex128 and r.tolist() == [2 + 1j, 4 - 2j]
    r = R.binary("add", f64.astype(np.float32), c64)
    assert r.dtype == np.complex64
    r = R.binary("add", f64.astype(np.float32), c64.astype(np.complex128))
    assert r.dtype == np.complex128
    r = R.binary("add", np.array([1 + 1j, 2 + 2j]), np.array([1.0, 2.0], np.float32))
    assert r.dtype == np.complex128 and r.tolist() == [2 + 1j, 4 + 2j]


# ---- contiguous() materialisation -------------------------------------------------------------
@pytest.mark.parametrize("dt", [np.bool_, np.int8, np.uint16, np.float16, np.int32, np.float32, np.int64,
                                np.float64, np.complex64, np.complex128])
def test_contiguous_matches_numpy(dt):
    """oracle_copy_bytes (cpu_copy_bytes, indexing.rs:1388-1409) against numpy's own copy."""
    raw = RNG.integers(0, 256, 6 * 7 * 9 * np.dtype(dt).itemsize, dtype=np.uint8)
    x = raw.view(dt).reshape(6, 7, 9)
    for v in (x, x.T, x.transpose(1, 0, 2), x[::-1, 2:, ::3], x[1:5:2, ::-2, 4], x[:, 3:3], x[2, 3, 4]):
        got = R.contiguous(v)
        want = np.array(v, order="C", copy=True)
        assert got.shape == want.shape and got.dtype == want.dtype
        assert got.tobytes() == want.tobytes()


def test_contiguous_reference_known_answers():
    """tests/python/test_indexing.py TestContiguous values."""
    c = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], np.float32)
    assert R.contiguous(c.T).tolist() == [[1.0, 4.0], [2.0, 5.0], [3.0, 6.0]]
    assert R.contiguous(c[:, ::-1]).tolist() == [[3.0, 2.0, 1.0], [6.0, 5.0, 4.0]]
    assert R.contiguous(np.arange(10, dtype=np.float32)[3:7]).tolist() == [3.0, 4.0, 5.0, 6.0]
