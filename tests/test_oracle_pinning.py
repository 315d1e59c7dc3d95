"""Pins the CPU oracle (oracle/) before it is trusted as the parity reference.

Each check compares the oracle with something computed independently of it: numpy's IEEE
float32/float64 arithmetic and sequential accumulate, numpy/torch format conversions, exact
(fsum / rational) sums, and known answers that follow from the reference's source
(rust/musapy-ops/src/op_builder.rs) or its own tests (tests/python/test_reduction.py,
test_elementwise.py).  A plausible slip in the oracle -- a wrong operand order, a dropped
term, a transposed stride, the wrong tie or NaN rule -- fails one of them.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import reference as R
from tests.conftest import assert_bits_equal, ulp_diff_f32, ulp_diff_f64

RNG = np.random.default_rng(1234)


# ---- binary: IEEE single/double ops are correctly rounded, so numpy must agree bit for bit ----
@pytest.mark.parametrize("op,npop", [("add", np.add), ("sub", np.subtract), ("mul", np.multiply),
                                     ("div", np.divide)])
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_binary_matches_ieee(op, npop, dt):
    a = RNG.standard_normal((37, 19)).astype(dt)
    b = RNG.standard_normal((37, 19)).astype(dt)
    b[0, :3] = 0.0
    a[1, 0] = np.inf
    a[1, 1] = np.nan
    assert_bits_equal(R.binary(op, a, b), npop(a, b), op)


def test_binary_operand_order_and_broadcast():
    a = RNG.standard_normal((4, 1)).astype(np.float32)
    b = RNG.standard_normal((5,)).astype(np.float32)
    assert_bits_equal(R.binary("sub", a, b), a - b, "broadcast sub a-b")
    assert_bits_equal(R.binary("div", b, a), b / a, "broadcast div b/a")
    x = RNG.standard_normal((6, 8)).astype(np.float64)
    assert_bits_equal(R.binary("sub", x.T, x[:, ::-1].T), x.T - x[:, ::-1].T, "strided views")


def test_binary_promotion_gpu_narrow():
    # promote(f32, f64, all_gpu=true) = f32 (dtype.rs GPU narrow rule); i64 + f64 -> f64 (JAX)
    a = np.array([1.5, 2.25], np.float32)
    b = np.array([0.1, 0.2], np.float64)
    r = R.binary("add", a, b)
    assert r.dtype == np.float32
    assert_bits_equal(r, a + b.astype(np.float32), "f32+f64 on device")
    i = np.array([3, -7], np.int64)
    r = R.binary("add", i, b)
    assert r.dtype == np.float64
    assert_bits_equal(r, i.astype(np.float64) + b, "i64+f64")


def test_pow_special_cases():
    # C99 / IEEE pow special values (glibc); the reference calls f32::powf / f64::powf
    a = np.array([1.0, np.nan, 2.0, -8.0, 0.0, 0.0, np.inf, -1.0], np.float64)
    b = np.array([np.nan, 0.0, -np.inf, 1.0 / 3.0, -1.0, 0.5, -2.0, np.inf], np.float64)
    want = np.array([1.0, 1.0, 0.0, np.nan, np.inf, 0.0, 0.0, 1.0])
    got = R.binary("pow", a, b)
    assert np.array_equal(np.isnan(got), np.isnan(want)) and np.all((got == want) | np.isnan(want))


def _pow_samples(n):
    """Positive bases over six decades with exponents that keep the result finite, plus negative
    bases with integral exponents (odd and even: the sign of the result depends on the parity)."""
    base = np.exp(RNG.uniform(np.log(1e-3), np.log(1e3), n))
    expo = RNG.uniform(-12, 12, n)
    nb = n // 4
    base[:nb] = -RNG.uniform(0.05, 20.0, nb)
    expo[:nb] = RNG.integers(-9, 10, nb).astype(np.float64)
    return base, expo


def test_pow_f32_close_to_exact():
    """f32 pow against the f64 evaluation rounded once to f32 (f64 pow is within 1 ulp of f64,
    far below half an ulp of f32)."""
    a, b = _pow_samples(20000)
    a32, b32 = a.astype(np.float32), b.astype(np.float32)
    got = R.binary("pow", a32, b32)
    want = np.power(a32.astype(np.float64), b32.astype(np.float64)).astype(np.float32)
    ok = np.isfinite(want) & (want != 0)
    assert ok.sum() > 19000
    assert ulp_diff_f32(got[ok], want[ok]).max() <= 1
    # negative base, integral exponent: the sign follows the exponent's parity
    neg = (a32 < 0) & ok
    assert np.array_equal(np.signbit(got[neg]), np.signbit(want[neg]))


def test_pow_f64_close_to_exact():
    """f64 pow against x87 extended precision (64-bit mantissa), rounded once to double."""
    a, b = _pow_samples(20000)
    got = R.binary("pow", a, b)
    want = np.power(a.astype(np.longdouble), b.astype(np.longdouble)).astype(np.float64)
    ok = np.isfinite(want) & (want != 0)
    assert ok.sum() > 19000
    assert ulp_diff_f64(got[ok], want[ok]).max() <= 1


# ---- unary ----
def _exact_f32(fn, x):
    """float32 result of `fn` evaluated in float64 (error <= 1 ulp(f64) << 0.5 ulp(f32))."""
    return fn(x.astype(np.float64)).astype(np.float32)


@pytest.mark.parametrize("op,fn", [("sin", np.sin), ("cos", np.cos), ("exp", np.exp), ("log", np.log)])
def test_unary_transcendental_f32_close_to_exact(op, fn):
    x = RNG.uniform(0.01 if op == "log" else -20, 20, 20000).astype(np.float32)
    got = R.unary(op, x)
    assert ulp_diff_f32(got, _exact_f32(fn, x)).max() <= 1


@pytest.mark.parametrize("op,fn", [("sin", np.sin), ("cos", np.cos), ("exp", np.exp), ("log", np.log)])
def test_unary_transcendental_f64_close_to_exact(op, fn):
    """f64 forms against x87 extended precision (64-bit mantissa), rounded once to double."""
    x = RNG.uniform(0.01 if op == "log" else -20, 20, 20000)
    got = R.unary(op, x)
    want = fn(x.astype(np.longdouble)).astype(np.float64)
    assert ulp_diff_f64(got, want).max() <= 1


def test_unary_exact_ops():
    x = np.array([-2.5, -0.0, 0.0, 3.0, np.inf, -np.inf, np.nan, 1e-40], np.float32)
    assert_bits_equal(R.unary("abs", x), np.abs(x), "abs")
    assert_bits_equal(R.unary("neg", x), -x, "neg")
    # sign: v>0 -> 1, v<0 -> -1, else +0.0 (NaN and -0.0 give +0.0), op_builder.rs:1885-1893
    assert_bits_equal(R.unary("sign", x), np.array([-1, 0, 0, 1, 1, -1, 0, 1], np.float32), "sign")


def test_unary_strided_view():
    x = RNG.standard_normal((16, 24)).astype(np.float64)
    v = x.T[::2, ::-1]
    assert_bits_equal(R.unary("neg", v), -v, "neg of strided view")
    assert_bits_equal(R.unary("exp", v)[3, 5:7], np.array([math.exp(v[3, 5]), math.exp(v[3, 6])]), "exp view")


def test_clamp_semantics():
    x = np.array([-3.0, -1.0, 0.5, 1.0, 2.0, np.nan, -0.0], np.float64)
    want = np.array([-1.0, -1.0, 0.5, 1.0, 1.0, np.nan, -0.0])
    assert_bits_equal(R.clamp(x, -1.0, 1.0), want, "clamp f64")
    # f32: lo/hi narrowed from f64 first
    x32 = np.array([0.1, 0.2], np.float32)
    got = R.clamp(x32, 0.15, 0.3)
    assert_bits_equal(got, np.array([np.float32(0.15), np.float32(0.2)]), "clamp f32 narrowing")


# ---- casts (Rust `as`) ----
def test_cast_int_to_float_rne():
    i = np.array([2**53 + 1, -(2**53) - 3, 2**63 - 1, -(2**63), 16777217, 123], np.int64)
    assert_bits_equal(R.cast(i, "f64"), i.astype(np.float64), "i64->f64")
    assert_bits_equal(R.cast(i, "f32"), i.astype(np.float32), "i64->f32")
    u = np.array([2**64 - 1, 2**63, 2**53 + 1, 7], np.uint64)
    assert_bits_equal(R.cast(u, "f32"), u.astype(np.float32), "u64->f32")
    assert_bits_equal(R.cast(u, "i64"), u.view(np.int64), "u64->i64 wraps")
    d = RNG.standard_normal(1000) * 1e30
    assert_bits_equal(R.cast(d, "f32"), d.astype(np.float32), "f64->f32")


def test_cast_float_to_i64_saturates():
    f = np.array([np.nan, np.inf, -np.inf, 9.3e18, -9.3e18, 2.0**63, -(2.0**63), -1.9, 1.9], np.float64)
    want = np.array([0, 2**63 - 1, -(2**63), 2**63 - 1, -(2**63), 2**63 - 1, -(2**63), -1, 1], np.int64)
    assert_bits_equal(R.cast(f, "i64"), want, "f64->i64 saturating")
    assert_bits_equal(R.cast(f.astype(np.float32), "i64"), want, "f32->i64 saturating")


def _f16_classes():
    xs = [0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 1e9, 6.1035156e-05, 6.0e-08, 5.96e-08, 2.98e-08,
          2.9802322e-08, 1e-30, 0.1, 1 / 3, 2049.0, 2051.0, 1.00048828125, 1.00146484375]
    xs = np.array(xs + [-v for v in xs], np.float32)
    rnd = RNG.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** RNG.integers(-9, 6, 20000).astype(np.float32)
    bits = RNG.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    bits = bits[~np.isnan(bits)]
    return np.concatenate([xs, rnd.astype(np.float32), bits])


def test_f16_matches_numpy():
    x = _f16_classes()
    assert_bits_equal(R.f32_to_f16_bits(x), x.astype(np.float16).view(np.uint16), "f32->f16")


def test_bf16_matches_torch():
    torch = pytest.importorskip("torch")
    x = _f16_classes()
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert_bits_equal(R.f32_to_bf16_bits(x), want, "f32->bf16")


def test_half_nan_rule():
    # quiet NaN, sign and leading payload kept (the convention of the new cast symbols)
    x = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0x7FA12345], np.uint32).view(np.float32)
    assert list(R.f32_to_f16_bits(x)) == [0x7E00, 0xFE00, 0x7E00, 0x7E00 | (0x212345 >> 13) & 0x3FF]
    assert list(R.f32_to_bf16_bits(x)) == [0x7FC0, 0xFFC0, 0x7FC0, 0x7FE1]


# ---- reductions ----
def test_sum_is_sequential():
    # cpu_reduce_typed: acc = 0; acc += x[k] in order -> numpy's add.accumulate ends on the same bits
    x = RNG.standard_normal((7, 3001)).astype(np.float32)
    got = R.reduce(x, "sum", 1)
    want = np.add.accumulate(x, axis=1, dtype=np.float32)[:, -1]
    assert_bits_equal(got, want, "row sums")
    got0 = R.reduce(x, "sum", 0)
    assert_bits_equal(got0, np.add.accumulate(x, axis=0, dtype=np.float32)[-1], "column sums")


def test_sum_close_to_exact():
    x = RNG.standard_normal(100000)
    got = float(R.reduce(x, "sum"))
    exact = math.fsum(x.tolist())
    assert abs(got - exact) <= 1e-12 * np.abs(x).sum()


def test_prod_and_mean():
    x = np.array([[1.0, 2.0], [3.0, 4.0]])
    assert R.reduce(x, "prod", 1).tolist() == [2.0, 12.0]
    assert R.reduce(x, "mean", 1).tolist() == [1.5, 3.5]
    assert float(R.reduce(np.array([1.0, 2.0, 3.0, 4.0]), "mean")) == 2.5
    i = np.array([1, 2, 3, 4], np.int64)
    m = R.reduce(i, "mean")
    assert m.dtype == np.float64 and float(m) == 2.5  # int mean -> f64 (op_builder.rs:2216-2222)
    assert R.reduce(np.array([1, 2, 3], np.int8), "sum").dtype == np.int64


def test_mean_count_saturates_in_f32():
    # count is built by repeated "+1.0f" (op_builder.rs:3608-3612): it stops at 2^24 in f32
    n = 2**24 + 5
    x = np.full(n, 2.0, np.float32)
    m = float(R.reduce(x, "mean"))
    s = float(np.float32(2.0) * np.float32(2**24))  # sequential f32 sum of 2.0 stalls at 2^25
    assert m == s / 2**24


def test_i64_sum_wraps():
    x = np.array([2**63 - 1, 1, 5], np.int64)
    assert int(R.reduce(x, "sum")) == -(2**63) + 5
    assert int(R.reduce(np.array([2**62, 4], np.int64), "prod")) == 0


def test_max_min_arg_semantics():
    # first occurrence wins ties; NaN at k=0 absorbs; later NaN is skipped (op_builder.rs:3543-3578)
    x = np.array([[1.0, 5.0, 5.0, 2.0],
                  [np.nan, 9.0, 1.0, 0.0],
                  [3.0, np.nan, 7.0, 7.0],
                  [-0.0, 0.0, -1.0, 0.0]], np.float32)
    assert R.reduce(x, "argmax", 1).tolist() == [1, 0, 2, 0]
    assert R.reduce(x, "argmin", 1).tolist() == [0, 0, 0, 2]
    mx = R.reduce(x, "max", 1)
    assert mx[0] == 5.0 and np.isnan(mx[1]) and mx[2] == 7.0
    assert np.signbit(mx[3])  # -0.0 seen first, +0.0 is not greater
    assert R.reduce(np.array([[-0.0, 0.0]], np.float32), "min", 1).view(np.uint32)[0] == 0x80000000


def test_arg_matches_numpy_without_nan():
    x = RNG.integers(-3, 4, (50, 60)).astype(np.float64)  # many ties
    for ax in (0, 1):
        assert_bits_equal(R.reduce(x, "argmax", ax), np.argmax(x, axis=ax).astype(np.int64), "argmax")
        assert_bits_equal(R.reduce(x, "argmin", ax), np.argmin(x, axis=ax).astype(np.int64), "argmin")


def test_reference_reduction_literals():
    # tests/python/test_reduction.py:30-110, 165-197 known answers
    a = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    assert float(R.reduce(np.array([1.0, 2.0, 3.0, 4.0], np.float32), "sum")) == 10.0
    assert R.reduce(a, "sum", 0).tolist() == [4.0, 6.0]
    assert R.reduce(a, "sum", -1).tolist() == [3.0, 7.0]
    assert R.reduce(a, "sum", 0, keepdims=True).shape == (1, 2)
    assert float(R.reduce(np.array([3.0, 1.0, 4.0, 1.0, 5.0], np.float32), "max")) == 5.0
    assert R.reduce(np.array([[1.0, 5.0], [3.0, 2.0]], np.float32), "argmin", 0).tolist() == [0, 1]
    assert int(R.reduce(np.array([10, 30, 20], np.int64), "argmax")) == 1


def test_multi_axis_per_axis_structure():
    # reduce_multi reduces the sorted axes one by one (reduction.rs:118-155); for sums that is
    # sum over axis 0 of the column sums
    x = RNG.standard_normal((5, 6, 7)).astype(np.float32)
    got = R.reduce(x, "sum", (0, 2))
    step = np.add.accumulate(x, axis=0, dtype=np.float32)[-1]
    want = np.add.accumulate(step, axis=1, dtype=np.float32)[:, -1]
    assert_bits_equal(got, want, "multi-axis sum")
    # argmax over several axes: index into the flattened reduced axes (NumPy 2 semantics)
    am = R.reduce(x, "argmax", (0, 2))
    flat = x.transpose(1, 0, 2).reshape(6, -1)
    assert_bits_equal(am, np.argmax(flat, axis=1).astype(np.int64), "multi-axis argmax")


def test_complex_reductions_f64_accumulate():
    z = (RNG.standard_normal((3, 50)) + 1j * RNG.standard_normal((3, 50))).astype(np.complex64)
    got = R.reduce(z, "sum", 1)
    want = np.array([complex(math.fsum(r.real.astype(float)), math.fsum(r.imag.astype(float))) for r in z])
    assert np.allclose(got, want.astype(np.complex64), rtol=1e-6, atol=0)
    p = R.reduce(z[:, :5], "prod", 1)
    assert np.allclose(p, np.prod(z[:, :5].astype(np.complex128), axis=1), rtol=1e-6)


# ---- cumsum ----
def test_cumsum_running_equals_literal_and_numpy():
    x = RNG.random((3, 257)).astype(np.float32)
    lit = R.cumsum(x, 1, literal=True)
    run = R.cumsum(x, 1)
    assert_bits_equal(run, lit, "O(L) vs O(L^2)")
    assert_bits_equal(run, np.cumsum(x, axis=1, dtype=np.float32), "vs numpy sequential cumsum")
    assert_bits_equal(R.cumsum(x, 0), np.cumsum(x, axis=0, dtype=np.float32), "axis 0")
    assert_bits_equal(R.cumsum(x.T, None), np.cumsum(x.T.reshape(-1)), "axis=None flattens in C order")
    ones = R.cumsum(np.ones(65537, np.int64), 0)
    assert ones[-1] == 65537 and ones[65535] == 65536  # test_reduction.py:337-364


def test_offset_nd_wraps_negative_strides():
    L = R.lib()
    import ctypes
    shape = (ctypes.c_size_t * 2)(3, 4)
    strides = (ctypes.c_int64 * 2)(-4, 1)
    assert L.oracle_offset_nd(ctypes.c_size_t(5), shape, strides, 2) == -4 + 1
