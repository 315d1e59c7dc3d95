"""The five BASELINE.json configurations at full size, GPU vs the CPU oracle on the same
seeded inputs (numpy default_rng, PCG64).  Bounds as in BASELINE.json north_star:
bit-exact for add/broadcast add/cast/clamp/max/argmax/argmin, <= 2 ulp for exp, and the
condition-aware relative bound (tol * sum|x|) for sum, mean, cumsum and the complex sum."""
import numpy as np
import pytest

import musapy_amd as ms
from oracle import reference as R
from tests.conftest import assert_bits_equal, ulp_diff_f32

pytestmark = pytest.mark.gpu


def dev(x):
    return ms.from_numpy(np.ascontiguousarray(x))


def test_c1_add_f32_16m():
    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, 16_777_216).astype(np.float32)
    b = rng.uniform(-1, 1, 16_777_216).astype(np.float32)
    assert_bits_equal(ms.add(dev(a), dev(b)).numpy(), R.binary("add", a, b), "C1 add")


def test_c2_broadcast_and_transposed_exp():
    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, (4096, 1)).astype(np.float32)
    b = rng.uniform(-1, 1, (8192,)).astype(np.float32)
    assert_bits_equal(ms.add(dev(a), dev(b)).numpy(), R.binary("add", a, b), "C2 broadcast add")
    x = np.random.default_rng(0).uniform(-4, 4, (8192, 4096)).astype(np.float32)
    got = ms.exp(ms.transpose(dev(x))).numpy()
    want = R.unary("exp", x.T)
    assert got.shape == (4096, 8192)
    assert ulp_diff_f32(got, want).max() <= 2


def test_c3_promotion_clamp_casts():
    rng = np.random.default_rng(0)
    a = rng.integers(-1000, 1001, (2048, 2048, 4), dtype=np.int64)
    b = rng.standard_normal((2048, 2048, 4))
    s = ms.add(dev(a), dev(b))
    s_ref = R.binary("add", a, b)
    assert s.dtype == "f64"
    assert_bits_equal(s.numpy(), s_ref, "C3 i64+f64")
    c = ms.clamp(s, -1.0, 1.0)
    c_ref = R.clamp(s_ref, -1.0, 1.0)
    assert_bits_equal(c.numpy(), c_ref, "C3 clamp")
    f = ms.astype(c, "f32")
    f_ref = R.cast(c_ref, "f32")
    assert_bits_equal(f.numpy(), f_ref, "C3 f64->f32")
    assert_bits_equal(ms.astype(f, "bf16").numpy().view(np.uint16), R.f32_to_bf16_bits(f_ref), "C3 f32->bf16")
    assert_bits_equal(ms.astype(f, "f16").numpy().view(np.uint16), R.f32_to_f16_bits(f_ref), "C3 f32->f16")


@pytest.fixture(scope="module")
def c4():
    x = np.random.default_rng(0).standard_normal((8192, 8192), dtype=np.float32)
    return x, dev(x)


@pytest.mark.parametrize("kind,axis", [("sum", -1), ("sum", 0), ("mean", -1), ("mean", 0)])
def test_c4_sum_mean(c4, kind, axis):
    x, X = c4
    got = getattr(ms, kind)(X, axis=axis).numpy()
    want = R.reduce(x, kind, axis)
    scale = np.sum(np.abs(x.astype(np.float64)), axis=axis)
    if kind == "mean":
        scale /= 8192
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= 1e-5 * scale), err.max()
    # also against the exact (f64) sum: a relative bound per element against the sequential CPU
    # sum is not usable, since that sum is itself up to n*eps*sum|x| away from the exact one
    exact = np.sum(x.astype(np.float64), axis=axis) / (8192 if kind == "mean" else 1)
    assert np.max(np.abs(got - exact) / scale) < 1e-6


def test_c4_max_and_args(c4):
    x, X = c4
    assert_bits_equal(ms.max(X, axis=(0, 1)).numpy(), R.reduce(x, "max", (0, 1)), "C4 max (0,1)")
    assert_bits_equal(ms.argmax(X, axis=1).numpy(), R.reduce(x, "argmax", 1), "C4 argmax")
    assert_bits_equal(ms.argmin(X, axis=1).numpy(), R.reduce(x, "argmin", 1), "C4 argmin")


def test_c5_cumsum_and_complex_sum():
    y = np.random.default_rng(0).random((1024, 65536))
    got = ms.cumsum(dev(y), axis=1).numpy()
    want = R.cumsum(y, 1)
    assert np.all(np.abs(got - want) <= 1e-12 * np.abs(want))
    # size-independent properties: prefixes of U(0,1) data never decrease, the last prefix is the row sum
    assert np.all(np.diff(got, axis=1) >= 0)
    assert np.all(np.abs(got[:, -1] - R.reduce(y, "sum", 1)) <= 1e-12 * got[:, -1])
    rng = np.random.default_rng(0)
    re = rng.standard_normal((16, 1024, 1024), dtype=np.float32)
    im = rng.standard_normal((16, 1024, 1024), dtype=np.float32)
    z = (re + 1j * im).astype(np.complex64)
    got = ms.sum(dev(z), axis=(1, 2)).numpy()
    want = R.reduce(z, "sum", (1, 2))
    scale = np.sum(np.abs(z.astype(np.complex128)), axis=(1, 2))
    assert np.all(np.abs(got.astype(np.complex128) - want) <= 1e-5 * scale)
    assert np.all(np.abs(got - want) <= 1e-5 * np.abs(want))
