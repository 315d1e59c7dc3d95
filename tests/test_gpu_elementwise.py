"""GPU parity of the elementwise path (binary / unary / clamp / cast) against the CPU oracle.

Bit-exact for IEEE add/sub/mul/div/abs/neg/sign/clamp and every cast; <= 2 ulp for
sin/cos/exp/log/pow (BASELINE.json north_star bounds).  Layouts cover every kernel variant:
contiguous (vector and misaligned), scalar broadcast, 2-D broadcast, transposed/permuted views
(LDS-tiled path), flipped/sliced strided views, 0-d, single element and empty arrays.
"""
import numpy as np
import pytest

import musapy_amd as ms
from oracle import reference as R
from tests.conftest import assert_bits_equal, ulp_diff_f32, ulp_diff_f64

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(2024)


def dev(x):
    return ms.from_numpy(x)


def check_float(got, want, ulps, what):
    if ulps == 0:
        assert_bits_equal(got, want, what)
        return
    assert got.shape == want.shape and got.dtype == want.dtype, what
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    assert np.array_equal(nan_g, nan_w), f"{what}: NaN pattern differs"
    ok = ~nan_w
    d = ulp_diff_f32(got[ok], want[ok]) if got.dtype == np.float32 else ulp_diff_f64(got[ok], want[ok])
    assert (d.max() if d.size else 0) <= ulps, f"{what}: max ulp {d.max()}"


# views: (name, numpy view function, device view function) applied to a base of shape (12, 20)
def _views():
    return [
        ("contig", lambda x: x, lambda a: a),
        ("transposed", lambda x: x.T, lambda a: ms.transpose(a)),
        ("flipped", lambda x: x[:, ::-1], lambda a: ms.flip(a, 1)),
        ("sliced", lambda x: x[1:11:2, 3:19], lambda a: ms.slice(a, [(1, 11, 2), (3, 19, 1)])),
        ("offset1", lambda x: x.reshape(-1)[1:], None),
    ]


@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "pow"])
def test_binary_layouts(op, dt):
    base_a = RNG.standard_normal((12, 20)).astype(dt)
    base_b = (RNG.standard_normal((12, 20)) + (2.0 if op == "pow" else 0.0)).astype(dt)
    if op == "pow":
        base_a = np.abs(base_a) + dt(0.1)
    A, B = dev(base_a), dev(base_b)
    ulps = 2 if op == "pow" else 0
    for name, nf, df in _views():
        if df is None:
            a1, b1 = base_a.reshape(-1)[1:], base_b.reshape(-1)[:-1]
            got = getattr(ms, op)(ms.slice(ms.from_numpy(base_a.reshape(-1)), [(1, 240, 1)]),
                                  ms.slice(ms.from_numpy(base_b.reshape(-1)), [(0, 239, 1)])).numpy()
            check_float(got, R.binary(op, a1, b1), ulps, f"{op} {name}")
            continue
        got = getattr(ms, op)(df(A), df(B)).numpy()
        check_float(got, R.binary(op, nf(base_a), nf(base_b)), ulps, f"{op} {name}")


@pytest.mark.parametrize("sa,sb", [((4096, 1), (8192,)), ((1,), (1000,)), ((), (33, 7)), ((5, 1, 3), (4, 1)),
                                   ((7, 1), (1, 9)), ((3,), ()), ((1, 1), (1, 1))])
def test_binary_broadcast(sa, sb):
    a = RNG.uniform(-1, 1, sa).astype(np.float32)
    b = RNG.uniform(-1, 1, sb).astype(np.float32)
    got = ms.add(dev(a), dev(b)).numpy()
    assert_bits_equal(got, R.binary("add", a, b), f"broadcast {sa}+{sb}")
    got = ms.div(dev(b), dev(a)).numpy()
    assert_bits_equal(got, R.binary("div", b, a), f"broadcast {sb}/{sa}")


def test_long_broadcast_rows():
    """Long output rows (>= 512 f32 / 256 f64 elements) take the row-piece kernel: ragged row
    lengths, a partial last piece group, the length threshold, f64, reversed and strided operands,
    and comparison / complex outputs through the same launcher."""
    cases = [((300, 1), (1001,), np.float32), ((257, 1), (5000,), np.float32), ((64, 1), (512,), np.float32),
             ((9, 1), (511,), np.float32), ((130, 1), (2049,), np.float64), ((3, 40, 1), (40, 777), np.float32)]
    for sa, sb, dt in cases:
        a = RNG.uniform(-1, 1, sa).astype(dt)
        b = RNG.uniform(-1, 1, sb).astype(dt)
        assert_bits_equal(ms.sub(dev(a), dev(b)).numpy(), R.binary("sub", a, b), f"rows {sa}-{sb} {np.dtype(dt).name}")
        assert_bits_equal(ms.lt(dev(a), dev(b)).numpy(), R.compare("lt", a, b), f"lt rows {sa},{sb}")
    base = RNG.uniform(-1, 1, (200, 3000)).astype(np.float32)
    row = RNG.uniform(-1, 1, (3000,)).astype(np.float32)
    B, Rw = dev(base), dev(row)
    assert_bits_equal(ms.mul(ms.flip(B, 1), Rw).numpy(), R.binary("mul", np.ascontiguousarray(base[:, ::-1]), row),
                      "reversed rows x broadcast row")
    got = ms.add(ms.slice(B, [(0, 200, 1), (0, 3000, 2)]), ms.slice(Rw, [(1, 3000, 2)])).numpy()
    assert_bits_equal(got, R.binary("add", np.ascontiguousarray(base[:, ::2]), np.ascontiguousarray(row[1::2])),
                      "stride-2 rows + stride-2 row")
    z = (RNG.standard_normal((64, 1)) + 1j * RNG.standard_normal((64, 1))).astype(np.complex64)
    w = (RNG.standard_normal(3000) + 1j * RNG.standard_normal(3000)).astype(np.complex64)
    assert_bits_equal(ms.mul(dev(z), dev(w)).numpy(), R.binary("mul", z, w), "c64 broadcast rows", nan_bits=True)


def test_binary_sizes_and_tails():
    for n in (1, 3, 255, 256, 1023, 1024, 1025, 4097, 65537, 1 << 20):
        a = RNG.standard_normal(n).astype(np.float32)
        b = RNG.standard_normal(n).astype(np.float32)
        assert_bits_equal(ms.mul(dev(a), dev(b)).numpy(), a * b, f"mul n={n}")


def test_binary_empty_and_promotion():
    e = ms.add(dev(np.zeros((0, 3), np.float32)), dev(np.zeros((0, 3), np.float32)))
    assert e.shape == (0, 3) and e.numpy().size == 0
    a = np.array([1.5, -2.0], np.float32)
    b = np.array([0.1, 1e-3], np.float64)
    r = ms.add(dev(a), dev(b))
    assert r.dtype == "f32"  # GPU-narrow promotion (dtype.rs:306-334)
    assert_bits_equal(r.numpy(), R.binary("add", a, b), "f32+f64")
    i = np.array([[3, -1000], [7, 2**40]], np.int64)
    f = RNG.standard_normal((2, 2))
    r = ms.add(dev(i), dev(f))
    assert r.dtype == "f64"
    assert_bits_equal(r.numpy(), R.binary("add", i, f), "i64+f64")


MIXED = [(np.int64, np.float64), (np.float64, np.int64), (np.int32, np.float64), (np.float64, np.int32),
         (np.int64, np.float32), (np.float32, np.int64), (np.int32, np.float32), (np.float32, np.int32),
         (np.float64, np.float32), (np.float32, np.float64)]


def _mixed_operand(dt, shape, op):
    if np.issubdtype(dt, np.integer):
        x = RNG.integers(-(2**40) if dt == np.int64 else -(2**30), 2**40 if dt == np.int64 else 2**30, shape)
        if op == "pow":
            x = RNG.integers(0, 4, shape)
        return x.astype(dt)
    x = RNG.standard_normal(shape) * 1e3
    if op == "pow":
        x = np.abs(x) * 1e-3 + 0.5
    return x.astype(dt)


@pytest.mark.parametrize("ta,tb", MIXED)
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "pow"])
def test_binary_mixed_dtypes_fused(op, ta, tb):
    """Promotion fused into the arithmetic pass must give the bits of cast-then-compute
    (dtype.rs:306-334 promotion, op_builder.rs cast then kernel) for every layout."""
    ulps = 2 if op == "pow" else 0
    for n in (1, 7, 1023, 4097, (1 << 16) + 3):
        a, b = _mixed_operand(ta, (n,), op), _mixed_operand(tb, (n,), op)
        got = getattr(ms, op)(dev(a), dev(b)).numpy()
        check_float(got, R.binary(op, a, b), ulps, f"{op} {ta.__name__}+{tb.__name__} n={n}")
    a, b = _mixed_operand(ta, (40, 24), op), _mixed_operand(tb, (24, 40), op)
    got = getattr(ms, op)(dev(a), ms.transpose(dev(b))).numpy()
    check_float(got, R.binary(op, a, np.ascontiguousarray(b.T)), ulps, f"{op} {ta.__name__}+{tb.__name__} T")
    # unaligned start: slice off the first element of both operands
    a, b = _mixed_operand(ta, (1001,), op), _mixed_operand(tb, (1001,), op)
    got = getattr(ms, op)(ms.slice(dev(a), [(1, 1001, 1)]), ms.slice(dev(b), [(1, 1001, 1)])).numpy()
    check_float(got, R.binary(op, a[1:], b[1:]), ulps, f"{op} {ta.__name__}+{tb.__name__} offset")


def test_binary_mixed_broadcast_and_out():
    a = RNG.integers(-1000, 1000, (300, 1)).astype(np.int64)
    b = RNG.standard_normal((300, 257))
    assert_bits_equal(ms.add(dev(a), dev(b)).numpy(), R.binary("add", a, b), "i64 col + f64 broadcast")
    a = RNG.integers(-1000, 1000, (300, 257)).astype(np.int32)
    b = RNG.standard_normal((300, 257)).astype(np.float32)
    out = ms.from_numpy(np.zeros((300, 257), np.float32))
    r = ms.mul(dev(a), dev(b), out=out)
    assert_bits_equal(out.numpy(), R.binary("mul", a, b), "i32*f32 out=")
    assert r.shape == (300, 257)


@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("op", ["sin", "cos", "exp", "log", "abs", "sign", "neg"])
def test_unary_layouts(op, dt):
    base = RNG.uniform(-8, 8, (12, 20)).astype(dt)
    if op == "log":
        base = np.abs(base) + dt(1e-3)
    base[0, :6] = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40 if dt == np.float64 else 1e-40]
    if op == "log":
        base[0, 1] = 0.0
    A = dev(base)
    ulps = 2 if op in ("sin", "cos", "exp", "log") else 0
    for name, nf, df in _views():
        if df is None:
            continue
        got = getattr(ms, op)(df(A)).numpy()
        check_float(got, R.unary(op, nf(base)), ulps, f"{op} {name}")


@pytest.mark.parametrize("op", ["sin", "cos", "exp", "log"])
def test_unary_transcendental_wide_sample(op):
    for dt in (np.float32, np.float64):
        x = RNG.uniform(-100, 100, 1 << 18).astype(dt)
        if op == "log":
            x = np.abs(x) * dt(10.0) ** RNG.integers(-30, 30, x.size).astype(dt)
        got = getattr(ms, op)(dev(x)).numpy()
        check_float(got, R.unary(op, x), 2, f"{op} {dt.__name__}")


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_clamp(dt):
    x = RNG.standard_normal((33, 65)).astype(dt)
    x[0, :3] = [np.nan, -0.0, np.inf]
    for lo, hi in ((-1.0, 1.0), (0.15, 0.3), (-0.0, 0.0)):
        got = ms.clamp(dev(x), lo, hi).numpy()
        assert_bits_equal(got, R.clamp(x, lo, hi), f"clamp {lo},{hi}", nan_bits=True)
        got = ms.clamp(ms.transpose(dev(x)), lo, hi).numpy()
        assert_bits_equal(got, R.clamp(x.T, lo, hi), "clamp transposed", nan_bits=True)


INT_SRC = {"i8": np.int8, "i16": np.int16, "i32": np.int32, "i64": np.int64, "u8": np.uint8, "u16": np.uint16,
           "u32": np.uint32, "u64": np.uint64}


def _int_values(np_t, n):
    info = np.iinfo(np_t)
    edges = np.array([info.min, info.max, 0, 1, info.max - 1, (info.max >> 1) + 1], dtype=np_t)
    return np.concatenate([edges, RNG.integers(info.min, info.max, n, dtype=np_t, endpoint=True)])


@pytest.mark.parametrize("src,dst", [(s, d) for d in ("f32", "f64", "i64") for s in list(INT_SRC) + ["f32", "f64"]
                                     if s != d])  # an identical pair is not a cast
def test_cast_pairs(src, dst):
    if src in INT_SRC:
        x = _int_values(INT_SRC[src], 5000)
    else:
        ft = np.float32 if src == "f32" else np.float64
        x = np.concatenate([np.array([np.nan, np.inf, -np.inf, 9.3e18, -9.3e18, 2.0**63, -(2.0**63), 1e-45, -0.0,
                                      16777217.0, 0.5, 1.5, 2.5, -2.5], ft),
                            (RNG.standard_normal(5000) * 10.0 ** RNG.integers(-40, 40, 5000)).astype(ft)])
    got = ms.astype(dev(x), dst).numpy()
    assert_bits_equal(got, R.cast(x, dst), f"cast {src}->{dst}", nan_bits=True)
    # strided source
    xs = x[: (x.size // 2) * 2].reshape(2, -1).T
    got = ms.astype(ms.transpose(dev(x[: (x.size // 2) * 2].reshape(2, -1))), dst).numpy()
    assert_bits_equal(got, R.cast(xs, dst), f"cast {src}->{dst} transposed", nan_bits=True)


@pytest.mark.parametrize("dst", ["f16", "bf16"])
def test_cast_f32_half_formats(dst):
    bits = RNG.integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    special = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0x7FA12345, 0x477FF000, 0x477FEFFF, 0x33000000,
                        0x33000001, 0x38800000, 0x387FFFFF, 0x7F7FFFFF, 0x00000001, 0x80000000], np.uint32).view(np.float32)
    x = np.concatenate([special, x])
    got = ms.astype(dev(x), dst).numpy().view(np.uint16)
    want = R.f32_to_f16_bits(x) if dst == "f16" else R.f32_to_bf16_bits(x)
    assert_bits_equal(got, want, f"f32->{dst}")


def test_out_and_alias_semantics():
    a, b = dev(np.array([1.0, 2.0, 3.0], np.float32)), dev(np.array([4.0, 5.0, 6.0], np.float32))
    out = dev(np.zeros(3, np.float32))
    r = ms.add(a, b, out=out)
    assert out.tolist() == [5.0, 7.0, 9.0] and r.tolist() == [5.0, 7.0, 9.0]
    with pytest.raises(ms.MemoryError):
        ms.add(a, b, out=a)
    with pytest.raises(ms.ShapeError):
        ms.add(a, dev(np.zeros(2, np.float32)))
    with pytest.raises(ms.DtypeError):
        ms.add(a, b, out=dev(np.zeros(3, np.float64)))
    with pytest.raises(ms.DtypeError):
        ms.sin(dev(np.array([1, 2], np.int64)))
    assert (a + a).tolist() == [2.0, 4.0, 6.0]
    assert ms.array([3.14], dtype="f32").item() == pytest.approx(3.14, abs=1e-6)
    with pytest.raises(ValueError):
        a.item()
