"""The reference's own Python test cases for this path, run against musapy_amd on the GPU.

Inputs and expected values come from the reference's tests (tests/python/test_add.py,
test_elementwise.py, test_reduction.py, test_stream.py); each test names the case it follows.
Where the reference checks its CPU device and its GPU device behaves differently, the GPU rule is
tested and the difference is noted (same-category promotion picks the narrower dtype when every
input is on the GPU, dtype.rs:306-334).  Cases that need operators outside this path (gather,
creation ops) read the result back with numpy instead.
"""
import math

import numpy as np
import pytest

import musapy_amd as ms

pytestmark = pytest.mark.gpu


def approx_list(xs):
    return [pytest.approx(x) for x in xs]


# ---- test_add.py ------------------------------------------------------------------------------
class TestAdd:
    def test_add_f32_and_f64(self):
        assert ms.add(ms.array([1.0, 2.0, 3.0], dtype="f32"), ms.array([4.0, 5.0, 6.0], dtype="f32")).tolist() == [
            5.0, 7.0, 9.0]
        assert ms.add(ms.array([1.0, 2.0], dtype="f64"), ms.array([3.0, 4.0], dtype="f64")).tolist() == [4.0, 6.0]

    def test_add_dunder_self_single_and_new_array(self):
        a, b = ms.array([1.0, 2.0, 3.0], dtype="f32"), ms.array([4.0, 5.0, 6.0], dtype="f32")
        assert (a + b).tolist() == [5.0, 7.0, 9.0]
        assert ms.add(a, a).tolist() == [2.0, 4.0, 6.0]
        assert ms.add(ms.array([1.0]), ms.array([2.0])).tolist() == [3.0]
        c = ms.add(a, b)
        assert a.tolist() == [1.0, 2.0, 3.0] and b.tolist() == [4.0, 5.0, 6.0] and c.tolist() == [5.0, 7.0, 9.0]

    def test_add_out_and_alias(self):
        a, b = ms.array([1.0, 2.0, 3.0], dtype="f32"), ms.array([4.0, 5.0, 6.0], dtype="f32")
        out = ms.array([0.0, 0.0, 0.0], dtype="f32")
        r = ms.add(a, b, out=out)
        assert out.tolist() == [5.0, 7.0, 9.0] and r.tolist() == [5.0, 7.0, 9.0]
        with pytest.raises(ms.MemoryError):
            ms.add(a, b, out=a)
        with pytest.raises(ms.MemoryError):
            ms.add(a, b, out=b)

    def test_shape_and_dtype_mismatch(self):
        with pytest.raises(ms.ShapeError):
            ms.add(ms.array([1.0, 2.0, 3.0]), ms.array([1.0, 2.0]))
        # the reference's CPU case widens to f64; on the GPU both inputs are device arrays and the
        # same-category rule picks the narrower f32
        c = ms.add(ms.array([1.0, 2.0], dtype="f32"), ms.array([3.0, 4.0], dtype="f64"))
        assert c.dtype == "f32" and c.tolist() == [4.0, 6.0]

    def test_readback(self):
        assert ms.array([1.0, 2.0, 3.0], dtype="f32").tolist() == [1.0, 2.0, 3.0]
        assert ms.array([10, 20, 30], dtype="i32").tolist() == [10, 20, 30]
        assert ms.array([], dtype="f32").tolist() == []
        assert abs(ms.array([3.14], dtype="f32").item() - 3.14) < 1e-5
        assert abs(ms.array([2.71828], dtype="f64").item() - 2.71828) < 1e-10
        with pytest.raises(ValueError):
            ms.array([1.0, 2.0]).item()


# ---- test_elementwise.py ----------------------------------------------------------------------
class TestBroadcast:
    def test_broadcast_cases(self):
        c = ms.add(ms.array([[1.0], [2.0], [3.0]]), ms.array([10.0, 20.0, 30.0, 40.0]))
        assert c.shape == (3, 4)
        assert c.tolist() == [[11.0, 21.0, 31.0, 41.0], [12.0, 22.0, 32.0, 42.0], [13.0, 23.0, 33.0, 43.0]]
        c = ms.add(ms.array([[1.0, 2.0, 3.0, 4.0]]), ms.array([[10.0], [20.0], [30.0]]))
        assert c.tolist() == [[11.0, 12.0, 13.0, 14.0], [21.0, 22.0, 23.0, 24.0], [31.0, 32.0, 33.0, 34.0]]
        assert ms.add(ms.array([[1.0, 2.0], [3.0, 4.0]]), ms.array([[10.0, 20.0], [30.0, 40.0]])).tolist() == [
            [11.0, 22.0], [33.0, 44.0]]
        c = ms.add(ms.array(100.0), ms.array([1.0, 2.0, 3.0]))
        assert c.shape == (3,) and c.tolist() == [101.0, 102.0, 103.0]
        c = ms.add(ms.array(10.0), ms.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]))
        assert c.tolist() == [[11.0, 12.0, 13.0], [14.0, 15.0, 16.0]]
        c = ms.add(ms.array(3.0), ms.array(4.0))
        assert c.shape == () and c.item() == 7.0
        c = ms.add(ms.array([[[1.0, 2.0, 3.0]], [[4.0, 5.0, 6.0]]]), ms.array([[10.0], [20.0], [30.0], [40.0]]))
        assert c.shape == (2, 4, 3)
        t = c.tolist()
        assert t[0][0] == [11.0, 12.0, 13.0] and t[0][3] == [41.0, 42.0, 43.0] and t[1][0] == [14.0, 15.0, 16.0]
        c = ms.add(ms.array([100.0]), ms.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]))
        assert c.tolist() == [[101.0, 102.0, 103.0], [104.0, 105.0, 106.0]]
        c = ms.array([[1.0], [2.0], [3.0]]) + ms.array([10.0, 20.0, 30.0, 40.0])
        assert c.tolist()[2] == [13.0, 23.0, 33.0, 43.0]
        c = ms.add(ms.array([[1.0], [2.0]], dtype="f64"), ms.array([0.1, 0.2, 0.3], dtype="f64"))
        assert c.dtype == "f64" and c.tolist()[0] == approx_list([1.1, 1.2, 1.3])
        out = ms.array([[0.0] * 4] * 3)
        r = ms.add(ms.array([[1.0], [2.0], [3.0]]), ms.array([10.0, 20.0, 30.0, 40.0]), out=out)
        assert r.shape == (3, 4) and out.tolist()[1] == [12.0, 22.0, 32.0, 42.0]

    def test_broadcast_errors(self):
        with pytest.raises(ms.ShapeError):
            ms.add(ms.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]), ms.array([1.0, 2.0, 3.0, 4.0]))
        with pytest.raises(ms.ShapeError):
            ms.add(ms.array([1.0, 2.0, 3.0]), ms.array([1.0, 2.0, 3.0, 4.0]))
        with pytest.raises(ms.ShapeError):
            ms.add(ms.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]), ms.array([[1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0]]))
        with pytest.raises(ms.ShapeError):
            ms.add(ms.array([[1.0], [2.0], [3.0]]), ms.array([10.0, 20.0, 30.0, 40.0]), out=ms.array([[0.0, 0.0, 0.0]]))

    def test_broadcast_musa_cases(self):
        c = ms.mul(ms.array([[1.0], [2.0], [3.0]]), ms.array([10.0, 20.0, 30.0, 40.0]))
        assert c.tolist()[0] == [10.0, 20.0, 30.0, 40.0] and c.tolist()[2] == [30.0, 60.0, 90.0, 120.0]
        c = ms.add(ms.array([[1.0], [2.0]]), ms.array([3.0, 4.0, 5.0]))
        assert c.shape == (2, 3) and c.tolist() == [[4.0, 5.0, 6.0], [5.0, 6.0, 7.0]]


class TestBinaryUnaryClamp:
    def test_binary_ops(self):
        assert ms.sub(ms.array([5.0, 3.0, 1.0]), ms.array([1.0, 2.0, 3.0])).tolist() == [4.0, 1.0, -2.0]
        assert ms.mul(ms.array([2.0, 3.0, 4.0]), ms.array([5.0, 6.0, 7.0])).tolist() == [10.0, 18.0, 28.0]
        assert ms.div(ms.array([10.0, 9.0, 8.0]), ms.array([2.0, 3.0, 4.0])).tolist() == [5.0, 3.0, 2.0]
        assert ms.pow(ms.array([2.0, 3.0, 4.0]), ms.array([3.0, 2.0, 0.5])).tolist() == approx_list([8.0, 9.0, 2.0])
        c = ms.sub(ms.array([[10.0], [20.0], [30.0]]), ms.array([1.0, 2.0, 3.0, 4.0]))
        assert c.tolist()[0] == [9.0, 8.0, 7.0, 6.0] and c.tolist()[2] == [29.0, 28.0, 27.0, 26.0]
        c = ms.mul(ms.array(3.0), ms.array([1.0, 2.0, 3.0]))
        assert c.shape == (3,) and c.tolist() == [3.0, 6.0, 9.0]
        out = ms.array([0.0, 0.0, 0.0])
        assert ms.mul(ms.array([1.0, 2.0, 3.0]), ms.array([4.0, 5.0, 6.0]), out=out).tolist() == [4.0, 10.0, 18.0]
        c = ms.add(ms.array([1.0, 2.0], dtype="f64"), ms.array([0.1, 0.2], dtype="f64"))
        assert c.dtype == "f64" and abs(c.tolist()[0] - 1.1) < 1e-10
        a, b = ms.array([6.0, 8.0, 10.0]), ms.array([2.0, 4.0, 5.0])
        assert ms.sub(a, b).tolist() == [4.0, 4.0, 5.0]
        assert ms.mul(a, b).tolist() == [12.0, 32.0, 50.0]
        assert ms.div(a, b).tolist() == [3.0, 2.0, 2.0]
        assert ms.pow(ms.array([2.0, 3.0]), ms.array([4.0, 3.0])).tolist() == approx_list([16.0, 27.0])

    def test_unary_ops(self):
        r = ms.sin(ms.array([0.0, math.pi / 2, math.pi])).tolist()
        assert abs(r[0]) < 1e-6 and abs(r[1] - 1.0) < 1e-6 and abs(r[2]) < 1e-5
        r = ms.cos(ms.array([0.0, math.pi / 2, math.pi])).tolist()
        assert abs(r[0] - 1.0) < 1e-6 and abs(r[1]) < 1e-5 and abs(r[2] + 1.0) < 1e-5
        r = ms.exp(ms.array([0.0, 1.0, 2.0])).tolist()
        assert abs(r[0] - 1.0) < 1e-6 and abs(r[1] - math.e) < 1e-5 and abs(r[2] - math.e ** 2) < 1e-4
        r = ms.log(ms.array([1.0, math.e, math.e ** 2])).tolist()
        assert abs(r[0]) < 1e-6 and abs(r[1] - 1.0) < 1e-5 and abs(r[2] - 2.0) < 1e-5
        assert ms.abs(ms.array([-3.0, 0.0, 5.0])).tolist() == [3.0, 0.0, 5.0]
        assert ms.sign(ms.array([-10.0, 0.0, 7.0])).tolist() == [-1.0, 0.0, 1.0]
        assert ms.neg(ms.array([1.0, -2.0, 0.0])).tolist() == [-1.0, 2.0, 0.0]
        c = ms.abs(ms.array([[-1.0, 2.0], [3.0, -4.0]]))
        assert c.shape == (2, 2) and c.tolist() == [[1.0, 2.0], [3.0, 4.0]]
        out = ms.array([0.0, 0.0, 0.0])
        r = ms.log(ms.array([1.0, 4.0, 9.0]), out=out).tolist()
        assert abs(r[0]) < 1e-6 and abs(r[1] - math.log(4.0)) < 1e-5
        c = ms.exp(ms.array([0.0, 1.0], dtype="f64"))
        assert c.dtype == "f64" and abs(c.tolist()[0] - 1.0) < 1e-12
        a = ms.array([-2.0, 0.0, 3.0])
        assert ms.abs(a).tolist() == [2.0, 0.0, 3.0]
        assert ms.sign(a).tolist() == [-1.0, 0.0, 1.0]
        assert ms.neg(a).tolist() == [2.0, 0.0, -3.0]

    def test_clamp(self):
        assert ms.clamp(ms.array([-5.0, 0.5, 3.0, 10.0]), 0.0, 1.0).tolist() == [0.0, 0.5, 1.0, 1.0]
        assert ms.clamp(ms.array([0.2, 0.5, 0.8]), 0.0, 1.0).tolist() == approx_list([0.2, 0.5, 0.8])
        assert ms.clamp(ms.array([-10.0, -5.0, -1.0]), 0.0, 100.0).tolist() == [0.0, 0.0, 0.0]
        assert ms.clamp(ms.array([[-1.0, 5.0], [0.5, 20.0]]), 0.0, 10.0).tolist() == [[0.0, 5.0], [0.5, 10.0]]
        c = ms.clamp(ms.array([-1.0, 0.5, 2.0], dtype="f64"), 0.0, 1.0)
        assert c.dtype == "f64" and c.tolist() == [0.0, 0.5, 1.0]

    def test_dunders(self):
        assert (ms.array([5.0, 3.0]) - ms.array([1.0, 2.0])).tolist() == [4.0, 1.0]
        assert (ms.array([2.0, 3.0]) * ms.array([4.0, 5.0])).tolist() == [8.0, 15.0]
        assert (ms.array([10.0, 6.0]) / ms.array([2.0, 3.0])).tolist() == [5.0, 2.0]
        assert (ms.array([2.0, 3.0]) ** ms.array([3.0, 2.0])).tolist() == approx_list([8.0, 9.0])
        assert (-ms.array([1.0, -2.0, 0.0])).tolist() == [-1.0, 2.0, 0.0]
        assert abs(ms.array([-3.0, 0.0, 5.0])).tolist() == [3.0, 0.0, 5.0]
        c = ms.array([[1.0], [2.0]]) * ms.array([10.0, 20.0, 30.0])
        assert c.tolist() == [[10.0, 20.0, 30.0], [20.0, 40.0, 60.0]]

    def test_vec4_paths(self):
        """test_vec4_path_correctness / _threshold_boundaries / _unaligned_offset_view / _broadcast."""
        rng = np.random.default_rng(51)
        n = 1_000_000
        x = rng.random(n).astype(np.float32) * 2.0 + 0.5
        y = rng.random(n).astype(np.float32) * 2.0 + 0.5
        a, b = ms.array(x), ms.array(y)
        for op, want in ((ms.add, x + y), (ms.sub, x - y), (ms.mul, x * y), (ms.div, x / y)):
            np.testing.assert_allclose(op(a, b).numpy(), want, rtol=1e-3, atol=1e-3)
        np.testing.assert_allclose(ms.pow(a, b).numpy(), np.power(x, y), rtol=1e-2, atol=1e-2)
        for op, want in ((ms.abs, np.abs(x)), (ms.neg, -x), (ms.exp, np.exp(x)), (ms.log, np.log(x)),
                         (ms.sin, np.sin(x)), (ms.cos, np.cos(x))):
            np.testing.assert_allclose(op(a).numpy(), want, rtol=1e-3, atol=1e-3)
        np.testing.assert_allclose(ms.sign(ms.sub(a, ms.array([0.5]))).numpy(), np.sign(x - 0.5))
        rng = np.random.default_rng(52)
        for n in (999_999, 1_000_001, 1_000_003):
            x = rng.random(n).astype(np.float32)
            np.testing.assert_allclose(ms.exp(ms.array(x)).numpy(), np.exp(x), rtol=1e-3, atol=1e-3)
        x = np.random.default_rng(53).random(1_000_002).astype(np.float32)
        sl = ms.slice(ms.array(x), [[1, 1_000_001, 1]])
        np.testing.assert_allclose(ms.add(sl, sl).numpy(), x[1:1_000_001] * 2, rtol=1e-3, atol=1e-3)


class TestPromotionAndAstype:
    def test_type_promotion(self):
        c = ms.add(ms.array([1, 2, 3], dtype="i64"), ms.array([0.5, 0.5, 0.5], dtype="f64"))
        assert c.dtype == "f64" and c.tolist() == [1.5, 2.5, 3.5]
        c = ms.add(ms.array([1, 2, 3], dtype="i32"), ms.array([0.5, 0.5, 0.5], dtype="f32"))
        assert c.dtype == "f32" and abs(c.tolist()[0] - 1.5) < 1e-6
        c = ms.add(ms.array([1, 2, 3], dtype="i64"), ms.array([0.5, 0.5, 0.5], dtype="f32"))
        assert c.dtype == "f32" and abs(c.tolist()[0] - 1.5) < 1e-6
        # test_f32_plus_f64 (CPU: f64); both on the GPU: the narrower f32
        assert ms.add(ms.array([1.0, 2.0], dtype="f32"), ms.array([0.1, 0.2], dtype="f64")).dtype == "f32"
        c = ms.add(ms.array([1.0, 2.0], dtype="f32"), ms.array([3.0, 4.0], dtype="f32"))
        assert c.dtype == "f32" and c.tolist() == [4.0, 6.0]
        c = ms.sub(ms.array([10, 20], dtype="i64"), ms.array([0.5, 1.5], dtype="f64"))
        assert c.dtype == "f64" and c.tolist() == [9.5, 18.5]
        f = ms.mul(ms.array([2, 3], dtype="i64"), ms.array([1.5, 2.5], dtype="f64"))
        assert f.dtype == "f64" and f.tolist() == [3.0, 7.5]

    def test_astype(self):
        b = ms.array([1.0, 2.0, 3.0], dtype="f32").astype("f64")
        assert b.dtype == "f64" and b.tolist() == [1.0, 2.0, 3.0]
        b = ms.array([1.5, 2.5], dtype="f64").astype("f32")
        assert b.dtype == "f32" and abs(b.tolist()[0] - 1.5) < 1e-6
        b = ms.array([1, 2, 3], dtype="i64").astype("f32")
        assert b.dtype == "f32" and b.tolist() == [1.0, 2.0, 3.0]
        b = ms.array([10, 20], dtype="i32").astype("f64")
        assert b.dtype == "f64" and b.tolist() == [10.0, 20.0]
        b = ms.array([[1.0, 2.0], [3.0, 4.0]], dtype="f32").astype("f64")
        assert b.shape == (2, 2) and b.tolist() == [[1.0, 2.0], [3.0, 4.0]]
        a = ms.array([1.0, 2.0], dtype="f32")
        b = a.astype("f32")
        assert b.dtype == "f32" and b.tolist() == [1.0, 2.0] and b.data_ptr != a.data_ptr
        b = ms.array([1.7, -2.9, 3.0], dtype="f32").astype("i64")
        assert b.dtype == "i64" and b.tolist() == [1, -2, 3]
        b = ms.array([1.7, 2.9, -0.9], dtype="f64").astype("i64")
        assert b.tolist() == [1, 2, 0]
        for src, dst in (("c64", "f64"), ("c64", "f32"), ("c128", "f64"), ("c128", "f32")):
            with pytest.raises(ms.DtypeError):
                ms.array([1 + 2j], dtype=src).astype(dst)
        y = ms.array([1 + 2j, 3 - 4j], dtype="c64").astype("c128")
        assert y.dtype == "c128" and y.tolist() == [1 + 2j, 3 - 4j]


# ---- test_reduction.py ------------------------------------------------------------------------
class TestReductions:
    def test_basic(self):
        m = ms.array([[1.0, 2.0], [3.0, 4.0]])
        assert ms.sum(ms.array([1.0, 2.0, 3.0, 4.0])).item() == pytest.approx(10.0)
        assert ms.sum(m, axis=0).tolist() == approx_list([4.0, 6.0])
        assert ms.sum(m, axis=1).tolist() == approx_list([3.0, 7.0])
        r = ms.sum(m, axis=0, keepdims=True)
        assert r.shape == (1, 2) and r.tolist() == [approx_list([4.0, 6.0])]
        assert ms.sum(m, axis=-1).tolist() == approx_list([3.0, 7.0])
        assert ms.prod(ms.array([1.0, 2.0, 3.0, 4.0])).item() == pytest.approx(24.0)
        assert ms.prod(m, axis=1).tolist() == approx_list([2.0, 12.0])
        assert ms.max(ms.array([3.0, 1.0, 4.0, 1.0, 5.0])).item() == pytest.approx(5.0)
        assert ms.max(ms.array([[1.0, 5.0], [3.0, 2.0]]), axis=0).tolist() == approx_list([3.0, 5.0])
        assert ms.min(ms.array([3.0, 1.0, 4.0, 1.0, 5.0])).item() == pytest.approx(1.0)
        assert ms.min(ms.array([[1.0, 5.0], [3.0, 2.0]]), axis=1).tolist() == approx_list([1.0, 2.0])
        assert ms.mean(ms.array([1.0, 2.0, 3.0, 4.0])).item() == pytest.approx(2.5)
        assert ms.mean(m, axis=1).tolist() == approx_list([1.5, 3.5])
        r = ms.mean(m, axis=0, keepdims=True)
        assert r.shape == (1, 2) and r.tolist() == [approx_list([2.0, 3.0])]
        r = ms.sum(ms.array([5.0]))
        assert r.shape == () and r.item() == pytest.approx(5.0)
        assert ms.sum(m).item() == pytest.approx(10.0)
        assert ms.argmax(m, axis=1).tolist() == [1, 1]
        assert ms.mean(ms.array([2.0, 4.0, 6.0, 8.0])).item() == pytest.approx(5.0)
        assert ms.max(ms.array([[1.0, 5.0], [3.0, 2.0]]), axis=1).tolist() == approx_list([5.0, 3.0])
        assert ms.prod(ms.array([2.0, 3.0, 4.0])).item() == pytest.approx(24.0)

    def test_accumulation_dtypes(self):
        r = ms.sum(ms.array([1, 2, 3], dtype="i64"))
        assert r.dtype == "i64" and r.item() == 6
        r = ms.sum(ms.array([1, 2, 3], dtype="i8"))
        assert r.dtype == "i64" and r.item() == 6
        r = ms.mean(ms.array([1, 2, 3, 4], dtype="i64"))
        assert r.dtype == "f64" and r.item() == pytest.approx(2.5)
        assert ms.mean(ms.array([1.0, 2.0, 3.0], dtype="f32")).dtype == "f32"
        r = ms.max(ms.array([3, 1, 4], dtype="i64"))
        assert r.dtype == "i64" and r.item() == 4
        assert ms.sum(ms.array([1.0, 2.0, 3.0], dtype="f32")).dtype == "f32"

    def test_arg_reductions(self):
        r = ms.argmax(ms.array([1.0, 5.0, 3.0, 2.0]))
        assert r.item() == 1 and r.dtype == "i64"
        assert ms.argmin(ms.array([3.0, 1.0, 4.0, 0.5])).item() == 3
        assert ms.argmax(ms.array([[1.0, 5.0], [3.0, 2.0]]), axis=1).tolist() == [1, 0]
        assert ms.argmin(ms.array([[1.0, 5.0], [3.0, 2.0]]), axis=0).tolist() == [0, 1]
        assert ms.argmax(ms.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]), axis=1).shape == (2,)
        assert ms.argmax(ms.array([10, 30, 20], dtype="i64")).item() == 1

    def test_cumsum(self):
        assert ms.cumsum(ms.array([1.0, 2.0, 3.0, 4.0]), axis=0).tolist() == approx_list([1.0, 3.0, 6.0, 10.0])
        r = ms.cumsum(ms.array([[1.0, 2.0], [3.0, 4.0]]))
        assert r.shape == (4,) and r.tolist() == approx_list([1.0, 3.0, 6.0, 10.0])
        r = ms.cumsum(ms.array([[1.0, 2.0], [3.0, 4.0]]), axis=0)
        assert r.shape == (2, 2) and r.tolist() == [approx_list([1.0, 2.0]), approx_list([4.0, 6.0])]
        r = ms.cumsum(ms.array([[1.0, 2.0], [3.0, 4.0]]), axis=1)
        assert r.tolist() == [approx_list([1.0, 3.0]), approx_list([3.0, 7.0])]
        r = ms.cumsum(ms.array([1, 2, 3], dtype="i64"), axis=0)
        assert r.dtype == "i64" and r.tolist() == [1, 3, 6]
        assert ms.cumsum(ms.array([1.0, 2.0, 3.0]), axis=0).tolist() == approx_list([1.0, 3.0, 6.0])

    @pytest.mark.parametrize("n,probe", [(65536, [65535]), (65537, [65536]), (1_000_000, [65535, 65536, 999_999])])
    def test_cumsum_long_axes_of_ones(self, n, probe):
        r = ms.cumsum(ms.ones(n, dtype="i64"), axis=0)
        assert ms.sum(r).item() == n * (n + 1) // 2
        assert [int(v) for v in r.numpy()[probe]] == [p + 1 for p in probe]

    def test_cumsum_random_long_axes(self):
        data = np.random.default_rng(42).random(100000, dtype=np.float32)
        assert np.allclose(ms.cumsum(ms.array(data), axis=0).numpy(), np.cumsum(data), rtol=1e-3, atol=1e-3)
        data = np.random.default_rng(43).random(100000, dtype=np.float64)
        assert np.allclose(ms.cumsum(ms.array(data, dtype="f64"), axis=0).numpy(), np.cumsum(data), rtol=1e-9,
                           atol=1e-9)
        data = np.random.default_rng(7).random((3, 70000), dtype=np.float32)
        got = ms.cumsum(ms.array(data), axis=1).numpy()
        assert got.shape == (3, 70000) and np.allclose(got, np.cumsum(data, axis=1), rtol=1e-3, atol=1e-3)
        for n in (1300, 1537):
            data = np.random.default_rng(n).random(n, dtype=np.float32)
            assert np.allclose(ms.cumsum(ms.array(data), axis=0).numpy(), np.cumsum(data), rtol=1e-3, atol=1e-3)
        with pytest.raises(Exception):
            ms.cumsum(ms.ones(256 ** 3 + 1, dtype="f32"), axis=0)

    def test_errors(self):
        a = ms.array([1.0, 2.0, 3.0])
        with pytest.raises(Exception):
            ms.sum(a, axis=5)
        with pytest.raises(Exception):
            ms.sum(a, axis=-4)
        with pytest.raises(Exception):
            ms.sum(ms.array([[1.0, 2.0], [3.0, 4.0]]), axis=0, out=ms.array([0.0, 0.0, 0.0]))
        with pytest.raises(Exception):
            ms.sum(a, axis=0, out=ms.array([0, 0], dtype="i64"))

    def test_small_axis_and_partial_paths(self):
        rng = np.random.default_rng(7)
        data = rng.random((256, 256), dtype=np.float32)
        a = ms.array(data)
        for op, ref in ((ms.sum, np.sum), (ms.max, np.max), (ms.min, np.min), (ms.prod, np.prod), (ms.mean, np.mean)):
            for ax in (0, 1):
                np.testing.assert_allclose(op(a, axis=ax).numpy(), ref(data, axis=ax), rtol=1e-5, atol=1e-5)
        rng = np.random.default_rng(8)
        for r, c in ((100, 17), (33, 33), (129, 129), (7, 1024), (1025, 5)):
            data = rng.random((r, c), dtype=np.float32)
            a = ms.array(data)
            for op, ref in ((ms.sum, np.sum), (ms.max, np.max), (ms.min, np.min), (ms.mean, np.mean)):
                for ax in (0, 1):
                    np.testing.assert_allclose(op(a, axis=ax).numpy(), ref(data, axis=ax), rtol=1e-5, atol=1e-5)
        data = np.random.default_rng(9).integers(-1000, 1000, (256, 256))
        a = ms.array(data, dtype="i64")
        for op, ref in ((ms.sum, np.sum), (ms.prod, np.prod), (ms.max, np.max), (ms.min, np.min)):
            for ax in (0, 1):
                assert op(a, axis=ax).tolist() == ref(data, axis=ax).tolist()
        data = np.random.default_rng(10).random(1_000_000, dtype=np.float32)
        a = ms.array(data)
        for op, ref in ((ms.sum, np.sum), (ms.max, np.max), (ms.min, np.min), (ms.mean, np.mean), (ms.prod, np.prod)):
            np.testing.assert_allclose(op(a).numpy(), ref(data), rtol=1e-5, atol=1e-5)
        data = np.random.default_rng(11).random((5000, 3), dtype=np.float32)
        a = ms.array(data)
        for op, ref in ((ms.sum, np.sum), (ms.max, np.max), (ms.min, np.min)):
            for ax in (0, 1):
                np.testing.assert_allclose(op(a, axis=ax).numpy(), ref(data, axis=ax), rtol=1e-5, atol=1e-5)
        base = np.random.default_rng(12).random((64, 64), dtype=np.float32)
        fv = ms.flip(ms.array(base), 1)
        for op, ref in ((ms.sum, np.sum), (ms.max, np.max), (ms.min, np.min)):
            for ax in (0, 1):
                np.testing.assert_allclose(op(fv, axis=ax).numpy(), ref(base[:, ::-1], axis=ax), rtol=1e-5, atol=1e-5)

    @pytest.mark.parametrize("dtype", ["f32", "f64"])
    @pytest.mark.parametrize("axes", [(0, 1), (1, 2), (0, 2), (0, 1, 2), (-1, 0)])
    def test_multi_axis(self, dtype, axes):
        data = np.random.default_rng(21).normal(size=(2, 3, 4)).astype(np.float32 if dtype == "f32" else np.float64)
        tol = 1e-4 if dtype == "f32" else 1e-10
        x = ms.array(data, dtype=dtype)
        for name in ("sum", "mean", "prod", "max", "min"):
            for keep in (False, True):
                got = getattr(ms, name)(x, axis=axes, keepdims=keep).numpy()
                assert np.allclose(got, getattr(np, name)(data, axis=axes, keepdims=keep), rtol=tol, atol=tol)
        data = np.random.default_rng(22).normal(size=(2, 3, 4))
        norm = tuple(sorted(ax % 3 for ax in axes))
        perm = [i for i in range(3) if i not in norm] + list(norm)
        t = data.transpose(perm)
        want = np.argmax(t.reshape(t.shape[: 3 - len(norm)] + (-1,)), axis=-1)
        assert np.array_equal(ms.argmax(ms.array(data, dtype="f64"), axis=axes).numpy(), want)

    def test_multi_axis_keepdims_and_errors(self):
        data = np.random.default_rng(23).normal(size=(2, 3, 4))
        got = ms.argmax(ms.array(data, dtype="f64"), axis=(0, 1), keepdims=True)
        assert got.shape == (1, 1, 4)
        want = np.argmax(data.transpose(2, 0, 1).reshape(4, -1), axis=-1).reshape(1, 1, 4)
        assert np.array_equal(got.numpy(), want)
        x = ms.array(np.zeros((2, 3, 4)), dtype="f64")
        with pytest.raises(ms.ShapeError):
            ms.sum(x, axis=(0, 0))
        with pytest.raises(ms.ShapeError):
            ms.sum(x, axis=(0, 5))
        with pytest.raises(ms.ShapeError):
            ms.sum(ms.array(np.zeros((2, 3)), dtype="f64"), axis=(0, 1), out=ms.array(np.zeros(2), dtype="f64"))

    @pytest.mark.parametrize("dtype", ["c64", "c128"])
    def test_complex(self, dtype):
        rng = np.random.default_rng(24)
        data = (rng.normal(size=(3, 4)) + 1j * rng.normal(size=(3, 4))).astype(
            np.complex64 if dtype == "c64" else np.complex128)
        tol = 1e-4 if dtype == "c64" else 1e-10
        x = ms.array(data, dtype=dtype)
        for axes in (None, 0, 1, (0, 1), -1):
            for name in ("sum", "mean", "prod"):
                got = getattr(ms, name)(x, axis=axes).numpy()
                assert np.allclose(got, getattr(np, name)(data, axis=axes), rtol=tol, atol=tol)
        y = ms.array([1 + 2j, 3 + 4j], dtype="c128")
        for f in (ms.max, ms.min, ms.argmax, ms.argmin):
            with pytest.raises(ms.DtypeError):
                f(y)


# ---- test_stream.py ---------------------------------------------------------------------------
class TestStreams:
    def test_two_streams_and_cross_stream_ops(self):
        s1, s2 = ms.Stream("musa:0"), ms.Stream("musa:0")
        with ms.stream(s1):
            a = ms.array([1.0, 2.0, 3.0], dtype="f32")
        with ms.stream(s2):
            b = ms.array([4.0, 5.0, 6.0], dtype="f32")
        s1.synchronize()
        s2.synchronize()
        assert a.tolist() == [1.0, 2.0, 3.0] and b.tolist() == [4.0, 5.0, 6.0]
        with ms.stream(s2):
            c = ms.add(a, b)
            out = ms.array([0.0, 0.0, 0.0], dtype="f32")
            r = ms.add(a, b, out=out)
        s2.synchronize()
        assert c.tolist() == [5.0, 7.0, 9.0] and out.tolist() == [5.0, 7.0, 9.0] and r.tolist() == [5.0, 7.0, 9.0]

    def test_interleaved_many_and_reuse(self):
        s1, s2 = ms.Stream("hip:0"), ms.Stream("hip:0")
        with ms.stream(s1):
            a1 = ms.array([1.0, 2.0], dtype="f32")
        with ms.stream(s2):
            b1 = ms.array([3.0, 4.0], dtype="f32")
        with ms.stream(s1):
            c1 = ms.add(a1, a1)
        with ms.stream(s2):
            d1 = ms.add(b1, b1)
        with ms.stream(s1):
            e1 = ms.add(c1, a1)
        with ms.stream(s2):
            f1 = ms.add(d1, b1)
        s1.synchronize()
        s2.synchronize()
        assert (c1.tolist(), d1.tolist(), e1.tolist(), f1.tolist()) == ([2.0, 4.0], [6.0, 8.0], [3.0, 6.0], [9.0, 12.0])
        streams = [ms.Stream() for _ in range(4)]
        arrays = []
        for i, s in enumerate(streams):
            with ms.stream(s):
                arrays.append(ms.array([float(i), float(i + 1)], dtype="f32"))
        for s in streams:
            s.synchronize()
        assert [x.tolist() for x in arrays] == [[float(i), float(i + 1)] for i in range(4)]
        s = ms.Stream()
        with ms.stream(s):
            b = ms.add(ms.array([1.0, 2.0]), ms.array([1.0, 2.0]))
        s.synchronize()
        assert b.tolist() == [2.0, 4.0]
        with ms.stream(s):
            c = ms.add(b, b)
        s.synchronize()
        assert c.tolist() == [4.0, 8.0]

    def test_stream_synchronize_pending_count(self):
        """test_acceptance_v03.py:112-116: an explicit synchronize leaves nothing pending."""
        s = ms.Stream("musa:0")
        s.synchronize()
        assert s.pending_count == 0


# ---- test_debug_summary.py (TestDebugMode) ----------------------------------------------------
class TestDebugMode:
    """test_debug_summary.py:95-156, on the GPU device instead of the reference's CPU device."""

    def test_set_debug_true_and_false(self):
        ms.set_debug(True)
        try:
            s = ms.Stream()
            with ms.stream(s):
                c = ms.add(ms.array([1.0, 2.0], dtype="f32"), ms.array([3.0, 4.0], dtype="f32"))
            assert s.pending_count == 1  # the add's OpContext (debug mode only)
            assert c.tolist() == [4.0, 6.0]
            assert s.pending_count == 0  # the readback's synchronize cleared it
        finally:
            ms.set_debug(False)
        c = ms.add(ms.array([1.0], dtype="f32"), ms.array([2.0], dtype="f32"))
        assert c.tolist() == [3.0]

    def test_debug_context_manager_nested(self):
        ms.set_debug(False)
        with ms.debug():
            with ms.debug():
                c = ms.array([1.0], dtype="f32") + ms.array([2.0], dtype="f32")
                assert c.tolist() == [3.0]
            c = ms.array([1.0], dtype="f32") + ms.array([2.0], dtype="f32")
            assert c.tolist() == [3.0]
            assert ms._core._is_debug()
        assert not ms._core._is_debug()
        a, b = ms.array([1.0, 2.0, 3.0], dtype="f32"), ms.array([4.0, 5.0, 6.0], dtype="f32")
        assert (a + b).tolist() == [5.0, 7.0, 9.0]
