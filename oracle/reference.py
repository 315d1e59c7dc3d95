"""Op-level CPU oracle: musapy's reference semantics for the elementwise + reduction path.

TEST INFRASTRUCTURE ONLY -- imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product (musapy_amd).

The arithmetic runs in oracle/liboracle.so (a C restatement of the reference's `cpu_*`
functions, see oracle.c).  This module restates the host-side control flow around it, for an
array that lives on the accelerator device (so promotion uses the GPU-narrow rule):
  promote                rust/musapy-core/src/dtype.rs:206-334
  broadcast shape/strides rust/musapy-ops/src/broadcast.rs:24-92
  binary/unary/clamp     rust/musapy-ops/src/op_builder.rs:315-532, 550-732, 740-891
  comparisons            op_builder.rs:1338-1557 (output bool; complex eq/ne only)
  cast validation        op_builder.rs:904-962 (+ the new f32 -> f16/bf16 pairs)
  reduction_axis         op_builder.rs:2310-3139 (compute dtype 2209-2225, axis=None -> 1-D)
  reduce_multi / arg_reduce_multi / resolve_axes   rust/musapy-ops/src/reduction.rs:21-226
  cumsum_op              op_builder.rs:3144-3363
  contiguous             rust/musapy-ops/src/indexing.rs:181-237 (copy_into 816-916)
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

BIN = {"add": 0, "sub": 1, "mul": 2, "div": 3, "pow": 4}
UN = {"sin": 0, "cos": 1, "exp": 2, "log": 3, "abs": 4, "sign": 5, "neg": 6}
CMP = {"eq": 0, "ne": 1, "lt": 2, "gt": 3, "le": 4, "ge": 5}
RED = {"sum": 0, "prod": 1, "max": 2, "min": 3, "mean": 4, "argmax": 5, "argmin": 6}
TCODE = {"i8": 0, "i16": 1, "i32": 2, "i64": 3, "u8": 4, "u16": 5, "u32": 6, "u64": 7, "f32": 8, "f64": 9,
         "c64": 10, "c128": 11}
NP = {"bool": np.bool_, "i8": np.int8, "i16": np.int16, "i32": np.int32, "i64": np.int64, "u8": np.uint8,
      "u16": np.uint16, "u32": np.uint32, "u64": np.uint64, "f16": np.float16, "f32": np.float32,
      "f64": np.float64, "bf16": np.uint16, "c64": np.complex64, "c128": np.complex128}
_FROM_NP = {np.dtype(v).name: k for k, v in NP.items() if k != "bf16"}


class OracleError(Exception):
    """A case the reference rejects (its DtypeError / ShapeError)."""


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            import subprocess

            subprocess.run(["make", "-s", "-C", HERE], check=True)
        _LIB = ctypes.CDLL(path)
        _LIB.oracle_f32_to_f16.restype = ctypes.c_uint16
        _LIB.oracle_f32_to_bf16.restype = ctypes.c_uint16
        _LIB.oracle_offset_nd.restype = ctypes.c_int64
    return _LIB


def dtype_of(x: np.ndarray) -> str:
    return _FROM_NP[x.dtype.name]


# ---------------------------------------------------------------------------------------------
# dtype.rs restated
_CAT = {"bool": 0, "i8": 1, "i16": 1, "i32": 1, "i64": 1, "u8": 2, "u16": 2, "u32": 2, "u64": 2,
        "f16": 3, "f32": 3, "f64": 3, "bf16": 3, "c64": 4, "c128": 4}
_W = {"bool": 8, "i8": 8, "u8": 8, "i16": 16, "u16": 16, "f16": 16, "bf16": 16, "i32": 32, "u32": 32,
      "f32": 32, "c64": 32, "i64": 64, "u64": 64, "f64": 64, "c128": 64}


def _jax(a, b):
    if a == b:
        return a
    if a == "bool":
        return b
    if b == "bool":
        return a
    ca, pa, cb, pb = _CAT[a], _W[a], _CAT[b], _W[b]
    if ca == cb:
        if ca == 3 and pa == pb:
            return "f32"
        return a if pa >= pb else b
    if {ca, cb} == {1, 2}:
        iw, uw = (pa, pb) if ca == 1 else (pb, pa)
        return {8: "i8", 16: "i16", 32: "i32", 64: "i64"}[iw if iw > uw else min(uw * 2, 64)]
    if ca in (1, 2) and cb == 3:
        return b
    if cb in (1, 2) and ca == 3:
        return a
    if ca in (1, 2) and cb == 4:
        return "c64" if max(pa, pb, 32) == 32 else "c128"
    if cb in (1, 2) and ca == 4:
        return "c64" if max(pa, pb, 32) == 32 else "c128"
    return "c64" if max(pa, pb) == 32 else "c128"


def promote(a: str, b: str, all_gpu: bool) -> str:
    if a == b:
        return a
    j = _jax(a, b)
    if not all_gpu or _CAT[a] != _CAT[b]:
        return j
    if _CAT[a] == 3 and _W[a] == _W[b] and {a, b} == {"f16", "bf16"}:
        return j
    return a if _W[a] <= _W[b] else b


# ---------------------------------------------------------------------------------------------
def broadcast_shape(*shapes):
    nd = max((len(s) for s in shapes), default=0)
    r = [1] * nd
    for s in shapes:
        off = nd - len(s)
        for i, d in enumerate(s):
            if r[off + i] == 1:
                r[off + i] = d
            elif d != 1 and d != r[off + i]:
                raise OracleError(f"broadcast: incompatible shapes {shapes}")
    return tuple(r)


def _bstrides(x: np.ndarray, target):
    st = [s // x.itemsize for s in x.strides]
    r = [0] * len(target)
    off = len(target) - x.ndim
    for i in range(x.ndim):
        if x.shape[i] == target[off + i]:
            r[off + i] = st[i]
    return r


def _estrides(x: np.ndarray):
    return [s // x.itemsize for s in x.strides]


def _c(arr, t):
    return (t * len(arr))(*arr)


def _ptr(x: np.ndarray):
    return ctypes.c_void_p(x.__array_interface__["data"][0])


# ---------------------------------------------------------------------------------------------
def validate_cast(src: str, dst: str):
    """validate_cast_pair, op_builder.rs:904-962 (+ the new f32 -> f16/bf16 pairs)."""
    if src == "f32" and dst in ("f16", "bf16"):
        return
    if src in ("c64", "c128"):
        if src == "c64" and dst == "c128":
            return
        raise OracleError(f"cast {src} -> {dst}")
    if src not in ("i8", "i16", "i32", "i64", "u8", "u16", "u32", "u64", "f32", "f64"):
        raise OracleError(f"cast source {src}")
    if dst not in ("f32", "f64", "i64", "c64", "c128"):
        raise OracleError(f"cast target {dst}")
    if dst in ("c64", "c128") and src not in ("f32", "f64"):
        raise OracleError(f"cast {src} -> {dst}")
    if src == dst:
        raise OracleError("identical cast")


def cast(x: np.ndarray, dst: str) -> np.ndarray:
    """cast_array / astype for a differing dtype: output is C-contiguous (op_builder.rs:1055-1119)."""
    src = dtype_of(x)
    validate_cast(src, dst)
    out = np.empty(x.shape, dtype=NP[dst])
    shp, st = _c(x.shape, ctypes.c_size_t), _c(_estrides(x), ctypes.c_int64)
    L = lib()
    if dst == "f16":
        L.oracle_cast_f32_f16(_ptr(x), _ptr(out), x.ndim, shp, st)
    elif dst == "bf16":
        L.oracle_cast_f32_bf16(_ptr(x), _ptr(out), x.ndim, shp, st)
    else:
        L.oracle_cast(TCODE[src], TCODE[dst], _ptr(x), _ptr(out), x.ndim, shp, st)
    return out


def binary(op: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    shape = broadcast_shape(a.shape, b.shape)
    dt = promote(dtype_of(a), dtype_of(b), True)
    if dt in ("c64", "c128") and op == "pow":
        raise OracleError(f"{op}: complex pow")
    if dt not in ("f32", "f64", "c64", "c128"):
        raise OracleError(f"{op}: promoted dtype {dt}")
    aw = a if dtype_of(a) == dt else cast(a, dt)
    bw = b if dtype_of(b) == dt else cast(b, dt)
    out = np.empty(shape, dtype=NP[dt])
    if out.size:
        ast = _estrides(aw) if aw.shape == shape else _bstrides(aw, shape)
        bst = _estrides(bw) if bw.shape == shape else _bstrides(bw, shape)
        args = (_ptr(aw), _ptr(bw), _ptr(out), len(shape), _c(shape, ctypes.c_size_t), _c(ast, ctypes.c_int64),
                _c(bst, ctypes.c_int64))
        if dt in ("c64", "c128"):
            lib().oracle_binary_cplx(BIN[op], TCODE[dt], *args)
        else:
            f = lib().oracle_binary_f32 if dt == "f32" else lib().oracle_binary_f64
            f(BIN[op], *args)
    return out


def compare(op: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """comparison_elementwise: promote for the kernel only, bool output (op_builder.rs:1338-1557)."""
    shape = broadcast_shape(a.shape, b.shape)
    dt = promote(dtype_of(a), dtype_of(b), True)
    if dt in ("c64", "c128") and op not in ("eq", "ne"):
        raise OracleError(f"{op}: complex ordering")
    if dt not in ("f32", "f64", "c64", "c128"):
        raise OracleError(f"{op}: promoted dtype {dt}")
    aw = a if dtype_of(a) == dt else cast(a, dt)
    bw = b if dtype_of(b) == dt else cast(b, dt)
    out = np.zeros(shape, dtype=np.uint8)
    if out.size:
        ast = _estrides(aw) if aw.shape == shape else _bstrides(aw, shape)
        bst = _estrides(bw) if bw.shape == shape else _bstrides(bw, shape)
        lib().oracle_compare(CMP[op], TCODE[dt], _ptr(aw), _ptr(bw), _ptr(out), len(shape),
                             _c(shape, ctypes.c_size_t), _c(ast, ctypes.c_int64), _c(bst, ctypes.c_int64))
    return out.view(np.bool_)


def unary(op: str, a: np.ndarray) -> np.ndarray:
    dt = dtype_of(a)
    if dt in ("c64", "c128"):
        if op not in ("neg", "abs"):
            raise OracleError(f"{op}: complex")
        odt = ("f32" if dt == "c64" else "f64") if op == "abs" else dt
        out = np.empty(a.shape, dtype=NP[odt])
        if out.size:
            lib().oracle_unary_cplx(UN[op], TCODE[dt], _ptr(a), _ptr(out), a.ndim, _c(a.shape, ctypes.c_size_t),
                                    _c(_estrides(a), ctypes.c_int64))
        return out
    if dt not in ("f32", "f64"):
        raise OracleError(f"{op}: dtype {dt}")
    out = np.empty(a.shape, dtype=NP[dt])
    if out.size:
        f = lib().oracle_unary_f32 if dt == "f32" else lib().oracle_unary_f64
        f(UN[op], _ptr(a), _ptr(out), a.ndim, _c(a.shape, ctypes.c_size_t), _c(_estrides(a), ctypes.c_int64))
    return out


def clamp(a: np.ndarray, lo: float, hi: float) -> np.ndarray:
    dt = dtype_of(a)
    if dt not in ("f32", "f64"):
        raise OracleError(f"clamp: dtype {dt}")
    out = np.empty(a.shape, dtype=NP[dt])
    if out.size:
        f = lib().oracle_clamp_f32 if dt == "f32" else lib().oracle_clamp_f64
        f(_ptr(a), _ptr(out), ctypes.c_double(lo), ctypes.c_double(hi), a.ndim, _c(a.shape, ctypes.c_size_t),
          _c(_estrides(a), ctypes.c_int64))
    return out


# ---------------------------------------------------------------------------------------------
def resolve_axes(axis, ndim):
    if axis is None:
        return []
    axs = list(axis) if isinstance(axis, (tuple, list)) else [axis]
    out = []
    for ax in axs:
        n = ax + ndim if ax < 0 else ax
        if n < 0 or n >= ndim:
            raise OracleError(f"axis {ax} out of bounds")
        out.append(n)
    out.sort()
    if len(set(out)) != len(out):
        raise OracleError("duplicate axis")
    return out


def _compute_dtype(dt, kind):
    if dt in ("f32", "f64", "c64", "c128"):
        return dt
    return "f64" if kind == "mean" else "i64"


def reduction_axis(x: np.ndarray, axis, keepdims: bool, kind: str) -> np.ndarray:
    dt = dtype_of(x)
    if dt in ("c64", "c128") and kind in ("max", "min", "argmax", "argmin"):
        raise OracleError("complex ordering reduction")
    ct = _compute_dtype(dt, kind)
    xw = x if dt == ct else cast(x, ct)
    if axis is None:
        out_shape = (1,) * x.ndim if keepdims else ()
        xw = np.ascontiguousarray(xw).reshape(-1)
        kshape, kax = (xw.size,), 0
    else:
        out_shape = tuple((1 if keepdims else None) if i == axis else d for i, d in enumerate(x.shape))
        out_shape = tuple(d for d in out_shape if d is not None)
        kshape, kax = x.shape, axis
    out_dt = "i64" if kind in ("argmax", "argmin") else ct
    out_size = max(int(np.prod(out_shape)) if out_shape else 1, 1)
    out = np.zeros(out_shape, dtype=NP[out_dt])
    axis_len = kshape[kax] if kshape else 1
    if int(np.prod(out_shape) if out_shape else 1) > 0 and axis_len > 0:
        lib().oracle_reduce(RED[kind], TCODE[ct], _ptr(xw), _ptr(out), len(kshape), _c(kshape, ctypes.c_size_t),
                            _c(_estrides(xw), ctypes.c_int64), kax, ctypes.c_size_t(axis_len),
                            ctypes.c_size_t(out_size))
    return out


def reduce(x: np.ndarray, kind: str, axis=None, keepdims=False) -> np.ndarray:
    """reduce_multi (sum/prod/max/min/mean) or arg_reduce_multi (argmax/argmin)."""
    axes = resolve_axes(axis, x.ndim)
    if len(axes) == 0:
        return reduction_axis(x, None, keepdims, kind)
    if len(axes) == 1:
        return reduction_axis(x, axes[0], keepdims, kind)
    if kind in ("argmax", "argmin"):
        perm = [i for i in range(x.ndim) if i not in axes] + axes
        t = np.ascontiguousarray(x.transpose(perm))
        merged = t.reshape(t.shape[: x.ndim - len(axes)] + (-1,))
        r = reduction_axis(merged, merged.ndim - 1, keepdims, kind)
        if not keepdims:
            return r
        split = r.reshape(r.shape[:-1] + (1,) * len(axes))
        inv = [0] * x.ndim
        for i, p in enumerate(perm):
            inv[p] = i
        return split.transpose(inv)
    cur = x
    for ax in axes:
        cur = reduction_axis(cur, ax, True, kind)
    if keepdims:
        return cur
    return cur.reshape(tuple(d for i, d in enumerate(cur.shape) if i not in axes))


def cumsum(x: np.ndarray, axis=None, literal=False) -> np.ndarray:
    dt = dtype_of(x)
    ct = dt if dt in ("f32", "f64") else "i64"
    xw = x if dt == ct else cast(x, ct)
    if axis is None:
        xw = np.ascontiguousarray(xw).reshape(-1)
        kax = 0
    else:
        kax = resolve_axes(axis, x.ndim)[0]
    out = np.empty(xw.shape, dtype=NP[ct])
    if out.size:
        lib().oracle_cumsum(TCODE[ct], int(literal), _ptr(xw), _ptr(out), xw.ndim, _c(xw.shape, ctypes.c_size_t),
                            _c(_estrides(xw), ctypes.c_int64), kax, ctypes.c_size_t(out.size))
    return out


def contiguous(x: np.ndarray) -> np.ndarray:
    """contiguous(): a C-ordered copy gathered element by element through the view's strides
    (cpu_copy_bytes, indexing.rs:1388-1409); any dtype, copied as raw bytes."""
    out = np.empty(x.shape, dtype=x.dtype)
    if out.size:
        lib().oracle_copy_bytes(_ptr(x), _ptr(out), x.ndim, _c(x.shape, ctypes.c_size_t),
                                _c(_estrides(x), ctypes.c_int64), ctypes.c_size_t(x.itemsize))
    return out


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    return cast(np.ascontiguousarray(x, dtype=np.float32), "f16").view(np.uint16)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    return cast(np.ascontiguousarray(x, dtype=np.float32), "bf16").view(np.uint16)
