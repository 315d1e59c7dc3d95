"""musapy_amd -- MI355X-native backend for musapy's stride-aware elementwise + reduction path.

The Python surface mirrors musapy's (python/musapy/__init__.py re-exporting the PyO3 module):
``ms.array``, ``ms.add`` ... ``ms.cumsum``, the same argument conventions, dtype strings
('f32', 'i64', ...) and exception classes.  Arrays live on a HIP device ("hip:N"; "musa:N" is
accepted as an alias so musapy code keeps working).  Every operator runs through the C-ABI
kernel library ``libmusapy_hip.so``; importing fails loudly when it has not been built.
"""
from __future__ import annotations

import builtins as _builtins
import os as _os

import numpy as _np

_here = _os.path.dirname(_os.path.abspath(__file__))
try:
    from . import _core
except ImportError as _e:  # pragma: no cover - exercised only on an unbuilt tree
    raise ImportError(
        "musapy_amd native extension is not built (run `python musapy_amd/build.py`): " + str(_e)
    ) from _e

from ._core import (  # noqa: F401
    Array, MusapyError, DeviceError, DeviceNotConfiguredError, DtypeError, ShapeError, MemoryError,
    OutOfMemoryError, StreamError, KernelError, InteropError,
    add, sub, mul, div, pow, sin, cos, exp, log, abs, sign, neg, clamp, astype,
    eq, ne, lt, gt, le, ge,
    sum, prod, max, min, mean, argmax, argmin, cumsum,
    transpose, flip, index_select, contiguous,
    set_default_device, get_default_device, synchronize, device_count, device_info, mem_stats, empty_cache,
    Stream, stream, current_stream, set_debug, debug,
)

__all__ = [
    "Array", "Dtype", "array", "from_numpy", "ones", "add", "sub", "mul", "div", "pow", "sin", "cos", "exp",
    "log", "abs", "sign", "neg", "clamp", "astype", "eq", "ne", "lt", "gt", "le", "ge", "sum", "prod", "max",
    "min", "mean", "argmax", "argmin", "cumsum", "transpose", "permute", "flip", "slice", "index_select",
    "contiguous", "Stream", "stream", "current_stream", "synchronize", "from_dlpack", "set_debug", "debug",
]

# dtype constants: Dtype objects that compare equal to their names and aliases
# (rust/musapy-python/src/dtype.rs:149-190; python/musapy/__init__.py exports `bool` as `bool_`)
Dtype = _core.Dtype
bool_ = getattr(_core, "bool")
int8, int16, int32, int64 = _core.int8, _core.int16, _core.int32, _core.int64
uint8, uint16, uint32, uint64 = _core.uint8, _core.uint16, _core.uint32, _core.uint64
float16, float32, float64, bfloat16 = _core.float16, _core.float32, _core.float64, _core.bfloat16
complex64, complex128 = _core.complex64, _core.complex128

_NP_OF = {"bool": _np.bool_, "i8": _np.int8, "i16": _np.int16, "i32": _np.int32, "i64": _np.int64,
          "u8": _np.uint8, "u16": _np.uint16, "u32": _np.uint32, "u64": _np.uint64, "f16": _np.float16,
          "f32": _np.float32, "f64": _np.float64, "c64": _np.complex64, "c128": _np.complex128}
_ALIASES = {"float32": "f32", "float64": "f64", "float16": "f16", "bfloat16": "bf16", "int8": "i8",
            "int16": "i16", "int32": "i32", "int64": "i64", "uint8": "u8", "uint16": "u16",
            "uint32": "u32", "uint64": "u64", "complex64": "c64", "complex128": "c128", "bool_": "bool",
            "b1": "bool", "bool8": "bool", "half": "f16", "single": "f32", "double": "f64"}


def _norm_dtype(d) -> str:
    if d is None:
        return None
    if isinstance(d, _np.dtype) or (isinstance(d, type) and issubclass(d, _np.generic)):
        d = _np.dtype(d).name
    if not isinstance(d, (str, Dtype)):
        raise TypeError("dtype must be a Dtype instance or a dtype string (e.g. 'f32', 'float32')")
    d = str(d).lower()
    d = _ALIASES.get(d, d)
    if d not in _NP_OF and d != "bf16":
        raise ValueError(f"unknown dtype: {d}")
    return d


def _c_order(x):
    """C-contiguous copy when needed; unlike numpy.ascontiguousarray it keeps 0-d arrays 0-d."""
    return x if x.flags.c_contiguous else x.copy(order="C")


def _contains_complex(x) -> bool:
    if isinstance(x, complex):
        return True
    if isinstance(x, (list, tuple)):
        return any(_contains_complex(v) for v in x)
    return False


def array(data, dtype=None, device=None) -> Array:
    """``ms.array(data, dtype=None, device=None)`` (rust/musapy-python/src/ops.rs:28-101).

    dtype resolution: explicit argument, else complex literals -> c128, else float32.
    ``data`` may be a (nested) list/tuple, a scalar or a numpy array.
    """
    dt = _norm_dtype(dtype)
    if dt is None:
        if isinstance(data, _np.ndarray):
            dt = "c128" if _np.iscomplexobj(data) else "f32"
        else:
            dt = "c128" if _contains_complex(data) else "f32"
    if dt == "bf16":
        host = _np.asarray(data)
        if host.dtype != _np.uint16:
            raise DtypeError("bf16 arrays are created from raw uint16 bit patterns")
    else:
        host = _np.asarray(data, dtype=_NP_OF[dt])
    return _core._from_numpy(_c_order(host), dt, device)


def from_numpy(x, device=None) -> Array:
    """Copy a numpy array (any dtype musapy knows) to the device, keeping its dtype."""
    x = _c_order(_np.asarray(x))
    dt = _ALIASES.get(x.dtype.name, x.dtype.name)
    return _core._from_numpy(x, dt, device)


def ones(shape, dtype="f32", device=None) -> Array:
    dt = _norm_dtype(dtype)
    if isinstance(shape, int):
        shape = (shape,)
    return array(_np.ones(shape, dtype=_NP_OF[dt]), dtype=dt, device=device)


def permute(a: Array, axes) -> Array:
    return transpose(a, list(axes))


def slice(a: Array, ranges) -> Array:  # noqa: A001 - musapy name
    """``ms.slice(a, [(start, stop, step), ...])`` (rust/musapy-core/src/layout.rs:214-259)."""
    start = [r[0] for r in ranges]
    stop = [r[1] for r in ranges]
    step = [r[2] if len(r) > 2 else 1 for r in ranges]
    return _core.slice(a, start, stop, step)


def _tolist(self: Array):
    if self.dtype in ("f16", "bf16"):
        raise NotImplementedError(f"tolist() is not supported for {self.dtype} (as in musapy)")
    return self.numpy().tolist()


def _item(self: Array):
    if self.size != 1:
        raise ValueError(f"item() requires an array of size 1, got size {self.size}")
    if self.dtype in ("f16", "bf16"):
        raise NotImplementedError(f"item() is not supported for {self.dtype} (as in musapy)")
    return self.numpy().reshape(-1)[0].item()


def _repr(self: Array) -> str:
    return f"Array(shape={self.shape}, dtype={self.dtype}, device={self.device})"


def _getitem(self: Array, key) -> Array:
    """Basic indexing as zero-copy views (rust/musapy-python/src/array.rs:225-450, view path):
    an int selects along an axis and drops it, a slice keeps it; a tuple applies item by item.
    Array indices (boolean masks, fancy indexing) are outside this backend's path."""
    items = key if isinstance(key, tuple) else (key,)
    if self.ndim == 0:
        raise IndexError("too many indices for 0-dim array")
    if len(items) > self.ndim:
        raise IndexError("too many indices for array")
    cur, dim = self, 0
    for it in items:
        size = cur.shape[dim]
        if isinstance(it, _builtins.slice):
            start, stop, step = it.indices(size)
            if step <= 0:
                raise ValueError("slice step must be positive")
            ranges = [(0, d, 1) for d in cur.shape]
            ranges[dim] = (start, _builtins.max(start, stop), step)
            cur = slice(cur, ranges)
            dim += 1
        elif isinstance(it, (int, _np.integer)) and not isinstance(it, bool):
            i = int(it)
            if i < 0:
                i += size
            if i < 0 or i >= size:
                raise IndexError(f"index {int(it)} out of bounds for dimension (size {size})")
            cur = index_select(cur, dim, i)
        else:
            raise TypeError("index must be an integer or slice (array indices are not supported by this backend)")
    return cur


# ---- interop: DLPack and the NumPy protocols (docs/v0.4-beta-plan-zh.md:42-43, 96-125) ----
_KDL_CPU, _KDL_ROCM = 1, 10


def from_dlpack(x, *, device=None, copy=None) -> Array:
    """``ms.from_dlpack(x)``: an array from any object with ``__dlpack__`` / ``__dlpack_device__``.

    A tensor on a HIP device (a PyTorch-ROCm tensor, another musapy_amd array) is adopted
    without a copy: the producer orders its pending work before this backend's stream, and its
    memory is handed back when the last view of the array goes.  A host tensor (NumPy, a
    PyTorch CPU tensor) is copied to the device (``copy=False`` then raises).  ``copy=True``
    always returns an independent array.
    """
    if not hasattr(x, "__dlpack__") or not hasattr(x, "__dlpack_device__"):
        raise TypeError(f"from_dlpack: {type(x).__name__} does not implement the DLPack protocol")
    dev_type, dev_id = x.__dlpack_device__()
    dev_type, dev_id = int(dev_type), int(dev_id)
    if dev_type == _KDL_ROCM:
        if device is not None and _core._parse_device(device) != dev_id:
            raise InteropError(f"from_dlpack: the tensor lives on hip:{dev_id}, not {device}")
        a = _core._from_dlpack_device(x, dev_id)
        return _core._clone(a) if copy else a
    if dev_type == _KDL_CPU:
        if copy is False:
            raise BufferError("from_dlpack: a host tensor has to be copied to reach the device (copy=False)")
        return from_numpy(_np.from_dlpack(x), device=device)
    raise InteropError(f"from_dlpack: DLPack device type {dev_type} is neither a HIP device (10) nor the host (1)")


def _array_protocol(self: Array, dtype=None, copy=None):
    """``np.asarray(a)``: synchronise, copy to the host (the readback of ``numpy()``)."""
    if copy is False:
        raise ValueError("a device array cannot be viewed as a NumPy array without a copy")
    host = self.numpy()
    return host if dtype is None else host.astype(dtype, copy=False)


# NumPy ufuncs this backend computes on the device; anything else is left to NumPy's own error
_UFUNCS = {
    "add": "add", "subtract": "sub", "multiply": "mul", "divide": "div", "true_divide": "div",
    "power": "pow", "sin": "sin", "cos": "cos", "exp": "exp", "log": "log", "absolute": "abs",
    "sign": "sign", "negative": "neg", "equal": "eq", "not_equal": "ne", "less": "lt", "greater": "gt",
    "less_equal": "le", "greater_equal": "ge",
}


def _array_ufunc(self: Array, ufunc, method, *inputs, **kwargs):
    """Strict policy: ``np.add(a, b)`` on device arrays runs the device op; mixing a device array
    with host data raises instead of silently computing on the host."""
    name = _UFUNCS.get(ufunc.__name__)
    if method != "__call__" or name is None:
        return NotImplemented
    if any(not isinstance(v, Array) for v in inputs):
        kinds = ", ".join(type(v).__name__ for v in inputs)
        raise DeviceError(f"np.{ufunc.__name__}({kinds}): operands live on different devices; move host data "
                          f"with ms.from_numpy / ms.from_dlpack, or read the device array back with .numpy()")
    out = kwargs.pop("out", None)
    if kwargs:
        return NotImplemented
    if out is not None:
        if len(out) != 1 or not isinstance(out[0], Array):
            return NotImplemented
        out = out[0]
    return globals()[name](*inputs, out=out)


Array.__array__ = _array_protocol
Array.__array_ufunc__ = _array_ufunc
Array.__getitem__ = _getitem
Array.tolist = _tolist
Array.item = _item
Array.__repr__ = _repr
Array.T = property(lambda self: transpose(self))
Array.__len__ = lambda self: self.shape[0] if self.ndim else 0
