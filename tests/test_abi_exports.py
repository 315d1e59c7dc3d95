"""The C-ABI library loads without a GPU and exports every function include/*.h declares."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "musapy_amd", "libmusapy_hip.so")
HEADERS = [os.path.join(ROOT, "include", h) for h in ("musapy_kernels.h", "musapy_hip_runtime.h")]


def declared(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.findall(r"^\s*(?:void|int|size_t|uint32_t|const char\*)\s+(\w+)\s*\(", text, flags=re.M)


def test_headers_declare_the_hot_path():
    names = declared(HEADERS[0])
    assert len(names) == len(set(names))
    # families of rust/musapy-ops/src/kernels.rs:16-305 that this backend implements
    for fam in ("add", "sub", "mul", "div", "pow"):
        assert f"musapy_{fam}_f32_v2" in names and f"musapy_{fam}_f64_v2" in names
    assert sum(n.startswith("musapy_cast_") for n in names) == 27 + 2 + 5
    assert sum("_partial_" in n for n in names) == 26
    assert sum("_final_" in n for n in names) == 26
    assert sum("_small_axis_" in n for n in names) == 20
    assert sum("_mid_" in n for n in names) == 6
    assert {"musapy_cumsum_i64_v3", "musapy_cumsum_f32_v3", "musapy_cumsum_f64_v3"} <= set(names)
    # comparisons (kernels.rs:84-95, 114-117)
    for fam in ("eq", "ne", "lt", "gt", "le", "ge"):
        assert f"musapy_{fam}_f32_v2" in names and f"musapy_{fam}_f64_v2" in names
    assert {f"musapy_{f}_{c}_v2" for f in ("eq", "ne") for c in ("c64", "c128")} <= set(names)
    # complex elementwise (kernels.rs:102-113)
    for fam in ("add", "sub", "mul", "div", "neg", "abs"):
        assert f"musapy_{fam}_c64_v2" in names and f"musapy_{fam}_c128_v2" in names


@pytest.mark.parametrize("header", HEADERS, ids=os.path.basename)
def test_library_exports_every_declared_symbol(header):
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared(header) if not hasattr(lib, n)]
    assert not missing, missing
