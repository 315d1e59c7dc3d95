"""Guards on the gfx950 code this tree builds, checked on the CPU by disassembling the code objects
that `__graft_entry__.build()` compiled from the sources here (musapy_amd/_build).

64-bit integer -> f32 conversions must not use 64-bit VGPR shifts.  The compiler's lowering of
that conversion shifts the value with v_lshlrev_b64 by a count computed the instruction before,
and in transpose instances built for measurement that shift used a stale count in whole waves
(wrong values such as -1.0 for -721, found by the transposed-cast test).  The conversion in
ew_ops.hpp uses 32-bit operations only; this test keeps every kernel that converts int64 or
uint64 to f32 free of such shifts."""
import os
import re

import pytest

from tests.test_streaming_stores import BUILD, _kernels, _tools

SHIFT64 = re.compile(r"\bv_(lshlrev|lshrrev|ashrrev)_(b64|i64)\b[^\n]*?,\s*v\d+\s*,")


def test_int64_to_f32_conversions_have_no_64bit_vgpr_shifts(tmp_path):
    path = os.path.join(BUILD, "kernels_elementwise.hip.o")
    if not os.path.exists(path) or not _tools():
        pytest.skip("build objects or ROCm LLVM tools missing (run __graft_entry__.build() first)")
    kernels = _kernels(path, str(tmp_path))
    # CastF<long, float> / CastF<unsigned long, float> (casts), and the fused mixed kernels whose
    # result is f32 with a 64-bit integer operand (TC, TA, TB = f, l, f or f, f, l in their mangled names)
    conv = [n for n in kernels if re.search(r"CastFI[lm]fE", n)
            or re.search(r"k_(binary_flat_mixed|binary_generic_mixed)I.*E(f[lm]f|ff[lm])E", n)]
    assert len(conv) >= 8, conv
    bad = [n for n in conv if SHIFT64.search(kernels[n])]
    assert not bad, f"64-bit VGPR shifts in: {bad[:5]}"
