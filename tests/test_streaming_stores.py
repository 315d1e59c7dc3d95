"""The built kernels really issue streaming stores, on CPU: the gfx950 code objects that
`__graft_entry__.build()` compiled in this tree from its own sources (musapy_amd/_build) are
disassembled, and the kernel instantiations that a launcher selects for large outputs must hold
`global_store_... nt` instructions.  A runtime choice between a streaming and a default store was
once merged by the compiler into a default store in every kernel, silently (results are the same,
only the HBM rate drops), and a one-trip loop around the store loses the hint the same way."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "musapy_amd", "_build")
LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"

# (object, kernel family, required): every streaming instantiation (store policy template argument
# true, `Lb1E` in the mangled name) of the family must hold a streaming store; the named ones must
# exist and hold one (they are what the measured configurations launch).
FAMILIES = {
    "kernels_elementwise.hip.o": ["k_binary_flat", "k_unary_flat", "k_unary_rows", "k_unary_transpose"],
    "kernels_scan.hip.o": ["k_scan_chain"],
}
REQUIRED = {
    "kernels_elementwise.hip.o": [
        "k_binary_flatILi4ELi1ELb1ENS_4AddFEff",  # C1 f32 add
        "k_binary_flat_mixedILi2ELb1ENS_4AddFEdld",  # C3 i64 + f64 -> f64
        "k_binary_rowpiecesILi4ELi2ELb1ENS_4AddFEff",  # C2 broadcast add
        "k_binary_rowsILi4ELi4ELb1ENS_4AddFEff",
        "k_unary_transposeINS_9IdentityFEiiLi32ELi128ELi1024ELb1E",  # contiguous X^T f32
        "k_unary_rowsILi4ELi4ELb1ENS_9IdentityFEii",  # flip
        "k_unary_flatILi2ELi1ELb1ENS_5CastFIf12musapy_c64_t",  # f32 -> c64
    ],
    "kernels_scan.hip.o": ["k_scan_chainIdLi1024ELi4ELb1E",  # C5 cumsum
                           "k_scan_chainIdLi512ELi2ELb1E"],  # rows of fewer than two 64 KB tiles
}


def _tools():
    need = [os.path.join(LLVM, t) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")]
    return all(os.path.exists(t) for t in need)


def _kernels(obj, tmp):
    """{mangled kernel name: disassembly} of the gfx950 code object inside a build object."""
    fat, co = os.path.join(tmp, "fat.bin"), os.path.join(tmp, "k.co")
    subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fat}", obj, os.path.join(tmp, "host.o")],
                   check=True)
    subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={fat}",
                    f"--targets={TARGET}", f"--output={co}"], check=True)
    dis = subprocess.run([f"{LLVM}/llvm-objdump", "-d", co], check=True, capture_output=True, text=True).stdout
    out = {}
    for m in re.finditer(r"^[0-9a-f]+ <(_ZN3mpy\w+)>:\n(.*?)(?=^[0-9a-f]+ <|\Z)", dis, re.M | re.S):
        out[m.group(1)] = m.group(2)
    return out


@pytest.mark.parametrize("obj", sorted(FAMILIES))
def test_streaming_instantiations_hold_streaming_stores(obj, tmp_path):
    path = os.path.join(BUILD, obj)
    if not os.path.exists(path) or not _tools():
        pytest.skip("build objects or ROCm LLVM tools missing (run __graft_entry__.build() first)")
    kernels = _kernels(path, str(tmp_path))
    assert kernels, "no kernels found in the code object"

    def has_nt_store(body):
        return any(re.search(r"\bglobal_store_\w+\b.*\bnt\b", ln) for ln in body.splitlines())

    checked = 0
    for fam in FAMILIES[obj]:
        pat = re.compile(rf"^_ZN3mpy\d+{fam}I")
        for name, body in kernels.items():
            if pat.match(name) and "Lb1E" in name:
                assert has_nt_store(body), f"{name}: streaming instantiation without a streaming store"
                checked += 1
            elif pat.match(name) and "Lb0E" in name:
                assert not has_nt_store(body), f"{name}: default-store instantiation with a streaming store"
    assert checked > 0
    for frag in REQUIRED[obj]:
        hits = [n for n in kernels if frag in n]
        assert hits, f"no kernel matching {frag}"
        assert all(has_nt_store(kernels[n]) for n in hits), frag
