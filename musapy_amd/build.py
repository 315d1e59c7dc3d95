"""In-tree build of the native parts.

* ``musapy_amd/libmusapy_hip.so`` -- the C-ABI library (include/musapy_kernels.h,
  include/musapy_hip_runtime.h): hand-written HIP kernels for gfx950 plus the thin runtime layer.
* ``musapy_amd/_core*.so`` -- the C++ op layer and its pybind11 binding, linked against the
  library above (rpath $ORIGIN).

Run ``python musapy_amd/build.py`` (or ``__graft_entry__.build()``).  Every call recompiles.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = os.environ.get("MUSAPY_OFFLOAD_ARCH", "gfx950")

HIPCC = os.path.join(ROCM, "bin", "hipcc")
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # bit-exact IEEE semantics: no contraction of a*b+c into fma, no fast-math
    "-ffp-contract=off",
    # never emit packed fp32 arithmetic (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function"]

HIP_SOURCES = [
    "kernels/elementwise.hip",
    "kernels/reduce.hip",
    "kernels/scan.hip",
    "runtime/hip_runtime.cpp",
]
CXX_SOURCES = ["ops/core.cpp", "ops/ops.cpp", "ops/interop.cpp", "python/module.cpp"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")


def _obj(src: str) -> str:
    return os.path.join(BUILD, src.replace("/", "_") + ".o")


def _compile_hip(src: str) -> str:
    obj = _obj(src)
    cmd = [HIPCC, *HIP_FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    _run(cmd)
    return obj


def _compile_cxx(src: str) -> str:
    import pybind11

    obj = _obj(src)
    incs = [f"-I{pybind11.get_include()}", f"-I{sysconfig.get_paths()['include']}"]
    _run(["g++", *CXX_FLAGS, *incs, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def lib_path() -> str:
    return os.path.join(PKG, "libmusapy_hip.so")


def core_path() -> str:
    return os.path.join(PKG, "_core" + sysconfig.get_config_var("EXT_SUFFIX"))


def build(jobs: int | None = None, verbose: bool = True) -> None:
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        hip_f = [ex.submit(_compile_hip, s) for s in HIP_SOURCES]
        cxx_f = [ex.submit(_compile_cxx, s) for s in CXX_SOURCES]
        hip_objs = [f.result() for f in hip_f]
        cxx_objs = [f.result() for f in cxx_f]
    lib_tmp = lib_path() + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", lib_tmp, *hip_objs])
    os.replace(lib_tmp, lib_path())
    core_tmp = core_path() + ".tmp"
    _run(["g++", "-shared", "-o", core_tmp, *cxx_objs, f"-L{PKG}", "-lmusapy_hip",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM}/lib"])
    os.replace(core_tmp, core_path())
    if verbose:
        print(f"built {lib_path()} and {core_path()}")


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)


if __name__ == "__main__":
    build()
    sys.exit(0)
