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


# ---- sanitized host build (CPU tests of the host code) ----------------------------------------
# The kernel sources are compiled for the host side only (no device code, so kernel launches fail
# at run time exactly as they do on a machine without a GPU); the host code of every source is
# built with AddressSanitizer + UndefinedBehaviorSanitizer by clang, so one sanitizer runtime
# (clang's) serves the whole process.  The result is a copy of the package under
# ``_build/sanitized/musapy_amd``; it is meant for the host-memory runtime backend
# (mpy_rt_set_backend) and must be loaded with clang's ASan runtime preloaded
# (``sanitizer_env()``).
CLANGXX = os.path.join(ROCM, "llvm", "bin", "clang++")
SAN_HIP_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined"]
SAN_CXX_FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"]
SAN_COMMON = ["-O1", "-g", "-std=c++17", "-fPIC", "-fno-omit-frame-pointer", "-ffp-contract=off"]


def sanitized_dir() -> str:
    return os.path.join(BUILD, "sanitized")


def asan_runtime() -> str:
    r = subprocess.run([CLANGXX, "-print-file-name=libclang_rt.asan-x86_64.so"], stdout=subprocess.PIPE, text=True)
    path = r.stdout.strip()
    if r.returncode != 0 or not os.path.isfile(path):
        raise RuntimeError("clang's ASan runtime (libclang_rt.asan-x86_64.so) was not found")
    return path


def sanitizer_env(env: dict | None = None) -> dict:
    """Environment for a Python process that imports the sanitized package."""
    env = dict(os.environ if env is None else env)
    env["LD_PRELOAD"] = asan_runtime()
    # the interpreter and HIP's runtime are not instrumented; their allocations are not ours
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0:halt_on_error=1:exitcode=86"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1:exitcode=87"
    env["PYTHONPATH"] = sanitized_dir() + os.pathsep + env.get("PYTHONPATH", "")
    return env


def build_sanitized(jobs: int | None = None, verbose: bool = True) -> str:
    import pybind11

    out = os.path.join(sanitized_dir(), "musapy_amd")
    objdir = os.path.join(sanitized_dir(), "obj")
    os.makedirs(out, exist_ok=True)
    os.makedirs(objdir, exist_ok=True)
    incs = [f"-I{pybind11.get_include()}", f"-I{sysconfig.get_paths()['include']}"]

    def obj(src: str) -> str:
        return os.path.join(objdir, src.replace("/", "_") + ".o")

    def hip(src: str) -> str:
        _run([HIPCC, f"--offload-arch={ARCH}", *SAN_HIP_FLAGS, *SAN_COMMON, "-x", "hip", "-c",
              os.path.join(CSRC, src), "-o", obj(src)])
        return obj(src)

    def cxx(src: str) -> str:
        _run([CLANGXX, *SAN_CXX_FLAGS, *SAN_COMMON, *incs, "-c", os.path.join(CSRC, src), "-o", obj(src)])
        return obj(src)

    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        hip_objs = [f.result() for f in [ex.submit(hip, s) for s in HIP_SOURCES]]
        cxx_objs = [f.result() for f in [ex.submit(cxx, s) for s in CXX_SOURCES]]
    lib = os.path.join(out, "libmusapy_hip.so")
    _run([CLANGXX, *SAN_CXX_FLAGS, "-shared-libsan", "-shared", "-o", lib, *hip_objs, f"-L{ROCM}/lib",
          "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib"])
    core = os.path.join(out, os.path.basename(core_path()))
    _run([CLANGXX, *SAN_CXX_FLAGS, "-shared-libsan", "-shared", "-o", core, *cxx_objs, f"-L{out}", "-lmusapy_hip",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM}/lib"])
    shutil.copyfile(os.path.join(PKG, "__init__.py"), os.path.join(out, "__init__.py"))
    if verbose:
        print(f"built the sanitized host package in {out}")
    return out


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)


if __name__ == "__main__":
    if "--sanitized" in sys.argv[1:]:
        build_sanitized()
    else:
        build()
    sys.exit(0)
