"""Builds the native parts of quiver_amd in-tree.

    python quiver_amd/build.py

* ``quiver_amd/lib/libqvh.so``        - HIP kernels + the qvh C-ABI (include/qvh.h), gfx950 only
* ``quiver_amd/lib/libquiver_amd.so`` - the C++ API (quiver::FlatIndex, ...) over the C-ABI
* ``quiver_amd/_quiver*.so``          - the pybind11 module under quiver_amd/__init__.py
* ``tests/cpp/test_cpp_api``          - the C++ API test program (run by tests/test_cpp_api_gpu.py)

Every HIP source is compiled with -ffp-contract=off (fused multiply-adds only where the source
writes fmaf(), as the bit-exact paths require) and without packed-FP32 instructions.
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "lib")
BUILD = os.path.join(ROOT, "_build")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    f"-I{INCLUDE}", f"-I{os.path.join(CSRC, 'hip')}",
]
CXX_FLAGS = ["-std=c++20", "-O2", "-fPIC", "-pthread", "-ffp-contract=off", "-Wall", "-Wextra",
             f"-I{INCLUDE}", f"-I{os.path.join(CSRC, 'host', 'include')}"]


def _run(cmd, quiet_warnings=("packed-fp32-ops",)):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines()
                    if not any(w in l for w in quiet_warnings))
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _hipcc() -> str:
    exe = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found (ROCm is required to build quiver_amd)")
    return exe


def build_hip(jobs: int = 8) -> str:
    os.makedirs(LIB, exist_ok=True)
    obj_dir = os.path.join(BUILD, "hip")
    os.makedirs(obj_dir, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "hip", "*.hip")))
    hipcc = _hipcc()

    def compile_one(src):
        obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
        _run([hipcc, *HIPCC_FLAGS, "-c", src, "-o", obj])
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    out = os.path.join(LIB, "libqvh.so")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", out + ".tmp",
          f"-Wl,-rpath,{ROCM}/lib"])
    os.replace(out + ".tmp", out)
    return out


def build_host() -> str:
    srcs = sorted(glob.glob(os.path.join(CSRC, "host", "src", "*.cc")))
    out = os.path.join(LIB, "libquiver_amd.so")
    _run(["g++", *CXX_FLAGS, "-shared", *srcs, f"-L{LIB}", "-lqvh", "-Wl,-rpath,$ORIGIN",
          "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_python() -> str:
    import pybind11

    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = os.path.join(PKG, "_quiver" + suffix)
    _run(["g++", *CXX_FLAGS, "-shared", "-fvisibility=hidden",
          f"-I{pybind11.get_include()}", f"-I{sysconfig.get_paths()['include']}",
          os.path.join(CSRC, "python", "quiver_ext.cc"),
          f"-L{LIB}", "-lquiver_amd", "-lqvh", "-Wl,-rpath,$ORIGIN/lib", "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_cpp_tests() -> str:
    src = os.path.join(ROOT, "tests", "cpp", "test_cpp_api.cc")
    out = os.path.join(ROOT, "tests", "cpp", "test_cpp_api")
    _run(["g++", *CXX_FLAGS, src, f"-L{LIB}", "-lquiver_amd", "-lqvh", f"-Wl,-rpath,{LIB}",
          "-Wl,-rpath,$ORIGIN/../../quiver_amd/lib", "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build(jobs: int = 8) -> None:
    build_hip(jobs)
    build_host()
    build_python()
    build_cpp_tests()


if __name__ == "__main__":
    build(int(sys.argv[1]) if len(sys.argv) > 1 else 8)
    print("built", os.path.join(LIB, "libqvh.so"))
