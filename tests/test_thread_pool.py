"""The host thread pool's semantics (tests/cpp/test_thread_pool.cc), compiled against the public
header and the built C++ library; CPU only."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "quiver_amd", "lib")


def test_thread_pool_semantics(tmp_path):
    if not os.path.exists(os.path.join(LIB, "libquiver_amd.so")) or shutil.which("g++") is None:
        pytest.skip("libquiver_amd.so or g++ missing")
    exe = str(tmp_path / "test_thread_pool")
    subprocess.run(["g++", "-std=c++20", "-O2", "-pthread",
                    "-I" + os.path.join(ROOT, "quiver_amd", "csrc", "host", "include"),
                    os.path.join(ROOT, "tests", "cpp", "test_thread_pool.cc"), "-L" + LIB, "-lquiver_amd",
                    "-Wl,-rpath," + LIB, "-o", exe], check=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(out.stdout)
    assert out.returncode == 0, out.stdout + out.stderr
