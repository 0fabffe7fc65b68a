"""Runs the C++ API test program (tests/cpp/test_cpp_api.cc, built by quiver_amd/build.py): the flat
and IVF-PQ indexes through the public C++ headers, the way a C++ caller of the reference uses them."""

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BINARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "test_cpp_api")


def test_cpp_api_program():
    if not os.path.exists(BINARY):
        pytest.fail("tests/cpp/test_cpp_api is not built (run __graft_entry__.build())")
    print("case: tests/cpp/test_cpp_api", flush=True)
    p = subprocess.run([BINARY], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=180)
    print(p.stdout)
    assert p.returncode == 0, p.stdout
    assert "all cases passed" in p.stdout
