"""Device allocation failures (QVH_FAULT_ALLOC=N makes the N-th device allocation of the process
fail) surface as ValueError and leave the index unchanged, as a failing call of the reference
leaves its index (quiver::Error raised before anything is committed). Each N runs in a child
process (tests/alloc_fault_child.py), one after another."""

import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

CHILD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "alloc_fault_child.py")


def test_injected_allocation_failures_leave_indexes_unchanged():
    faults = set()
    for n in (1, 2, 3, 4, 5, 6, 8, 10, 12, 15, 19, 24, 30, 40, 60):
        env = dict(os.environ, QVH_FAULT_ALLOC=str(n))
        print(f"case: QVH_FAULT_ALLOC={n}", flush=True)
        out = subprocess.run([sys.executable, CHILD], env=env, capture_output=True, text=True, timeout=120)
        print(out.stdout.strip())
        assert out.returncode == 0 and "state ok" in out.stdout, out.stdout + out.stderr
        faults.update(line for line in out.stdout.splitlines() if line.startswith("fault at"))
    print(sorted(faults))
    assert len(faults) >= 4  # failures met in several different operations
