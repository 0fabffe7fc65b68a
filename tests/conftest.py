import os
import subprocess
import sys

import pytest

# torch (when installed) is imported before any test module loads quiver_amd: torch ships its own
# HIP runtime, and loading it after quiver_amd's would leave two runtime copies in the process,
# whose device memory cannot be exchanged (the device-tensor tests pass torch tensors to the
# library). Loaded first, torch's copy is the only one and the library binds to it.
try:
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - torch is optional
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs on the MI355X box)")
    config.addinivalue_line("markers", "slow: longer CPU-side checks")


@pytest.fixture(scope="session")
def oracle():
    """The C restatement of the reference (oracle/liboracle.so), built on demand."""
    from oracle.oracle import ORACLE_SO, Oracle

    if not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    return Oracle()


@pytest.fixture(scope="session")
def reference():
    """The compiled reference (oracle/_ref/libquiver_ref.so) when it has been built here."""
    from oracle.oracle import REF_SO, Reference

    if not os.path.exists(REF_SO):
        pytest.skip("compiled reference library not present (built only where the reference "
                    "sources are)")
    return Reference()
