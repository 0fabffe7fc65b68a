"""The C-ABI library loads and exports every entry point include/qvh.h declares (no GPU needed)."""

import ctypes as C

import numpy as np

from qvh_ctypes import LIB, Qvh, declared_functions


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(LIB)
    names = declared_functions()
    assert len(names) >= 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"libqvh.so lacks {missing}"


def test_invalid_arguments_are_rejected_before_any_device_work():
    q = Qvh()
    h = C.c_void_p()
    assert q.lib.qvh_flat_create(0, 0, C.byref(h)) == -22
    assert "dimension" in q.error()
    assert q.lib.qvh_flat_create(16, 7, C.byref(h)) == -22
    assert "metric" in q.error()
    x = np.zeros((1, 4), np.float32)
    assert q.lib.qvh_normalize(x, 1, 0) == -22
