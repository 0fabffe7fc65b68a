"""The filter forms of the flat search through the C-ABI on device buffers (torch allocates them):
qvh_flat_search_device takes a device bitmap and tests it over every row; qvh_flat_search_device_rows
takes the admitted rows as an ascending device list and scans only those (or, for a k the listed-row
scan does not serve, turns the list into a device bitmap first). Both give the rows and the
bit-identical distances of qvh_flat_search with the same filter from host memory, and the oracle's
answer (src/flat_index.cc:84-106 with the Filter of :85), at densities from none to every row."""

import ctypes as C

import numpy as np
import pytest

from oracle.oracle import rows_bitmap
from parity import assert_same_topk
from qvh_ctypes import LIB
from quiver_amd import datasets as D

pytestmark = pytest.mark.gpu

_vp = C.c_void_p
_METRICS = {"l2": 0, "cosine": 2}


def _lib():
    L = C.CDLL(LIB)
    L.qvh_last_error.restype = C.c_char_p
    L.qvh_flat_create.argtypes = [C.c_uint32, C.c_int, C.POINTER(_vp)]
    L.qvh_flat_destroy.argtypes = [_vp]
    L.qvh_flat_append.argtypes = [_vp, _vp, C.c_uint64, _vp]
    L.qvh_flat_search.argtypes = [_vp, _vp, C.c_uint64, C.c_uint32, _vp, _vp, _vp]
    L.qvh_flat_search_device.argtypes = [_vp, _vp, C.c_uint64, C.c_uint32, _vp, _vp, _vp, _vp]
    L.qvh_flat_search_device_rows.argtypes = [_vp, _vp, C.c_uint64, C.c_uint32, _vp, C.c_uint64, _vp, _vp, _vp]
    L.qvh_flat_sync.argtypes = [_vp]
    return L


def _ok(L, status):
    assert status == 0, L.qvh_last_error().decode()


def _ptr(a: np.ndarray):
    return _vp(a.ctypes.data)


@pytest.mark.parametrize("metric", ["l2", "cosine"])
@pytest.mark.parametrize("fraction", [0.0, 0.005, 0.1, 0.6, 0.97, 1.0])
def test_device_bitmap_and_row_list_match_host_filter(oracle, metric, fraction):
    import torch

    L = _lib()
    base, q = D.unit_mix(40_000, 300)
    n, dim = base.shape
    allowed = D.allowed_ids(n, fraction, seed=61)
    bits = rows_bitmap(allowed.astype(np.int64), n)
    print(f"case: device filters {metric} n={n} nq={q.shape[0]} admitted={allowed.size}", flush=True)
    h = _vp()
    _ok(L, L.qvh_flat_create(dim, _METRICS[metric], C.byref(h)))
    try:
        _ok(L, L.qvh_flat_append(h, _ptr(base), n, None))
        dq = torch.from_numpy(q).to("cuda:0")
        dbits = torch.from_numpy(bits.view(np.int64)).to("cuda:0")
        dlist = torch.from_numpy(allowed.astype(np.uint32).view(np.int32)).to("cuda:0")
        stored = oracle.normalize(base) if metric == "cosine" else base
        for k in (1, 10, 50, 100):
            nq = q.shape[0]
            host_rows = np.empty((nq, k), np.uint32)
            host_dist = np.empty((nq, k), np.float32)
            _ok(L, L.qvh_flat_search(h, _ptr(q), nq, k, _ptr(bits), _ptr(host_rows), _ptr(host_dist)))
            outs = []
            for form in ("bitmap", "rows"):
                rows = torch.empty((nq, k), dtype=torch.int32, device="cuda:0")
                dist = torch.empty((nq, k), dtype=torch.float32, device="cuda:0")
                if form == "bitmap":
                    st = L.qvh_flat_search_device(h, _vp(dq.data_ptr()), nq, k, _vp(dbits.data_ptr()),
                                                  _vp(rows.data_ptr()), _vp(dist.data_ptr()), None)
                else:
                    st = L.qvh_flat_search_device_rows(h, _vp(dq.data_ptr()), nq, k, _vp(dlist.data_ptr()),
                                                       allowed.size, _vp(rows.data_ptr()), _vp(dist.data_ptr()),
                                                       None)
                _ok(L, st)
                _ok(L, L.qvh_flat_sync(h))
                outs.append((form, rows.cpu().numpy().view(np.uint32), dist.cpu().numpy()))
            for form, rows, dist in outs:
                assert np.array_equal(rows, host_rows), (form, k)
                assert np.array_equal(dist.view(np.uint32), host_dist.view(np.uint32)), (form, k)
            exp_rows, exp_dist = oracle.flat_search(stored, q, k, metric, bits)
            print(k, assert_same_topk(host_rows, host_dist, exp_rows, exp_dist))
    finally:
        L.qvh_flat_destroy(h)


def test_row_list_longer_than_the_store_is_refused():
    import torch

    L = _lib()
    base, q = D.unit_mix(1_000, 4)
    h = _vp()
    _ok(L, L.qvh_flat_create(base.shape[1], 0, C.byref(h)))
    try:
        _ok(L, L.qvh_flat_append(h, _ptr(base), base.shape[0], None))
        dq = torch.from_numpy(q).to("cuda:0")
        dlist = torch.arange(1_001, dtype=torch.int32, device="cuda:0")
        rows = torch.empty((4, 5), dtype=torch.int32, device="cuda:0")
        dist = torch.empty((4, 5), dtype=torch.float32, device="cuda:0")
        st = L.qvh_flat_search_device_rows(h, _vp(dq.data_ptr()), 4, 5, _vp(dlist.data_ptr()), 1_001,
                                           _vp(rows.data_ptr()), _vp(dist.data_ptr()), None)
        assert st == -22
        assert "listed rows" in L.qvh_last_error().decode()
    finally:
        L.qvh_flat_destroy(h)
