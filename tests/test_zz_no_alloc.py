"""qvh_flat_search_device_noalloc (workspace in a fixed device array, no allocation) against
qvh_flat_search_device on the same handle and inputs, through the C-ABI: identical rows and
bit-identical distances on two calls in a row, the second with fewer queries; the MFMA scan, the
few-query scan and cosine; the library's device-allocation counter does not move across the
no-allocation calls; a search too large for the array is refused before anything runs; and calls on
two handles and two streams, issued without synchronizing in between, take the shared array in
turn (each still equals the allocating entry point's result)."""

import ctypes as C

import numpy as np
import pytest

from qvh_ctypes import LIB

pytestmark = pytest.mark.gpu

_vp = C.c_void_p


class Dev:
    """Device buffers as torch tensors (torch's HIP runtime is the one the library binds to; the entry
    point under test allocates none)."""

    def __init__(self):
        import torch

        self.torch = torch
        self.held = []

    def put(self, a):
        t = self.torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")
        self.held.append(t)
        return _vp(t.data_ptr())

    def empty(self, nbytes):
        t = self.torch.empty(max(nbytes, 1), dtype=self.torch.uint8, device="cuda:0")
        self.held.append(t)
        return _vp(t.data_ptr())

    def get(self, p, shape, dtype):
        t = next(t for t in self.held if t.data_ptr() == p.value)
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        return t.cpu().numpy().view(np.uint8)[:n].view(dtype).reshape(shape).copy()

    def free(self):
        self.held = []


def _lib():
    L = C.CDLL(LIB)
    L.qvh_last_error.restype = C.c_char_p
    L.qvh_flat_create.argtypes = [C.c_uint32, C.c_int, C.POINTER(_vp)]
    L.qvh_flat_destroy.argtypes = [_vp]
    L.qvh_flat_append.argtypes = [_vp, _vp, C.c_uint64, _vp]
    sig = [_vp, _vp, C.c_uint64, C.c_uint32, _vp, _vp, _vp, _vp]
    L.qvh_flat_search_device.argtypes = sig
    L.qvh_flat_search_device_noalloc.argtypes = sig
    L.qvh_flat_sync.argtypes = [_vp]
    L.qvh_device_allocations.argtypes = [C.POINTER(C.c_uint64)]
    return L


def _allocations(L):
    n = C.c_uint64()
    assert L.qvh_device_allocations(C.byref(n)) == 0
    return n.value


def _search(L, dev, fn, h, d_q, nq, k):
    d_rows, d_dist = dev.empty(nq * k * 4), dev.empty(nq * k * 4)
    st = fn(h, d_q, nq, k, None, d_rows, d_dist, None)
    assert st == 0, L.qvh_last_error().decode()
    assert L.qvh_flat_sync(h) == 0
    return dev.get(d_rows, (nq, k), np.uint32), dev.get(d_dist, (nq, k), np.float32)


@pytest.mark.parametrize("metric", [0, 2])
def test_noalloc_search_matches_the_allocating_entry_point(metric):
    L, dev = _lib(), Dev()
    rng = np.random.default_rng(metric + 3)
    dim = 96
    base = rng.standard_normal((40_000, dim)).astype(np.float32)
    h = _vp()
    assert L.qvh_flat_create(dim, metric, C.byref(h)) == 0, L.qvh_last_error().decode()
    try:
        assert L.qvh_flat_append(h, base.ctypes.data_as(_vp), base.shape[0], None) == 0
        for nq, k in ((600, 10), (5, 20), (300, 100)):  # MFMA scan, few-query scan, wide merge
            print(f"case: noalloc metric={metric} nq={nq} k={k}", flush=True)
            q = rng.standard_normal((nq, dim)).astype(np.float32)
            d_q = dev.put(q)
            want = _search(L, dev, L.qvh_flat_search_device, h, d_q, nq, k)
            allocs = _allocations(L)
            got = _search(L, dev, L.qvh_flat_search_device_noalloc, h, d_q, nq, k)
            again = _search(L, dev, L.qvh_flat_search_device_noalloc, h, d_q, max(1, nq // 3), k)
            assert _allocations(L) == allocs, "the no-allocation entry point allocated device memory"
            assert np.array_equal(got[0], want[0]) and np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32))
            small = _search(L, dev, L.qvh_flat_search_device, h, d_q, max(1, nq // 3), k)
            assert np.array_equal(again[0], small[0])
            assert np.array_equal(again[1].view(np.uint32), small[1].view(np.uint32))
        # A batch whose workspace exceeds the fixed array is refused before anything is enqueued.
        nq = 200_000
        d_q = dev.put(np.zeros((nq, dim), np.float32))
        d_rows, d_dist = dev.empty(nq * 10 * 4), dev.empty(nq * 10 * 4)
        st = L.qvh_flat_search_device_noalloc(h, d_q, nq, 10, None, d_rows, d_dist, None)
        assert st == -22 and "scratch" in L.qvh_last_error().decode()
        assert L.qvh_flat_sync(h) == 0
    finally:
        L.qvh_flat_destroy(h)
        dev.free()


def test_noalloc_calls_on_two_handles_and_streams_take_the_array_in_turn():
    import torch

    L, dev = _lib(), Dev()
    rng = np.random.default_rng(11)
    dim, k = 64, 10
    handles, queries, want = [], [], []
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    try:
        for i in range(2):
            base = rng.standard_normal((60_000 + 5_000 * i, dim)).astype(np.float32)
            h = _vp()
            assert L.qvh_flat_create(dim, 0, C.byref(h)) == 0, L.qvh_last_error().decode()
            handles.append(h)
            assert L.qvh_flat_append(h, base.ctypes.data_as(_vp), base.shape[0], None) == 0
            nq = 700 - 300 * i  # the MFMA scan on one handle, its row-split form on the other
            q = rng.standard_normal((nq, dim)).astype(np.float32)
            d_q = dev.put(q)
            queries.append((d_q, nq))
            want.append(_search(L, dev, L.qvh_flat_search_device, h, d_q, nq, k))
        torch.cuda.synchronize()
        outs = []
        print("case: noalloc, two handles on two streams, 3 rounds without synchronizing", flush=True)
        for _ in range(3):
            for i, h in enumerate(handles):
                d_q, nq = queries[i]
                d_rows, d_dist = dev.empty(nq * k * 4), dev.empty(nq * k * 4)
                st = L.qvh_flat_search_device_noalloc(h, d_q, nq, k, None, d_rows, d_dist,
                                                      _vp(streams[i].cuda_stream))
                assert st == 0, L.qvh_last_error().decode()
                outs.append((i, d_rows, d_dist, nq))
        for s in streams:
            s.synchronize()
        for h in handles:
            assert L.qvh_flat_sync(h) == 0
        for i, d_rows, d_dist, nq in outs:
            rows = dev.get(d_rows, (nq, k), np.uint32)
            dist = dev.get(d_dist, (nq, k), np.float32)
            assert np.array_equal(rows, want[i][0]) and np.array_equal(dist.view(np.uint32), want[i][1].view(np.uint32))
    finally:
        for h in handles:
            L.qvh_flat_destroy(h)
        dev.free()
