"""ctypes view of the qvh C-ABI (include/qvh.h), for tests that call the boundary directly."""

from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "quiver_amd", "lib", "libqvh.so")
HEADER = os.path.join(ROOT, "include", "qvh.h")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")


def declared_functions():
    """Names of the functions include/qvh.h declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qvh_[a-z0-9_]+)\s*\(", text)))


class Qvh:
    def __init__(self, path=LIB):
        self.lib = L = C.CDLL(path)
        L.qvh_last_error.restype = C.c_char_p
        L.qvh_init.argtypes = [C.c_int]
        L.qvh_flat_create.argtypes = [C.c_uint32, C.c_int, C.POINTER(C.c_void_p)]
        L.qvh_flat_destroy.argtypes = [C.c_void_p]
        L.qvh_flat_append.argtypes = [C.c_void_p, _f32p, C.c_uint64, C.c_void_p]
        L.qvh_flat_size.argtypes = [C.c_void_p]
        L.qvh_flat_size.restype = C.c_uint64
        L.qvh_flat_search.argtypes = [C.c_void_p, _f32p, C.c_uint64, C.c_uint32, C.c_void_p,
                                      _u32p, _f32p]
        L.qvh_flat_search_rows.argtypes = [C.c_void_p, _f32p, C.c_uint64, C.c_uint32, _u32p, C.c_uint64,
                                           _u32p, _f32p]
        L.qvh_normalize.argtypes = [_f32p, C.c_uint64, C.c_uint32]
        L.qvh_flat_last_fallbacks.argtypes = [C.c_void_p, C.POINTER(C.c_uint32)]
        L.qvh_ivfpq_last_fallbacks.argtypes = [C.c_void_p, C.POINTER(C.c_uint32)]
        _u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
        L.qvh_pq_create.argtypes = [C.c_uint32, C.c_uint32, _f32p, C.POINTER(C.c_void_p)]
        L.qvh_pq_destroy.argtypes = [C.c_void_p]
        L.qvh_pq_encode.argtypes = [C.c_void_p, _f32p, C.c_uint64, _u8p]
        L.qvh_pq_decode.argtypes = [C.c_void_p, _u8p, C.c_uint64, _f32p]
        L.qvh_pq_tables.argtypes = [C.c_void_p, _f32p, C.c_uint64, C.c_int, _f32p]
        L.qvh_pq_adc.argtypes = [C.c_void_p, _f32p, _u8p, C.c_uint64, _f32p]
        L.qvh_nearest_centroid.argtypes = [_f32p, C.c_uint64, _f32p, C.c_uint32, C.c_uint32, _u32p]
        L.qvh_points_create.argtypes = [_f32p, C.c_uint64, C.c_uint32, C.POINTER(C.c_void_p)]
        L.qvh_points_destroy.argtypes = [C.c_void_p]
        L.qvh_points_nearest.argtypes = [C.c_void_p, _f32p, C.c_uint32, C.c_int, _u32p]

    def pq(self, dim, m, codebook):
        return QvhPq(self, dim, m, codebook)

    def points_nearest(self, x, cent, max_inner_product=False):
        """qvh_points_nearest (CentroidTable::nearest_batch) of the rows of x against cent."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        cent = np.ascontiguousarray(cent, dtype=np.float32)
        h = C.c_void_p()
        self.check(self.lib.qvh_points_create(x, x.shape[0], x.shape[1], C.byref(h)))
        try:
            out = np.empty(x.shape[0], dtype=np.uint32)
            self.check(self.lib.qvh_points_nearest(h, cent, cent.shape[0], int(max_inner_product), out))
        finally:
            self.lib.qvh_points_destroy(h)
        return out

    def nearest_centroid(self, x, cent):
        """qvh_nearest_centroid of each row of x against the rows of cent."""
        x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
        cent = np.ascontiguousarray(cent, dtype=np.float32)
        out = np.empty(x.shape[0], dtype=np.uint32)
        self.check(self.lib.qvh_nearest_centroid(x, x.shape[0], cent, cent.shape[0], x.shape[1], out))
        return out

    def error(self) -> str:
        return self.lib.qvh_last_error().decode()

    def check(self, status):
        if status != 0:
            raise RuntimeError(f"qvh status {status}: {self.error()}")

    def normalize(self, x):
        x = np.array(x, dtype=np.float32, copy=True, order="C")
        self.check(self.lib.qvh_normalize(x, x.shape[0], x.shape[1]))
        return x

    def flat(self, dim, metric):
        return QvhFlat(self, dim, metric)

    def last_fallbacks(self, handle) -> int:
        """Queries of the flat handle's last MFMA-scan search that the merge sent to the exact kernel."""
        n = C.c_uint32(0)
        self.check(self.lib.qvh_flat_last_fallbacks(C.c_void_p(handle), C.byref(n)))
        return n.value

    def ivf_last_fallbacks(self, handle) -> int:
        """Queries of the IVF-PQ handle's last search whose approximate ranking was recomputed exactly."""
        n = C.c_uint32(0)
        self.check(self.lib.qvh_ivfpq_last_fallbacks(C.c_void_p(handle), C.byref(n)))
        return n.value


class QvhFlat:
    METRIC = {"l2": 0, "ip": 1, "cosine": 2}

    def __init__(self, q: Qvh, dim, metric):
        self.q, self.dim = q, dim
        h = C.c_void_p()
        q.check(q.lib.qvh_flat_create(dim, self.METRIC[metric], C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            self.q.lib.qvh_flat_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def append(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        stored = np.empty_like(x)
        self.q.check(self.q.lib.qvh_flat_append(self.h, x, x.shape[0], stored.ctypes.data_as(C.c_void_p)))
        return stored

    def size(self):
        return int(self.q.lib.qvh_flat_size(self.h))

    def search(self, queries, k, bitmap=None):
        queries = np.ascontiguousarray(queries, dtype=np.float32)
        nq = queries.shape[0]
        rows = np.empty((nq, k), dtype=np.uint32)
        dist = np.empty((nq, k), dtype=np.float32)
        bm = None if bitmap is None else np.ascontiguousarray(bitmap, dtype=np.uint64)
        self.q.check(self.q.lib.qvh_flat_search(
            self.h, queries, nq, k, None if bm is None else bm.ctypes.data_as(C.c_void_p), rows, dist))
        return rows, dist

    def search_rows(self, queries, k, rows):
        """Exact top-k over the listed rows (qvh_flat_search_rows); returns (status, rows, dist)."""
        queries = np.ascontiguousarray(queries, dtype=np.float32)
        listed = np.ascontiguousarray(rows, dtype=np.uint32)
        nq = queries.shape[0]
        out_rows = np.empty((nq, k), dtype=np.uint32)
        dist = np.empty((nq, k), dtype=np.float32)
        st = self.q.lib.qvh_flat_search_rows(self.h, queries, nq, k, listed, listed.size, out_rows, dist)
        return st, out_rows, dist


class QvhPq:
    """A qvh_pq handle: ProductQuantizer with an installed codebook [m][256][dim/m]."""

    def __init__(self, q: Qvh, dim, m, codebook):
        self.q, self.dim, self.m = q, dim, m
        h = C.c_void_p()
        q.check(q.lib.qvh_pq_create(dim, m, np.ascontiguousarray(codebook, dtype=np.float32), C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            self.q.lib.qvh_pq_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def encode(self, x):
        x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
        codes = np.empty((x.shape[0], self.m), dtype=np.uint8)
        self.q.check(self.q.lib.qvh_pq_encode(self.h, x, x.shape[0], codes))
        return codes

    def decode(self, codes):
        codes = np.ascontiguousarray(np.atleast_2d(codes), dtype=np.uint8)
        out = np.empty((codes.shape[0], self.dim), dtype=np.float32)
        self.q.check(self.q.lib.qvh_pq_decode(self.h, codes, codes.shape[0], out))
        return out

    def tables(self, queries, inner_product=False):
        queries = np.ascontiguousarray(np.atleast_2d(queries), dtype=np.float32)
        out = np.empty((queries.shape[0], self.m, 256), dtype=np.float32)
        self.q.check(self.q.lib.qvh_pq_tables(self.h, queries, queries.shape[0], int(inner_product), out))
        return out

    def adc(self, table, codes):
        codes = np.ascontiguousarray(np.atleast_2d(codes), dtype=np.uint8)
        out = np.empty(codes.shape[0], dtype=np.float32)
        self.q.check(self.q.lib.qvh_pq_adc(self.h, np.ascontiguousarray(table, dtype=np.float32), codes,
                                           codes.shape[0], out))
        return out
