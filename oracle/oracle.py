"""ORACLE — test infrastructure, NOT product code.

numpy wrappers (ctypes) over two CPU checkers:

* ``Oracle`` — ``oracle/liboracle.so``, the C restatement of the reference algorithms
  (``oracle/oracle.c``; each function cites the reference file:line it follows).
* ``Reference`` — ``oracle/_ref/libquiver_ref.so``, the reference's own sources compiled in place
  by ``oracle/Makefile`` plus a C-ABI shim (``oracle/refbind/quiver_ref_capi.cc``). Used to make the
  golden fixtures and as the bench's CPU baseline. Absent where it has not been built.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg import this module.
"""

from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libquiver_ref.so")

METRICS = {"l2": 0, "ip": 1, "cosine": 2}

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(dtype=np.uint64, flags="C_CONTIGUOUS")
_sz = C.c_size_t


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def metric_id(metric) -> int:
    return METRICS[metric] if isinstance(metric, str) else int(metric)


def rows_bitmap(admitted: np.ndarray, n: int) -> np.ndarray:
    """Bitmap of ceil(n/64) u64 words with bit i set for every i in ``admitted``."""
    words = np.zeros((n + 63) // 64, dtype=np.uint64)
    idx = np.asarray(admitted, dtype=np.int64)
    idx = idx[(idx >= 0) & (idx < n)]
    np.bitwise_or.at(words, idx >> 6, np.left_shift(np.uint64(1), (idx & 63).astype(np.uint64)))
    return words


class _IvfPqStruct(C.Structure):
    _fields_ = [
        ("dim", _sz), ("nlist", _sz), ("m", _sz), ("metric", C.c_int),
        ("centroids", C.c_void_p), ("codebook", C.c_void_p), ("precomputed", C.c_void_p),
        ("offsets", C.c_void_p), ("codes", C.c_void_p), ("vectors", C.c_void_p),
    ]


class Oracle:
    """The C restatement (oracle/oracle.c)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run: make -C oracle)")
        self.lib = L = C.CDLL(path)
        L.orc_mt64_seed.argtypes = [C.c_void_p, C.c_uint64]
        L.orc_mt64_next.argtypes = [C.c_void_p]
        L.orc_mt64_next.restype = C.c_uint64
        L.orc_mt64_canonical.argtypes = [C.c_void_p]
        L.orc_mt64_canonical.restype = C.c_double
        for fn in ("orc_l2sqr_avx2", "orc_dot_avx2", "orc_l2sqr_scalar", "orc_dot_scalar"):
            getattr(L, fn).argtypes = [_f32p, _f32p, _sz]
            getattr(L, fn).restype = C.c_float
        L.orc_normalize.argtypes = [_f32p, _sz, _sz]
        L.orc_ct_l2.argtypes = [_f32p, _f32p, _sz, _sz, _f32p]
        L.orc_ct_dot.argtypes = [_f32p, _f32p, _sz, _sz, _f32p]
        L.orc_argmin_n.argtypes = [_f32p, _sz]
        L.orc_argmin_n.restype = _sz
        L.orc_nearest_centroid.argtypes = [_f32p, _f32p, _sz, _sz]
        L.orc_nearest_centroid.restype = _sz
        L.orc_nearest_batch.argtypes = [_f32p, _sz, _f32p, _sz, _sz, C.c_int, _u32p, C.c_int]
        L.orc_flat_search.argtypes = [_f32p, _sz, _sz, C.c_int, _f32p, _sz, _sz, C.c_void_p,
                                      C.c_int, _u32p, _f32p]
        L.orc_flat_pair_dist.argtypes = [_f32p, _sz, C.c_int, _f32p, _sz, _u64p, _u64p, _f32p]
        L.orc_kmeans.argtypes = [_f32p, _sz, _sz, _sz, _sz, _sz, C.c_uint64, C.c_int, _f32p]
        L.orc_pq_train.argtypes = [_f32p, _sz, _sz, _sz, _sz, C.c_uint64, C.c_int, _f32p]
        L.orc_pq_encode.argtypes = [_f32p, _sz, _sz, _f32p, _sz, _u8p, C.c_int]
        L.orc_pq_tables.argtypes = [_f32p, _sz, _sz, _f32p, _f32p, _f32p]
        L.orc_pq_adc.argtypes = [_f32p, _sz, _u8p, _sz, _f32p]
        L.orc_ivfpq_train.argtypes = [_f32p, _sz, _sz, C.c_int, _sz, _sz, _sz, C.c_uint64,
                                      C.c_int, _f32p, _f32p, C.c_void_p]
        L.orc_ivfpq_precompute.argtypes = [_f32p, _f32p, _sz, _sz, _sz, _f32p]
        L.orc_ivfpq_encode.argtypes = [_f32p, _f32p, _sz, _sz, _sz, C.c_int, _f32p, _sz, C.c_int,
                                       _u32p, _u8p, C.c_void_p]
        L.orc_ivfpq_search.argtypes = [C.c_void_p, _f32p, _sz, _sz, _sz, _sz, C.c_void_p,
                                       C.c_int, _u64p, _f32p]

    # -- engine / kernels --
    def mt64(self, seed: int, count: int) -> np.ndarray:
        st = C.create_string_buffer(312 * 8 + 16)
        self.lib.orc_mt64_seed(st, C.c_uint64(seed))
        return np.array([self.lib.orc_mt64_next(st) for _ in range(count)], dtype=np.uint64)

    def l2sqr(self, a, b) -> float:
        a, b = _f32(a), _f32(b)
        return float(self.lib.orc_l2sqr_avx2(a, b, a.size))

    def dot(self, a, b) -> float:
        a, b = _f32(a), _f32(b)
        return float(self.lib.orc_dot_avx2(a, b, a.size))

    def normalize(self, x) -> np.ndarray:
        x = np.array(x, dtype=np.float32, copy=True, order="C")
        n, d = (1, x.size) if x.ndim == 1 else x.shape
        self.lib.orc_normalize(x, n, d)
        return x

    def argmin_n(self, v) -> int:
        v = _f32(v)
        return int(self.lib.orc_argmin_n(v, v.size))

    def nearest_centroid(self, x, cent) -> np.ndarray:
        """nearest_centroid (src/product_quantizer.cc:14-27) of each row of x."""
        x, cent = _f32(np.atleast_2d(x)), _f32(cent)
        return np.array([self.lib.orc_nearest_centroid(x[i], cent, cent.shape[0], x.shape[1])
                         for i in range(x.shape[0])], dtype=np.uint32)

    def nearest(self, x, cent, max_inner_product=False, threads=0) -> np.ndarray:
        x, cent = _f32(x), _f32(cent)
        out = np.zeros(x.shape[0], dtype=np.uint32)
        self.lib.orc_nearest_batch(x, x.shape[0], cent, cent.shape[0], x.shape[1],
                                   int(max_inner_product), out, threads)
        return out

    # -- flat --
    def flat_search(self, base, queries, k, metric="l2", row_bitmap=None, threads=0
                    ) -> Tuple[np.ndarray, np.ndarray]:
        """Rows (uint32, 0xFFFFFFFF empty) and distances. ``base`` as stored (normalized for
        cosine); queries raw."""
        base, queries = _f32(base), _f32(queries)
        nq, d = queries.shape
        rows = np.empty((nq, k), dtype=np.uint32)
        dist = np.empty((nq, k), dtype=np.float32)
        bm = None if row_bitmap is None else np.ascontiguousarray(row_bitmap, dtype=np.uint64)
        self.lib.orc_flat_search(base, base.shape[0], d, metric_id(metric), queries, nq, k,
                                 _ptr(bm), threads, rows, dist)
        return rows, dist

    def flat_pair_dist(self, base, queries, qidx, ridx, metric="l2") -> np.ndarray:
        base, queries = _f32(base), _f32(queries)
        qidx = np.ascontiguousarray(qidx, dtype=np.uint64)
        ridx = np.ascontiguousarray(ridx, dtype=np.uint64)
        out = np.empty(qidx.size, dtype=np.float32)
        self.lib.orc_flat_pair_dist(base, base.shape[1], metric_id(metric), queries, qidx.size,
                                    qidx, ridx, out)
        return out

    # -- k-means / PQ --
    def kmeans(self, x, k, iterations=25, max_points_per_centroid=256, seed=1234, threads=0):
        x = _f32(x)
        out = np.empty((k, x.shape[1]), dtype=np.float32)
        rc = self.lib.orc_kmeans(x, x.shape[0], x.shape[1], k, iterations,
                                 max_points_per_centroid, C.c_uint64(seed), threads, out)
        if rc != 0:
            raise ValueError("kmeans: bad arguments")
        return out

    def pq_train(self, x, m, iterations=25, seed=1234, threads=0):
        x = _f32(x)
        d = x.shape[1]
        cb = np.empty((m, 256, d // m), dtype=np.float32)
        rc = self.lib.orc_pq_train(x, x.shape[0], d, m, iterations, C.c_uint64(seed), threads, cb)
        if rc != 0:
            raise ValueError("pq_train: bad arguments")
        return cb

    def pq_encode(self, codebook, x, threads=0) -> np.ndarray:
        codebook, x = _f32(codebook), _f32(x)
        m = codebook.shape[0]
        codes = np.empty((x.shape[0], m), dtype=np.uint8)
        self.lib.orc_pq_encode(codebook, x.shape[1], m, x, x.shape[0], codes, threads)
        return codes

    def pq_tables(self, codebook, q):
        codebook, q = _f32(codebook), _f32(q)
        m = codebook.shape[0]
        l2 = np.empty((m, 256), dtype=np.float32)
        ip = np.empty((m, 256), dtype=np.float32)
        self.lib.orc_pq_tables(codebook, q.size, m, q, l2, ip)
        return l2, ip

    def pq_adc(self, table, codes) -> np.ndarray:
        table = _f32(table)
        codes = np.ascontiguousarray(codes, dtype=np.uint8)
        out = np.empty(codes.shape[0], dtype=np.float32)
        self.lib.orc_pq_adc(table, codes.shape[1], codes, codes.shape[0], out)
        return out

    # -- IVF-PQ --
    def ivfpq_train(self, x, metric, nlist, m, iterations=20, seed=1234, threads=0):
        """(centroids, codebook, precomputed-or-None)."""
        x = _f32(x)
        n, d = x.shape
        cent = np.empty((nlist, d), dtype=np.float32)
        cb = np.empty((m, 256, d // m), dtype=np.float32)
        pre = np.empty((nlist, m, 256), dtype=np.float32) if metric_id(metric) == 0 else None
        rc = self.lib.orc_ivfpq_train(x, n, d, metric_id(metric), nlist, m, iterations,
                                      C.c_uint64(seed), threads, cent, cb, _ptr(pre))
        if rc < 0:
            raise ValueError("ivfpq_train: bad arguments")
        return cent, cb, (pre if rc == 1 else None)

    def ivfpq_precompute(self, cent, cb) -> np.ndarray:
        cent, cb = _f32(cent), _f32(cb)
        nlist, d = cent.shape
        m = cb.shape[0]
        out = np.empty((nlist, m, 256), dtype=np.float32)
        self.lib.orc_ivfpq_precompute(cent, cb, nlist, d, m, out)
        return out

    def ivfpq_encode(self, cent, cb, metric, x, threads=0):
        """(assign u32[n], codes u8[n, m], stored vectors f32[n, d])."""
        cent, cb, x = _f32(cent), _f32(cb), _f32(x)
        nlist, d = cent.shape
        m = cb.shape[0]
        n = x.shape[0]
        assign = np.empty(n, dtype=np.uint32)
        codes = np.empty((n, m), dtype=np.uint8)
        stored = np.empty((n, d), dtype=np.float32)
        self.lib.orc_ivfpq_encode(cent, cb, nlist, d, m, metric_id(metric), x, n, threads,
                                  assign, codes, _ptr(stored))
        return assign, codes, stored

    def _ivf_struct(self, ix: "IvfPqState"):
        s = _IvfPqStruct()
        s.dim, s.nlist, s.m, s.metric = ix.dim, ix.nlist, ix.m, metric_id(ix.metric)
        s.centroids, s.codebook = _ptr(ix.centroids), _ptr(ix.codebook)
        s.precomputed = _ptr(ix.precomputed)
        s.offsets, s.codes = _ptr(ix.offsets), _ptr(ix.codes)
        s.vectors = _ptr(ix.vectors)
        return s

    def ivfpq_search(self, ix: "IvfPqState", queries, k, nprobe, refine_factor=0,
                     pos_bitmap=None, threads=0):
        """(refs u64 [nq, k] = list<<32 | offset, UINT64_MAX empty; distances)."""
        queries = _f32(queries)
        nq = queries.shape[0]
        refs = np.empty((nq, k), dtype=np.uint64)
        dist = np.empty((nq, k), dtype=np.float32)
        bm = None if pos_bitmap is None else np.ascontiguousarray(pos_bitmap, dtype=np.uint64)
        s = self._ivf_struct(ix)
        self.lib.orc_ivfpq_search(C.byref(s), queries, nq, k, nprobe, refine_factor, _ptr(bm),
                                  threads, refs, dist)
        return refs, dist


class IvfPqState:
    """Trained IVF-PQ state plus CSR inverted lists (the layout of the reference's LOFF / CODE /
    LABL / VECT sections, src/ivfpq_index.cc:479-503)."""

    def __init__(self, metric, centroids, codebook, precomputed=None):
        self.metric = metric
        self.centroids = _f32(centroids)
        self.codebook = _f32(codebook)
        self.precomputed = None if precomputed is None else _f32(precomputed)
        self.nlist, self.dim = self.centroids.shape
        self.m = self.codebook.shape[0]
        self.offsets = np.zeros(self.nlist + 1, dtype=np.uint64)
        self.codes = np.zeros((0, self.m), dtype=np.uint8)
        self.labels = np.zeros(0, dtype=np.uint64)
        self.vectors = None

    def set_lists(self, assign, codes, labels, vectors=None):
        """CSR from per-vector cells, in input order within each list (Impl::add's append
        order, src/ivfpq_index.cc:263-269)."""
        assign = np.asarray(assign, dtype=np.int64)
        order = np.argsort(assign, kind="stable")
        counts = np.bincount(assign, minlength=self.nlist)
        self.offsets = np.zeros(self.nlist + 1, dtype=np.uint64)
        self.offsets[1:] = np.cumsum(counts)
        self.codes = np.ascontiguousarray(np.asarray(codes, dtype=np.uint8)[order])
        self.labels = np.ascontiguousarray(np.asarray(labels, dtype=np.uint64)[order])
        self.vectors = None if vectors is None else _f32(np.asarray(vectors)[order])
        self.order = order
        return self

    def ref_to_label(self, refs: np.ndarray) -> np.ndarray:
        refs = np.asarray(refs, dtype=np.uint64)
        out = np.full(refs.shape, np.uint64(2**64 - 1), dtype=np.uint64)
        ok = refs != np.uint64(2**64 - 1)
        lst = (refs[ok] >> np.uint64(32)).astype(np.int64)
        off = (refs[ok] & np.uint64(0xFFFFFFFF)).astype(np.int64)
        out[ok] = self.labels[self.offsets[lst].astype(np.int64) + off]
        return out


class Reference:
    """The compiled reference library (oracle/_ref/libquiver_ref.so)."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run: make -C oracle ref)")
        self.lib = L = C.CDLL(path)
        L.qref_last_error.restype = C.c_char_p
        L.qref_simd_isa.restype = C.c_char_p
        L.qref_l2sqr.argtypes = [_f32p, _f32p, _sz]
        L.qref_l2sqr.restype = C.c_float
        L.qref_dot.argtypes = [_f32p, _f32p, _sz]
        L.qref_dot.restype = C.c_float
        L.qref_normalize.argtypes = [_f32p, _sz, _sz]
        L.qref_flat_new.argtypes = [_sz, C.c_int]
        L.qref_flat_new.restype = C.c_void_p
        L.qref_flat_free.argtypes = [C.c_void_p]
        L.qref_flat_add.argtypes = [C.c_void_p, _f32p, _sz, C.c_void_p]
        L.qref_flat_search.argtypes = [C.c_void_p, _f32p, _sz, _sz, C.c_void_p, C.c_int64, _sz,
                                       _u64p, _f32p]
        L.qref_ivfpq_new.argtypes = [_sz, C.c_int, _sz, _sz, _sz, C.c_int, C.c_uint64]
        L.qref_ivfpq_new.restype = C.c_void_p
        L.qref_ivfpq_free.argtypes = [C.c_void_p]
        L.qref_ivfpq_train.argtypes = [C.c_void_p, _f32p, _sz, _sz]
        L.qref_ivfpq_add.argtypes = [C.c_void_p, _f32p, _sz, C.c_void_p, _sz]
        L.qref_ivfpq_search.argtypes = [C.c_void_p, _f32p, _sz, _sz, _sz, _sz, C.c_void_p,
                                        C.c_int64, _sz, _u64p, _f32p]
        L.qref_ivfpq_save.argtypes = [C.c_void_p, C.c_char_p]
        L.qref_flat_save.argtypes = [C.c_void_p, C.c_char_p]
        L.qref_flat_load.argtypes = [C.c_char_p, C.c_int]
        L.qref_flat_load.restype = C.c_void_p
        L.qref_flat_size.argtypes = [C.c_void_p]
        L.qref_flat_size.restype = _sz
        L.qref_ivfpq_load.argtypes = [C.c_char_p, C.c_int]
        L.qref_ivfpq_load.restype = C.c_void_p
        L.qref_ivfpq_size.argtypes = [C.c_void_p]
        L.qref_ivfpq_size.restype = _sz
        L.qref_ivfpq_memory_bytes.argtypes = [C.c_void_p]
        L.qref_ivfpq_memory_bytes.restype = _sz
        L.qref_ivfpq_list_sizes.argtypes = [C.c_void_p, C.c_void_p]
        L.qref_kmeans.argtypes = [_f32p, _sz, _sz, _sz, _sz, _sz, C.c_uint64, _sz, _f32p]
        L.qref_nearest_centroid.argtypes = [_f32p, _f32p, _sz, _sz]
        L.qref_nearest_centroid.restype = _sz
        L.qref_pq_encode.argtypes = [_sz, _sz, _f32p, _f32p, _sz, _u8p]
        L.qref_pq_tables.argtypes = [_sz, _sz, _f32p, _f32p, _f32p, _f32p]
        L.qref_pq_adc.argtypes = [_sz, _sz, _f32p, _f32p, _u8p, _sz, _f32p, _f32p]
        L.qref_pq_train.argtypes = [_sz, _sz, _f32p, _sz, _sz, C.c_uint64, _sz, _f32p]

    def _check(self, rc):
        if rc != 0:
            raise ValueError(self.lib.qref_last_error().decode())

    @property
    def simd_isa(self) -> str:
        return self.lib.qref_simd_isa().decode()

    def l2sqr(self, a, b):
        a, b = _f32(a), _f32(b)
        return float(self.lib.qref_l2sqr(a, b, a.size))

    def dot(self, a, b):
        a, b = _f32(a), _f32(b)
        return float(self.lib.qref_dot(a, b, a.size))

    def normalize(self, x):
        x = np.array(x, dtype=np.float32, copy=True, order="C")
        n, d = (1, x.size) if x.ndim == 1 else x.shape
        self.lib.qref_normalize(x, n, d)
        return x

    def flat(self, dim, metric="l2"):
        return RefFlat(self, dim, metric)

    def flat_load(self, path, verify_checksums=True):
        """FlatIndex::load of the reference (src/flat_index.cc:155-176)."""
        return RefFlat(self, 0, None, handle=self._load(self.lib.qref_flat_load, path, verify_checksums))

    def ivfpq_load(self, path, verify_checksums=True):
        """IvfPqIndex::load of the reference (src/ivfpq_index.cc:507-576)."""
        return RefIvfPq(self, 0, None, 0, 0, 0, False, 0,
                        handle=self._load(self.lib.qref_ivfpq_load, path, verify_checksums))

    def _load(self, fn, path, verify):
        h = fn(str(path).encode(), int(bool(verify)))
        if not h:
            raise ValueError(self.lib.qref_last_error().decode())
        return h

    def ivfpq(self, dim, metric="l2", nlist=1024, m=16, train_iterations=20,
              store_vectors=False, seed=1234):
        return RefIvfPq(self, dim, metric, nlist, m, train_iterations, store_vectors, seed)

    def kmeans(self, x, k, iterations=25, max_points_per_centroid=256, seed=1234, threads=0):
        x = _f32(x)
        out = np.empty((k, x.shape[1]), dtype=np.float32)
        self._check(self.lib.qref_kmeans(x, x.shape[0], x.shape[1], k, iterations,
                                         max_points_per_centroid, C.c_uint64(seed), threads, out))
        return out

    def nearest_centroid(self, x, cent) -> np.ndarray:
        x, cent = _f32(np.atleast_2d(x)), _f32(cent)
        return np.array([self.lib.qref_nearest_centroid(np.ascontiguousarray(x[i]), cent, cent.shape[0], x.shape[1])
                         for i in range(x.shape[0])], dtype=np.uint32)

    def pq_train(self, x, m, iterations=25, seed=1234, threads=0):
        x = _f32(x)
        d = x.shape[1]
        cb = np.empty((m, 256, d // m), dtype=np.float32)
        self._check(self.lib.qref_pq_train(d, m, x, x.shape[0], iterations, C.c_uint64(seed),
                                           threads, cb))
        return cb

    def pq_encode(self, codebook, x):
        codebook, x = _f32(codebook), _f32(x)
        m = codebook.shape[0]
        codes = np.empty((x.shape[0], m), dtype=np.uint8)
        self._check(self.lib.qref_pq_encode(x.shape[1], m, codebook, x, x.shape[0], codes))
        return codes

    def pq_tables(self, codebook, q):
        codebook, q = _f32(codebook), _f32(q)
        m = codebook.shape[0]
        l2 = np.empty((m, 256), dtype=np.float32)
        ip = np.empty((m, 256), dtype=np.float32)
        self._check(self.lib.qref_pq_tables(q.size, m, codebook, q, l2, ip))
        return l2, ip

    def pq_adc(self, codebook, table, codes):
        codebook, table = _f32(codebook), _f32(table)
        codes = np.ascontiguousarray(codes, dtype=np.uint8)
        m = codebook.shape[0]
        n = codes.shape[0]
        b = np.empty(n, dtype=np.float32)
        s = np.empty(n, dtype=np.float32)
        self._check(self.lib.qref_pq_adc(m * codebook.shape[2], m, codebook, table, codes, n, b, s))
        return b, s


def _labels_arg(allowed):
    if allowed is None:
        return None, -1
    a = np.ascontiguousarray(np.asarray(list(allowed) if not isinstance(allowed, np.ndarray)
                                        else allowed, dtype=np.uint64))
    return a, a.size


class RefFlat:
    def __init__(self, ref: Reference, dim, metric, handle=None):
        self.ref, self.dim = ref, dim
        self.h = handle if handle else ref.lib.qref_flat_new(dim, metric_id(metric))
        if not self.h:
            raise ValueError(ref.lib.qref_last_error().decode())

    def __del__(self):
        if getattr(self, "h", None):
            self.ref.lib.qref_flat_free(self.h)
            self.h = None

    def add(self, x, labels=None):
        x = _f32(x)
        lab = None if labels is None else np.ascontiguousarray(labels, dtype=np.uint64)
        self.ref._check(self.ref.lib.qref_flat_add(self.h, x, x.shape[0], _ptr(lab)))

    def search(self, q, k, allowed=None, threads=0):
        q = _f32(q)
        nq = q.shape[0]
        labels = np.empty((nq, k), dtype=np.uint64)
        dist = np.empty((nq, k), dtype=np.float32)
        a, na = _labels_arg(allowed)
        self.ref._check(self.ref.lib.qref_flat_search(self.h, q, nq, k, _ptr(a), na, threads,
                                                      labels, dist))
        return labels, dist

    def save(self, path):
        self.ref._check(self.ref.lib.qref_flat_save(self.h, str(path).encode()))

    def __len__(self):
        return int(self.ref.lib.qref_flat_size(self.h))


class RefIvfPq:
    def __init__(self, ref: Reference, dim, metric, nlist, m, iters, store_vectors, seed,
                 handle=None):
        self.ref, self.dim = ref, dim
        self.h = handle if handle else ref.lib.qref_ivfpq_new(
            dim, metric_id(metric), nlist, m, iters, int(store_vectors), C.c_uint64(seed))
        if not self.h:
            raise ValueError(ref.lib.qref_last_error().decode())

    def __del__(self):
        if getattr(self, "h", None):
            self.ref.lib.qref_ivfpq_free(self.h)
            self.h = None

    def train(self, x, threads=0):
        x = _f32(x)
        self.ref._check(self.ref.lib.qref_ivfpq_train(self.h, x, x.shape[0], threads))

    def add(self, x, labels=None, threads=0):
        x = _f32(x)
        lab = None if labels is None else np.ascontiguousarray(labels, dtype=np.uint64)
        self.ref._check(self.ref.lib.qref_ivfpq_add(self.h, x, x.shape[0], _ptr(lab), threads))

    def search(self, q, k, nprobe=16, refine_factor=0, allowed=None, threads=0):
        q = _f32(q)
        nq = q.shape[0]
        labels = np.empty((nq, k), dtype=np.uint64)
        dist = np.empty((nq, k), dtype=np.float32)
        a, na = _labels_arg(allowed)
        self.ref._check(self.ref.lib.qref_ivfpq_search(self.h, q, nq, k, nprobe, refine_factor,
                                                       _ptr(a), na, threads, labels, dist))
        return labels, dist

    def save(self, path):
        self.ref._check(self.ref.lib.qref_ivfpq_save(self.h, str(path).encode()))

    def __len__(self):
        return int(self.ref.lib.qref_ivfpq_size(self.h))

    @property
    def memory_bytes(self) -> int:
        return int(self.ref.lib.qref_ivfpq_memory_bytes(self.h))

    def list_sizes(self, nlist: int) -> np.ndarray:
        out = np.zeros(nlist, dtype=np.uint64)
        self.ref.lib.qref_ivfpq_list_sizes(self.h, out.ctypes.data_as(C.c_void_p))
        return out
