"""Quiver's data-parallel search path on AMD Instinct MI355X (gfx950).

    >>> import numpy as np, quiver_amd as quiver
    >>> index = quiver.FlatIndex(dim=128, metric="l2")
    >>> index.add(np.random.rand(10_000, 128))
    >>> labels, distances = index.search(np.random.rand(5, 128), k=10)

The classes keep the reference's Python API (python/quiver/__init__.py:166-251): distances are
"smaller is closer" (squared L2 for ``"l2"``, ``1 - <q, x>`` for ``"ip"``, ``1 - cos(q, x)`` for
``"cosine"``); missing results (k larger than the index or filter) come back as label ``-1`` and
distance ``inf``.

``search`` also takes queries that already live in GPU memory, as a torch (ROCm) tensor: the
search is then ordered on torch's current stream of that device and the labels (int64) and
distances (float32) come back as tensors on the same device, without a round trip through host
memory. torch must be imported before quiver_amd for this: torch ships its own HIP runtime, and
memory of one runtime copy cannot be used by another (a ValueError says so). The scans run as hand-written HIP kernels on the GPU (``quiver_amd/lib/libqvh.so``);
there is no CPU fallback: without a gfx950 device, adding or searching raises ``ValueError``.
"""

from __future__ import annotations

import os
from typing import Iterable, Optional, Tuple, Union

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))


def _load_extension():
    try:
        from . import _quiver  # noqa: F401
    except ImportError as e:  # pragma: no cover - exercised only without a build
        raise ImportError(
            "quiver_amd native extension is not built; run `python -c \"import __graft_entry__ as g; "
            "g.build()\"` (or python quiver_amd/build.py) first") from e
    return _quiver


_quiver = _load_extension()
simd_isa = _quiver.simd_isa

__all__ = ["FlatIndex", "IvfPqIndex", "kmeans", "simd_isa"]
__version__ = "0.1.0"

ArrayLike = Union[np.ndarray, Iterable]


def _as_matrix(x: ArrayLike, dim: int) -> np.ndarray:
    """Vectors as a C-contiguous float32 [n, dim] matrix; a single vector may be 1-D. The messages
    are the reference's (python/quiver/__init__.py:28-36)."""
    a = np.asarray(x, dtype=np.float32)
    if a.ndim == 1:
        a = a[np.newaxis, :]
    elif a.ndim != 2:
        raise ValueError(f"expected a 1-D or 2-D array, got shape {a.shape}")
    if a.shape[1] != dim:
        raise ValueError(f"expected dimension {dim}, got {a.shape[1]}")
    return np.ascontiguousarray(a)


def _is_device_tensor(x) -> bool:
    """A torch tensor in GPU memory (torch-ROCm names HIP devices "cuda")."""
    return type(x).__module__.startswith("torch") and bool(getattr(x, "is_cuda", False))


def _hip_runtimes():
    """Paths of the HIP runtime libraries mapped into this process."""
    try:
        with open("/proc/self/maps") as f:
            return {line.split()[-1] for line in f if "libamdhip64" in line}
    except OSError:  # pragma: no cover - non-Linux
        return set()


def _device_queries(queries, dim: int, k: int):
    """Checks a device query batch the way _as_matrix and the host path check host ones."""
    import torch

    runtimes = _hip_runtimes()
    if len(runtimes) > 1:
        raise ValueError("torch and quiver_amd run on different HIP runtimes in this process "
                         f"({', '.join(sorted(runtimes))}), so device tensors cannot be shared: "
                         "import torch before quiver_amd")

    q = queries
    if q.dim() == 1:
        q = q.reshape(1, -1)
    if q.dim() != 2:
        raise ValueError(f"expected a 1-D or 2-D array, got shape {tuple(queries.shape)}")
    if q.shape[1] != dim:
        raise ValueError(f"expected dimension {dim}, got {q.shape[1]}")
    if k <= 0:
        raise ValueError("k must be positive")
    index_device = _quiver._device_index()
    if q.device.index != index_device:
        raise ValueError(f"queries are on {q.device}, the index on cuda:{index_device}")
    q = q.to(torch.float32).contiguous()
    if q.numel() and not bool(torch.isfinite(q).all()):
        raise ValueError("vectors must be finite")
    return q


def _device_results(nq: int, k: int, device):
    import torch

    return (torch.full((nq, k), -1, dtype=torch.int64, device=device),
            torch.full((nq, k), float("inf"), dtype=torch.float32, device=device))


def _on_torch_stream(device, tensors, launch) -> None:
    """Calls launch(stream) so that its device work runs after the work already queued on torch's
    current stream and before the work queued there afterwards. The library reads a null stream
    as "the handle's own stream", so torch's null stream is replaced by a side stream that joins
    it on both ends."""
    import torch

    cur = torch.cuda.current_stream(device)
    if cur.cuda_stream != 0:
        launch(cur.cuda_stream)
        return
    side = torch.cuda.Stream(device=device)
    side.wait_stream(cur)
    for t in tensors:
        if t is not None:
            t.record_stream(side)
    launch(side.cuda_stream)
    cur.wait_stream(side)


def _device_bitmap(bits: np.ndarray, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int64)).to(device)


def _device_rows(bits: np.ndarray, n: int, device):
    """The rows among the first n that a row bitmap admits (bit r % 64 of word r // 64), ascending,
    as an int32 tensor on `device` holding the rows' uint32 bits (empty when none is admitted)."""
    import torch

    flags = np.unpackbits(np.ascontiguousarray(bits).view(np.uint8), bitorder="little")[:n]
    rows = np.flatnonzero(flags).astype(np.uint32)
    return torch.from_numpy(rows.view(np.int32)).to(device)


_MAX_LABEL = 2**63 - 1  # labels come back as int64, and -1 marks an empty slot


def _check_label(v) -> None:
    """One label: an integer (bool excluded) in [0, 2**63)."""
    if isinstance(v, bool) or not isinstance(v, (int, np.integer)):
        raise TypeError("labels must be integers")
    if v < 0:
        raise ValueError("labels must be non-negative")
    if v > _MAX_LABEL:
        raise ValueError("labels must be below 2**63")


def _label_array(labels) -> np.ndarray:
    if isinstance(labels, np.ndarray) and labels.dtype != object:
        flat = labels.ravel()
        if flat.size == 0:
            return flat.astype(np.uint64)
        if not np.issubdtype(flat.dtype, np.integer):
            raise TypeError("labels must be integers")
        if flat.min() < 0:
            raise ValueError("labels must be non-negative")
        if flat.max() > _MAX_LABEL:
            raise ValueError("labels must be below 2**63")
        return flat.astype(np.uint64)
    # Python objects are checked one by one as ints: numpy would read [0, 2**63] as float64.
    if isinstance(labels, np.ndarray):
        items = labels.ravel().tolist()
    elif isinstance(labels, (int, np.integer)):
        items = [labels]
    else:
        items = list(labels)
    for v in items:
        _check_label(v)
    return np.fromiter((int(v) for v in items), dtype=np.uint64, count=len(items))


def _as_labels(labels: Optional[ArrayLike], n: Optional[int] = None) -> Optional[np.ndarray]:
    """Labels as uint64: integers in [0, 2**63) from an array, a list, a set or an iterator, with
    the reference's messages (python/quiver/__init__.py:42-72); n, when given, is the count."""
    if labels is None:
        return None
    a = _label_array(labels)
    if n is not None and a.shape[0] != n:
        raise ValueError(f"got {a.shape[0]} labels for {n} vectors")
    return a


class IvfPqIndex:
    """Inverted-file index over product-quantized residuals: ~``m`` bytes per vector.

    Args:
        dim: vector dimensionality (must be divisible by ``m``).
        metric: ``"l2"``, ``"ip"``, or ``"cosine"``.
        nlist: number of coarse cells (roughly ``4 * sqrt(n)``).
        m: bytes per vector (PQ sub-quantizers).
        store_vectors: keep float32 copies to enable exact re-ranking (``refine_factor``).

    Call :meth:`train` on a representative sample before :meth:`add`. Encoding and search run on
    the GPU; training runs the reference's k-means with its assignment steps on the GPU.
    """

    def __init__(self, dim: int, metric: str = "l2", nlist: int = 1024, m: int = 16,
                 store_vectors: bool = False, train_iterations: int = 20, seed: int = 1234,
                 *, _native=None):
        self._index = _native if _native is not None else _quiver.IvfPqIndex(
            dim, metric, nlist, m, store_vectors, train_iterations, seed)

    def train(self, vectors: ArrayLike, num_threads: int = 0) -> None:
        self._index._train(_as_matrix(vectors, self.dim), num_threads)

    def add(self, vectors: ArrayLike, labels: Optional[ArrayLike] = None, num_threads: int = 0) -> None:
        x = _as_matrix(vectors, self.dim)
        self._index._add(x, _as_labels(labels, x.shape[0]), num_threads)

    def search(self, queries: ArrayLike, k: int = 10, nprobe: int = 16, refine_factor: int = 0,
               filter: Optional[ArrayLike] = None, num_threads: int = 0) -> Tuple[np.ndarray, np.ndarray]:
        if _is_device_tensor(queries):
            return self._search_device(queries, int(k), int(nprobe), int(refine_factor), filter)
        q = _as_matrix(queries, self.dim)
        if k <= 0:
            raise ValueError("k must be positive")
        allowed = _as_labels(filter) if filter is not None else None
        return self._index._search(q, int(k), int(nprobe), int(refine_factor), allowed, num_threads)

    def _search_device(self, queries, k: int, nprobe: int, refine_factor: int, filter):
        import torch

        q = _device_queries(queries, self.dim, k)
        if refine_factor < 0:
            raise ValueError("refine_factor must be non-negative")
        labels, dist = _device_results(q.shape[0], k, q.device)
        n = len(self)
        if q.shape[0] == 0 or n == 0 or not self.is_trained:
            return labels, dist
        bitmap = None
        if filter is not None:
            bitmap = _device_bitmap(self._index._position_bitmap(_as_labels(filter)), q.device)
        refs = torch.empty((q.shape[0], k), dtype=torch.int64, device=q.device)
        _on_torch_stream(q.device, (q, bitmap, refs, dist), lambda stream: self._index._search_device(
            q.data_ptr(), q.shape[0], k, max(nprobe, 1), refine_factor, 0 if bitmap is None else bitmap.data_ptr(),
            refs.data_ptr(), dist.data_ptr(), stream))
        offsets, table = self._label_tables(q.device, n)
        found = refs != -1
        pos = offsets[(refs >> 32).clamp(0, offsets.numel() - 1)] + (refs & 0xFFFFFFFF)
        return torch.where(found, table[pos.clamp(0, n - 1)], labels), dist

    def _label_tables(self, device, n: int):
        """CSR offsets and labels on `device` (refs -> labels), rebuilt when the index grows."""
        import torch

        cached = getattr(self, "_dev_tables", None)
        if cached is None or cached[0] != (n, device):
            offsets = torch.from_numpy(self._index._list_offsets().view(np.int64)).to(device)
            table = torch.from_numpy(self._index._list_labels().view(np.int64)).to(device)
            cached = ((n, device), offsets, table)
            self._dev_tables = cached
        return cached[1], cached[2]

    def set_trained(self, centroids: ArrayLike, codebook: ArrayLike) -> None:
        """Install trained state (coarse centroids [nlist, dim], PQ codebook [m, 256, dim/m])
        instead of training, e.g. state trained elsewhere."""
        self._index._set_trained(np.ascontiguousarray(centroids, dtype=np.float32),
                                 np.ascontiguousarray(codebook, dtype=np.float32))

    @property
    def centroids(self) -> np.ndarray:
        return self._index._centroids()

    @property
    def codebook(self) -> np.ndarray:
        return self._index._codebook()

    def lists(self):
        """(offsets [nlist+1], labels, codes [n, m]) in list order."""
        return self._index._list_offsets(), self._index._list_labels(), self._index._list_codes()

    def list_vectors(self) -> np.ndarray:
        return self._index._list_vectors()

    def list_sizes(self):
        return self._index.list_sizes()

    def save(self, path: str) -> None:
        """Writes a ``.qvr`` file that the reference's ``IvfPqIndex.load`` also reads."""
        self._index.save(str(path))

    @classmethod
    def load(cls, path: str, verify_checksums: bool = True) -> "IvfPqIndex":
        """Reads a ``.qvr`` IVF-PQ file (ours or the reference's) onto the GPU."""
        return cls(0, _native=_quiver.IvfPqIndex.load(str(path), verify_checksums))

    def __len__(self) -> int:
        return len(self._index)

    dim = property(lambda self: self._index.dim)
    metric = property(lambda self: self._index.metric)
    nlist = property(lambda self: self._index.nlist)
    m = property(lambda self: self._index.m)
    is_trained = property(lambda self: self._index.is_trained)
    memory_bytes = property(lambda self: self._index.memory_bytes)

    def __repr__(self) -> str:
        return f"IvfPqIndex(dim={self.dim}, nlist={self.nlist}, m={self.m}, size={len(self)})"


def kmeans(vectors: ArrayLike, k: int, iterations: int = 25, max_points_per_centroid: int = 256,
           seed: int = 1234, num_threads: int = 0) -> np.ndarray:
    """Lloyd's k-means with the reference's initialization and empty-cluster rule (k x dim)."""
    x = np.ascontiguousarray(vectors, dtype=np.float32)
    return _quiver.kmeans(x, int(k), int(iterations), int(max_points_per_centroid), int(seed), num_threads)


class FlatIndex:
    """Exact brute-force index; the scan is a fused FP32-MFMA GEMM + top-k kernel on the GPU."""

    def __init__(self, dim: int, metric: str = "l2", *, _native=None):
        self._index = _native if _native is not None else _quiver.FlatIndex(dim, metric)

    def add(self, vectors: ArrayLike, labels: Optional[ArrayLike] = None) -> None:
        x = _as_matrix(vectors, self.dim)
        self._index._add(x, _as_labels(labels, x.shape[0]))

    def search(self, queries: ArrayLike, k: int = 10, filter: Optional[ArrayLike] = None,
               num_threads: int = 0) -> Tuple[np.ndarray, np.ndarray]:
        if _is_device_tensor(queries):
            return self._search_device(queries, int(k), filter)
        q = _as_matrix(queries, self.dim)
        if k <= 0:
            raise ValueError("k must be positive")
        allowed = _as_labels(filter) if filter is not None else None
        return self._index._search(q, int(k), allowed, num_threads)

    def _search_device(self, queries, k: int, filter):
        import torch

        q = _device_queries(queries, self.dim, k)
        labels, dist = _device_results(q.shape[0], k, q.device)
        n = len(self)
        if q.shape[0] == 0 or n == 0:
            return labels, dist
        rows = torch.empty((q.shape[0], k), dtype=torch.int32, device=q.device)
        listed = None
        if filter is not None:
            # The admitted rows, ascending, as a device list: the scan then reads only those rows.
            listed = _device_rows(self._index._row_bitmap(_as_labels(filter)), n, q.device)
        if listed is None:
            _on_torch_stream(q.device, (q, rows, dist), lambda stream: self._index._search_device(
                q.data_ptr(), q.shape[0], k, 0, rows.data_ptr(), dist.data_ptr(), stream))
        else:
            _on_torch_stream(q.device, (q, listed, rows, dist), lambda stream: self._index._search_device_rows(
                q.data_ptr(), q.shape[0], k, listed.data_ptr(), listed.numel(), rows.data_ptr(), dist.data_ptr(),
                stream))
        table = self._label_table(q.device, n)
        return torch.where(rows != -1, table[rows.clamp(0, n - 1).long()], labels), dist

    def _label_table(self, device, n: int):
        """Labels by row on `device`, rebuilt when the index grows."""
        import torch

        cached = getattr(self, "_dev_labels", None)
        if cached is None or cached[0] != (n, device):
            cached = ((n, device), torch.from_numpy(self._index._labels().view(np.int64)).to(device))
            self._dev_labels = cached
        return cached[1]

    def get_vector(self, row: int) -> np.ndarray:
        """Stored row ``row`` (normalized for cosine)."""
        return self._index.get_vector(int(row))

    def save(self, path: str) -> None:
        """Writes a ``.qvr`` file that the reference's ``FlatIndex.load`` also reads."""
        self._index.save(str(path))

    @classmethod
    def load(cls, path: str, verify_checksums: bool = True) -> "FlatIndex":
        """Reads a ``.qvr`` flat file (ours or the reference's) onto the GPU."""
        return cls(0, _native=_quiver.FlatIndex.load(str(path), verify_checksums))

    def __len__(self) -> int:
        return len(self._index)

    dim = property(lambda self: self._index.dim)
    metric = property(lambda self: self._index.metric)

    def __repr__(self) -> str:
        return f"FlatIndex(dim={self.dim}, metric={self.metric!r}, size={len(self)})"
