"""Quiver's data-parallel search path on AMD Instinct MI355X (gfx950).

    >>> import numpy as np, quiver_amd as quiver
    >>> index = quiver.FlatIndex(dim=128, metric="l2")
    >>> index.add(np.random.rand(10_000, 128))
    >>> labels, distances = index.search(np.random.rand(5, 128), k=10)

The classes keep the reference's Python API (python/quiver/__init__.py:166-251): distances are
"smaller is closer" (squared L2 for ``"l2"``, ``1 - <q, x>`` for ``"ip"``, ``1 - cos(q, x)`` for
``"cosine"``); missing results (k larger than the index or filter) come back as label ``-1`` and
distance ``inf``. The scans run as hand-written HIP kernels on the GPU (``quiver_amd/lib/libqvh.so``);
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

__all__ = ["FlatIndex", "simd_isa"]
__version__ = "0.1.0"

ArrayLike = Union[np.ndarray, Iterable]


def _as_matrix(x: ArrayLike, dim: int) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32)
    if a.ndim == 1:
        a = a.reshape(1, -1)
    if a.ndim != 2:
        raise ValueError(f"expected a 1-D or 2-D array, got shape {a.shape}")
    if a.shape[1] != dim:
        raise ValueError(f"expected dimension {dim}, got {a.shape[1]}")
    return a


_MAX_LABEL = 2**63 - 1  # labels come back as int64, and -1 marks an empty slot


def _as_labels(labels: Optional[ArrayLike], n: Optional[int] = None) -> Optional[np.ndarray]:
    """Validate labels: integers in [0, 2**63). Accepts arrays, lists, sets, and iterators."""
    if labels is None:
        return None
    if isinstance(labels, np.ndarray):
        a = labels.reshape(-1)
        if a.dtype == object:
            return _as_labels(a.tolist(), n)
        if a.size and not np.issubdtype(a.dtype, np.integer):
            raise TypeError("labels must be integers")
        if a.size:
            if np.issubdtype(a.dtype, np.signedinteger) and a.min() < 0:
                raise ValueError("labels must be non-negative")
            if a.max() > _MAX_LABEL:
                raise ValueError("labels must be below 2**63")
        a = np.ascontiguousarray(a, dtype=np.uint64)
    else:
        # Check as Python ints before numpy sees them: numpy would turn [0, 2**63] into float64.
        items = [labels] if isinstance(labels, (int, np.integer)) else list(labels)
        for v in items:
            if isinstance(v, bool) or not isinstance(v, (int, np.integer)):
                raise TypeError("labels must be integers")
            if v < 0:
                raise ValueError("labels must be non-negative")
            if v > _MAX_LABEL:
                raise ValueError("labels must be below 2**63")
        a = np.array([int(v) for v in items], dtype=np.uint64)
    if n is not None and a.shape[0] != n:
        raise ValueError(f"got {a.shape[0]} labels for {n} vectors")
    return a


class FlatIndex:
    """Exact brute-force index; the scan is a fused FP32-MFMA GEMM + top-k kernel on the GPU."""

    def __init__(self, dim: int, metric: str = "l2", *, _native=None):
        self._index = _native if _native is not None else _quiver.FlatIndex(dim, metric)

    def add(self, vectors: ArrayLike, labels: Optional[ArrayLike] = None) -> None:
        x = _as_matrix(vectors, self.dim)
        self._index._add(x, _as_labels(labels, x.shape[0]))

    def search(self, queries: ArrayLike, k: int = 10, filter: Optional[ArrayLike] = None,
               num_threads: int = 0) -> Tuple[np.ndarray, np.ndarray]:
        q = _as_matrix(queries, self.dim)
        if k <= 0:
            raise ValueError("k must be positive")
        allowed = _as_labels(filter) if filter is not None else None
        return self._index._search(q, int(k), allowed, num_threads)

    def get_vector(self, row: int) -> np.ndarray:
        """Stored row ``row`` (normalized for cosine)."""
        return self._index.get_vector(int(row))

    def __len__(self) -> int:
        return len(self._index)

    dim = property(lambda self: self._index.dim)
    metric = property(lambda self: self._index.metric)

    def __repr__(self) -> str:
        return f"FlatIndex(dim={self.dim}, metric={self.metric!r}, size={len(self)})"
