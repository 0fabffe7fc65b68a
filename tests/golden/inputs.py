"""Seeded inputs of the golden fixtures, shared by make_golden.py (which runs the compiled
reference on them) and the tests (which run the oracle and the device path on them). Each
fixture also records the SHA-256 of the inputs it was made from."""

from __future__ import annotations

import hashlib

import numpy as np


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def kernel_pairs():
    """70 pairs of vectors; pair i is compared over its first i + 1 dimensions."""
    rng = np.random.default_rng(40)
    return rng.standard_normal((70, 70)).astype(np.float32), rng.standard_normal((70, 70)).astype(np.float32)


def normalize_rows(d: int):
    """64 rows of dimension d at scales 0.01..100, with a zero row, an overflowing row (its
    float dot product is infinite) and a row whose dot product underflows."""
    rng = np.random.default_rng(41 + d)
    x = (rng.standard_normal((64, d)) * rng.uniform(0.01, 100, (64, 1))).astype(np.float32)
    x[0] = 0.0
    x[1] = 3.0e19
    x[2, :] = 0.0
    x[2, 0] = 1.0e-30
    return x


NORMALIZE_DIMS = (3, 7, 100, 128)


def kmeans_points():
    x = np.random.default_rng(0).standard_normal((3000, 12)).astype(np.float32)
    dup = np.ones((1000, 2), np.float32)  # identical points: empty clusters get split
    dup[:20, 0] = np.arange(20)
    return x, dup


def pq_points():
    return (np.random.default_rng(5).standard_normal((4000, 16)).astype(np.float32),
            np.random.default_rng(6).standard_normal((5, 16)).astype(np.float32))


def clustered(n, dim, seed):
    centers = (2.0 * np.random.default_rng(77).standard_normal((30, dim))).astype(np.float32)
    rng = np.random.default_rng(seed)
    return (centers[rng.integers(0, 30, n)] + rng.standard_normal((n, dim))).astype(np.float32)


def ivf_points():
    return clustered(4000, 32, 1), clustered(60, 32, 2)


IVF_CASES = [  # (name, metric, store_vectors, refine_factor)
    ("l2", "l2", False, 0),
    ("l2r", "l2", True, 4),
    ("cos", "cosine", True, 8),
    ("ip", "ip", False, 0),
]
IVF_NLIST, IVF_M, IVF_ITERS = 32, 8, 6
IVF_NPROBES = (1, 8, 32)


def flat_filter(n: int):
    return np.sort(np.random.default_rng(3).choice(n, 1000, replace=False)).astype(np.uint64)


def few_rows():
    return np.random.default_rng(4).standard_normal((10, 8)).astype(np.float32)


def int_mix_sample(n: int):
    """Training rows of the 1M-row IVF-PQ workload: the first 100,000 of a seeded permutation."""
    return np.random.default_rng(31).permutation(n)[:100_000]


def nearest_centroid_cases():
    """(points, centroids) pairs for nearest_centroid: dims that take every branch of the AVX2
    reduction (32-element blocks, 8-element blocks, the tail), duplicated centroids (the first of
    equal distances wins), and centroids so large that some or all distances overflow to +inf."""
    rng = np.random.default_rng(61)
    cases = []
    for n, k, dim in ((200, 50, 37), (100, 300, 128), (150, 40, 3), (80, 64, 70)):
        cases.append((rng.standard_normal((n, dim)).astype(np.float32),
                      rng.standard_normal((k, dim)).astype(np.float32)))
    rows = rng.standard_normal((20, 16)).astype(np.float32)
    twins = np.repeat(rows, 2, axis=0)
    cases.append(((rows + 1e-3 * rng.standard_normal(rows.shape)).astype(np.float32), twins))
    big = rng.standard_normal((12, 8)).astype(np.float32)
    big[:6] *= np.float32(3e37)
    pts = rng.standard_normal((10, 8)).astype(np.float32)
    pts[0] = np.float32(3e37)
    cases.append((pts, big))
    allbig = np.full((5, 8), np.float32(3e38))
    allbig[::2] *= -1
    cases.append((np.zeros((3, 8), np.float32), allbig))
    return cases
