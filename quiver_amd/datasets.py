"""Seeded synthetic workloads for the five benchmark configurations (no network, no files).

* ``gaussian``        - i.i.d. N(0, 1) float32 (1: flat L2, 10,000 x 128, 100 queries).
* ``int_mixture``     - 64-component Gaussian mixture in 128-d with means ~ U[0, 160], per-component
                        sigma ~ U[8, 32], equal weights, rounded and clipped to the integers 0..255
                        (2: flat L2 1,000,000 x 128 and 4: IVF-PQ on the same data). All L2
                        partial sums stay below 2^24, so fp32 distances are exact integers.
* ``unit_mixture``    - 256-component mixture in 100-d, component means ~ N(0, 1), shared
                        anisotropic per-dimension std exp(U[-1.5, 0.5]), each vector unit-normalized
                        (3: flat cosine 1,183,514 x 100 and 5: IVF-PQ cosine on the same data).
* ``allowed_ids``     - uniform random id subsets without replacement (the filter of 3).

Base and query sets draw from the same mixture (the component parameters depend only on the
mixture seed) with different sample seeds.
"""

from __future__ import annotations

import hashlib

import numpy as np

FLAT_SMALL = dict(n=10_000, dim=128, nq=100, base_seed=1, query_seed=2)
INT_MIX = dict(n=1_000_000, dim=128, nq=10_000, comps=64, mix_seed=10, base_seed=11, query_seed=12)
UNIT_MIX = dict(n=1_183_514, dim=100, nq=10_000, comps=256, mix_seed=20, base_seed=21,
                query_seed=22, filter_seed=23)


def gaussian(n: int, dim: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((n, dim), dtype=np.float32)


_CHUNK = 8192  # rows drawn per step; fixed so that any prefix of a set is the smaller set


def _chunks(n: int):
    for b in range(0, n, _CHUNK):
        yield b, min(n, b + _CHUNK)


def int_mixture(n: int, dim: int = 128, comps: int = 64, mix_seed: int = 10,
                seed: int = 11) -> np.ndarray:
    mrng = np.random.default_rng(mix_seed)
    means = mrng.uniform(0.0, 160.0, (comps, dim)).astype(np.float32)
    sigma = mrng.uniform(8.0, 32.0, comps).astype(np.float32)
    rng = np.random.default_rng(seed)
    out = np.empty((n, dim), dtype=np.float32)
    for b, e in _chunks(n):
        c = rng.integers(0, comps, _CHUNK)[: e - b]
        z = rng.standard_normal((_CHUNK, dim), dtype=np.float32)[: e - b]
        np.clip(np.rint(means[c] + sigma[c, None] * z), 0.0, 255.0, out=out[b:e])
    return out


def unit_mixture(n: int, dim: int = 100, comps: int = 256, mix_seed: int = 20,
                 seed: int = 21) -> np.ndarray:
    mrng = np.random.default_rng(mix_seed)
    means = mrng.standard_normal((comps, dim)).astype(np.float32)
    scale = np.exp(mrng.uniform(-1.5, 0.5, dim)).astype(np.float32)
    rng = np.random.default_rng(seed)
    out = np.empty((n, dim), dtype=np.float32)
    for b, e in _chunks(n):
        c = rng.integers(0, comps, _CHUNK)[: e - b]
        z = rng.standard_normal((_CHUNK, dim), dtype=np.float32)[: e - b]
        x = means[c] + scale[None, :] * z
        x /= np.linalg.norm(x, axis=1, keepdims=True).astype(np.float32)
        out[b:e] = x
    return out


def allowed_ids(n: int, fraction: float, seed: int = 23) -> np.ndarray:
    count = int(round(n * fraction))
    return np.sort(np.random.default_rng(seed).choice(n, count, replace=False)).astype(np.uint64)


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def flat_small():
    """(base, queries) of the 10,000 x 128 N(0,1) flat L2 workload."""
    c = FLAT_SMALL
    return gaussian(c["n"], c["dim"], c["base_seed"]), gaussian(c["nq"], c["dim"], c["query_seed"])


def int_mix(n: int = INT_MIX["n"], nq: int = INT_MIX["nq"]):
    """(base, queries) of the 1,000,000 x 128 integer-valued mixture (first n / nq rows)."""
    c = INT_MIX
    return (int_mixture(n, c["dim"], c["comps"], c["mix_seed"], c["base_seed"]),
            int_mixture(nq, c["dim"], c["comps"], c["mix_seed"], c["query_seed"]))


def unit_mix(n: int = UNIT_MIX["n"], nq: int = UNIT_MIX["nq"]):
    """(base, queries) of the 1,183,514 x 100 unit-normalized mixture (first n / nq rows)."""
    c = UNIT_MIX
    return (unit_mixture(n, c["dim"], c["comps"], c["mix_seed"], c["base_seed"]),
            unit_mixture(nq, c["dim"], c["comps"], c["mix_seed"], c["query_seed"]))
