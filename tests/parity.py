"""Result comparison for top-k search outputs.

Two kinds of check:

* ``assert_same_topk`` — both sides computed the SAME float distances (the C restatement vs the
  compiled reference, or the device path vs the restatement where the arithmetic is bit-exact).
  Distances must be bit-identical. Labels must be identical except inside groups of exactly equal
  distance, whose order the reference leaves to libstdc++ heap mechanics
  (src/internal/search_util.h:26-28, src/flat_index.cc:91-97): inside a group the label SETS must
  match, and in the last (boundary) group every label must carry exactly that distance.

* ``assert_topk_within`` — the device computed distances in another summation order (MFMA GEMM
  form ||q||^2 + ||x||^2 - 2<q,x>). Distances must agree within the stated tolerance, and every
  label that differs from the expected one must be a near-tie: its true distance (recomputed in
  the reference's arithmetic) lies within the tolerance of the expected k-th distance.

Both return counters so tests can report how many adjudications happened.
"""

from __future__ import annotations

from typing import Callable, Dict, Optional

import numpy as np

INVALID = np.uint64(2**64 - 1)


def _as_u64(labels) -> np.ndarray:
    a = np.asarray(labels)
    if a.dtype == np.int64:
        return a.view(np.uint64)
    if a.dtype == np.uint32:
        out = a.astype(np.uint64)
        out[a == np.uint32(0xFFFFFFFF)] = INVALID
        return out
    return a.astype(np.uint64)


def assert_same_topk(labels_a, dist_a, labels_b, dist_b,
                     true_dist: Optional[Callable[[int, np.ndarray], np.ndarray]] = None
                     ) -> Dict[str, int]:
    """``true_dist(q, labels) -> float32 distances`` recomputes distances for boundary-group
    checks (optional; without it boundary members are only checked for distance equality)."""
    la, lb = _as_u64(labels_a), _as_u64(labels_b)
    da = np.asarray(dist_a, dtype=np.float32)
    db = np.asarray(dist_b, dtype=np.float32)
    assert la.shape == lb.shape == da.shape == db.shape, (la.shape, lb.shape)
    stats = {"queries": la.shape[0], "tie_groups": 0, "boundary_swaps": 0}
    bad = np.flatnonzero(~((da == db) | (np.isnan(da) & np.isnan(db))).all(axis=1))
    assert bad.size == 0, (
        f"{bad.size} queries differ in distances; first q={bad[0]}: {da[bad[0]]} vs {db[bad[0]]}")
    for q in np.flatnonzero((la != lb).any(axis=1)):
        row_d = da[q]
        k = row_d.size
        j = 0
        while j < k:
            e = j
            while e + 1 < k and row_d[e + 1] == row_d[j]:
                e += 1
            ga, gb = set(la[q, j:e + 1].tolist()), set(lb[q, j:e + 1].tolist())
            if ga != gb:
                boundary = e == k - 1
                assert boundary, (f"q={q}: labels differ inside an interior tie group at "
                                  f"positions {j}..{e}: {sorted(ga)} vs {sorted(gb)}")
                if true_dist is not None:
                    members = np.array(sorted((ga | gb) - {int(INVALID)}), dtype=np.uint64)
                    td = true_dist(int(q), members)
                    assert np.all(td == row_d[j]), (
                        f"q={q}: boundary labels {members} have distances {td}, not {row_d[j]}")
                stats["boundary_swaps"] += 1
            if e > j:
                stats["tie_groups"] += 1
            j = e + 1
    return stats


def assert_topk_within(labels_got, dist_got, labels_exp, dist_exp,
                       true_dist: Callable[[int, np.ndarray], np.ndarray],
                       rtol: float, atol: float) -> Dict[str, int]:
    """Device result vs expected result computed in a different float order.

    * distances: |got - exp| <= atol + rtol * |exp| position by position (sorted lists of the
      true top-k move by at most the per-element error);
    * labels: no duplicates; every label in ``got`` but not in ``exp`` has a true distance within
      tolerance of the expected k-th distance (a near-tie), and its reported distance agrees with
      its true distance within tolerance.
    """
    lg, le = _as_u64(labels_got), _as_u64(labels_exp)
    dg = np.asarray(dist_got, dtype=np.float64)
    de = np.asarray(dist_exp, dtype=np.float64)
    assert lg.shape == le.shape == dg.shape == de.shape, (lg.shape, le.shape)
    stats = {"queries": lg.shape[0], "near_ties": 0, "exact_label_rows": 0}
    both_inf = np.isinf(dg) & np.isinf(de)
    tol = atol + rtol * np.abs(np.where(np.isinf(de), 0.0, de))
    ok = both_inf | (np.abs(dg - de) <= tol)
    bad = np.flatnonzero(~ok.all(axis=1))
    assert bad.size == 0, (f"{bad.size} queries exceed tolerance; first q={bad[0]}: "
                           f"{dg[bad[0]]} vs {de[bad[0]]}")
    assert np.array_equal(lg == INVALID, le == INVALID), "padding (empty slots) differs"
    for q in range(lg.shape[0]):
        g = lg[q][lg[q] != INVALID]
        e = le[q][le[q] != INVALID]
        assert np.unique(g).size == g.size, f"q={q}: duplicate labels {g}"
        if np.array_equal(lg[q], le[q]):
            stats["exact_label_rows"] += 1
            continue
        extra = np.setdiff1d(g, e)
        if extra.size:
            kth = de[q][e.size - 1]
            td = np.asarray(true_dist(q, extra), dtype=np.float64)
            lim = atol + rtol * abs(kth)
            assert np.all(td <= kth + lim), (
                f"q={q}: labels {extra} (true dist {td}) are not near-ties of k-th {kth}")
        stats["near_ties"] += 1
    return stats
