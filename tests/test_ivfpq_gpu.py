"""IVF-PQ on the GPU vs the oracle (the C restatement of IvfPqIndex, src/ivfpq_index.cc), same
seeded inputs.

Bit-exact: k-means centroids, PQ codebooks, cell assignments, PQ codes and list order (integer and
byte outputs), and every returned distance (the scan re-scores its survivors in the reference's
arithmetic). Labels: identical except inside groups of exactly equal distance at the k-th
boundary (assert_same_topk), where the reference's order is a libstdc++ heap artifact.
"""

import numpy as np
import pytest

import quiver_amd as quiver
from oracle.oracle import IvfPqState, rows_bitmap
from parity import assert_same_topk
from quiver_amd import datasets as D
from qvh_ctypes import Qvh

pytestmark = pytest.mark.gpu


def clustered(n, dim, clusters, seed, center_seed=None):
    crng = np.random.default_rng(1000 + clusters if center_seed is None else center_seed)
    centers = (2.0 * crng.standard_normal((clusters, dim))).astype(np.float32)
    rng = np.random.default_rng(seed)
    return (centers[rng.integers(0, clusters, n)] + rng.standard_normal((n, dim))).astype(np.float32)


def build_pair(oracle, base, metric, nlist, m, store, train_n=None, iters=10):
    """Product index trained + filled on the GPU, and the oracle's state from the same data."""
    print(f"case: n={base.shape[0]} dim={base.shape[1]} metric={metric} nlist={nlist} m={m} "
          f"store={store}", flush=True)
    tn = base.shape[0] if train_n is None else train_n
    idx = quiver.IvfPqIndex(base.shape[1], metric, nlist=nlist, m=m, store_vectors=store,
                            train_iterations=iters)
    idx.train(base[:tn])
    cent, cb, pre = oracle.ivfpq_train(base[:tn], metric, nlist, m, iters, 1234)
    assert np.array_equal(idx.centroids.view(np.uint32), cent.view(np.uint32)), "centroids differ"
    assert np.array_equal(idx.codebook.view(np.uint32), cb.view(np.uint32)), "codebook differs"
    idx.add(base)
    assign, codes, stored = oracle.ivfpq_encode(cent, cb, metric, base)
    st = IvfPqState(metric, cent, cb, pre).set_lists(assign, codes, np.arange(base.shape[0], dtype=np.uint64),
                                                     stored if store else None)
    off, labels, got_codes = idx.lists()
    assert np.array_equal(off, st.offsets), "list offsets differ"
    assert np.array_equal(labels, st.labels), "list order differs"
    assert np.array_equal(got_codes, st.codes), "PQ codes differ"
    if store:
        assert np.array_equal(idx.list_vectors().view(np.uint32), st.vectors.view(np.uint32))
    return idx, st


def compare_search(oracle, idx, st, queries, k, nprobe, refine=0, allowed=None):
    got_l, got_d = idx.search(queries, k, nprobe=nprobe, refine_factor=refine, filter=allowed)
    bm = None
    if allowed is not None:
        bm = rows_bitmap(np.flatnonzero(np.isin(st.labels, allowed)), st.labels.size)
    refs, dist = oracle.ivfpq_search(st, queries, k, nprobe, refine, bm)
    exp_l = st.ref_to_label(refs)
    return assert_same_topk(got_l, got_d, exp_l, dist)


def test_kmeans_matches_oracle(oracle):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((6000, 12)).astype(np.float32)
    assert np.array_equal(quiver.kmeans(x, 40, 8, seed=3), oracle.kmeans(x, 40, 8, seed=3))
    dup = np.ones((1000, 2), np.float32)  # identical points: empty clusters get split
    dup[:20, 0] = np.arange(20)
    assert np.array_equal(quiver.kmeans(dup, 16), oracle.kmeans(dup, 16))
    # subsampling beyond k * max_points_per_centroid
    assert np.array_equal(quiver.kmeans(x, 8, 5, max_points_per_centroid=100, seed=7),
                          oracle.kmeans(x, 8, 5, max_points_per_centroid=100, seed=7))


@pytest.mark.parametrize("max_ip", [False, True])
@pytest.mark.parametrize("dim,n,k", [(128, 20_000, 2048), (100, 8_000, 300), (32, 5_000, 64), (64, 3_000, 1),
                                     (30, 4_000, 100), (16, 4_000, 256), (128, 500, 256)])
def test_points_nearest_matches_oracle(oracle, max_ip, dim, n, k):
    """CentroidTable::nearest_batch (src/internal/centroid_table.h:94-144) for a batch of points:
    the MFMA assignment (dims that are multiples of 4 from 32 to 128, batches of 1024 or more)
    with its certificate, or the exact kernel (dims 30 and 16, 500 points); cell ids bit-equal to
    the oracle."""
    print(f"case: dim={dim} n={n} k={k} max_ip={max_ip}", flush=True)
    x = clustered(n, dim, 64, 21)
    cent = clustered(k, dim, 64, 22)
    got = Qvh().points_nearest(x, cent, max_ip)
    assert np.array_equal(got, oracle.nearest(x, cent, max_ip))


@pytest.mark.parametrize("max_ip", [False, True])
def test_points_nearest_ties_fall_back_exactly(oracle, max_ip):
    """Points exactly between two centroids, points within rounding of a tie, and duplicated
    centroids: the first of equal values must win, as in the reference, which the MFMA pass
    cannot decide; it leaves those points to the exact kernel."""
    rng = np.random.default_rng(5)
    dim, k = 64, 512
    cent = rng.standard_normal((k, dim)).astype(np.float32)
    cent[300:310] = cent[10:20]                       # duplicated centroids (ties at every point near them)
    x = rng.standard_normal((6000, dim)).astype(np.float32)
    i = np.arange(2000)
    mid = (0.5 * (cent[i % 200] + cent[200 + i % 100])).astype(np.float32)
    x[:2000] = mid                                    # equidistant from two centroids (up to rounding)
    x[2000:2600] = cent[np.arange(600) % k] + np.float32(1e-6)
    x[2600:3000] = cent[np.arange(10, 20).repeat(40)]  # on a duplicated centroid
    got = Qvh().points_nearest(x, cent, max_ip)
    assert np.array_equal(got, oracle.nearest(x, cent, max_ip))


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
def test_large_batches_select_probes_exactly(oracle, metric):
    """2,000 queries (the multi-query coarse kernel and the streaming scan), a third of them
    planted exactly between two centroids so that coarse scores tie at the probe boundary, where
    ties go to the smaller list id; results equal the oracle's at every nprobe."""
    base = clustered(20_000, 64, 80, 31)
    idx, st = build_pair(oracle, base, metric, 256, 16, metric != "ip", train_n=8000, iters=6)
    q = clustered(2000, 64, 80, 32)
    cent = idx.centroids
    i = np.arange(700)
    q[:700] = (0.5 * (cent[i % 128] + cent[128 + i % 97])).astype(np.float32)
    for nprobe in (1, 8, 33, 64):
        print(f"case: {metric} nprobe={nprobe}", flush=True)
        print(compare_search(oracle, idx, st, q, 10, nprobe, refine=2 if metric != "ip" else 0))


def test_integer_points_assign_exactly(oracle):
    """Integer-valued points and integer centroids: every g is exact, so ties (common) are
    decided by the exact kernel and everything else by the MFMA pass."""
    rng = np.random.default_rng(8)
    x = rng.integers(-8, 9, (20_000, 32)).astype(np.float32)
    cent = rng.integers(-8, 9, (256, 32)).astype(np.float32)
    got = Qvh().points_nearest(x, cent)
    assert np.array_equal(got, oracle.nearest(x, cent))


@pytest.mark.parametrize("metric,store,refine", [("l2", False, 0), ("l2", True, 4), ("cosine", True, 4),
                                                 ("ip", True, 8)])
def test_ivfpq_small_matches_oracle(oracle, metric, store, refine):
    """dim 32, 10k clustered vectors, nlist 64, m 16 (the reference's IvfPqRecall setup)."""
    base = clustered(10_000, 32, 50, 6)
    q = clustered(100, 32, 50, 7)
    idx, st = build_pair(oracle, base, metric, 64, 16, store)
    for nprobe in (1, 8, 16, 64):
        print(compare_search(oracle, idx, st, q, 10, nprobe, refine))


@pytest.mark.parametrize("metric,refine", [("l2", 0), ("l2", 8), ("ip", 0), ("cosine", 2)])
def test_ivfpq_batch_sizes_and_slices(oracle, metric, refine):
    """Batches below one resident generation of blocks scan each query in slices merged by the last
    one to finish (1 query, 300); larger ones scan whole queries (6000). refine 8 keeps 80
    candidates (120 with L2's re-score margin): 256-entry queues and the block merge, on four waves
    (inner product, cosine) or eight (L2); the others take the single-wave finish."""
    base = clustered(10_000, 32, 50, 12)
    idx, st = build_pair(oracle, base, metric, 64, 16, metric != "ip")
    for nq in (1, 300, 6_000):
        q = clustered(nq, 32, 50, 13 + nq)
        print(nq, compare_search(oracle, idx, st, q, 10, 16, refine))
    allowed = np.arange(0, 10_000, 3, dtype=np.uint64)
    print("filtered", compare_search(oracle, idx, st, clustered(6_000, 32, 50, 14), 10, 16, refine, allowed))


@pytest.mark.parametrize("metric,k,refine", [("l2", 100, 0), ("l2", 170, 0), ("ip", 200, 0), ("cosine", 150, 0),
                                             ("l2", 20, 8), ("cosine", 32, 8), ("l2", 65, 0), ("ip", 256, 0)])
def test_ivfpq_large_candidate_sets(oracle, metric, k, refine):
    """Candidate sets of 129..256 (k * refine plus the re-score margin for L2) stream through
    512-entry wave queues: the same results as the oracle, for a batch of whole queries and a
    sliced small batch."""
    base = clustered(12_000, 32, 24, seed=41)
    q = clustered(700, 32, 24, seed=42)
    idx, st = build_pair(oracle, base, metric, 64, 8, refine > 0)
    for qs in (q, q[:3]):
        print(k, refine, qs.shape[0], compare_search(oracle, idx, st, qs, k, 16, refine))


@pytest.mark.parametrize("metric,k,refine", [("l2", 200, 0), ("l2", 341, 0), ("ip", 300, 0), ("ip", 512, 0),
                                             ("cosine", 400, 0), ("l2", 30, 10), ("cosine", 50, 8), ("ip", 257, 0)])
def test_ivfpq_1024_entry_queues(oracle, metric, k, refine):
    """Candidate sets of 257..512 (L2 k = 341: 341 + 170 = 511 with the re-score margin; k = 30 with
    refine 10: 450) stream through 1024-entry wave queues on eight-wave blocks: the same results as
    the oracle, for a batch of whole queries and a sliced small batch."""
    base = clustered(12_000, 32, 24, seed=45)
    q = clustered(700, 32, 24, seed=46)
    idx, st = build_pair(oracle, base, metric, 64, 8, refine > 0)
    for qs in (q, q[:3]):
        print(k, refine, qs.shape[0], compare_search(oracle, idx, st, qs, k, 16, refine))


@pytest.mark.parametrize("metric,k,refine", [("ip", 65, 0), ("ip", 100, 0), ("cosine", 128, 0), ("cosine", 12, 8),
                                             ("l2", 50, 0)])
def test_ivfpq_256_entry_queues(oracle, metric, k, refine):
    """Candidate sets of 65..128 stream through 256-entry wave queues: four-wave blocks for inner
    product and cosine, eight-wave blocks for L2 (k = 50: 75 candidates with the re-score margin),
    merged across the block's waves; whole queries and a sliced small batch against the oracle."""
    base = clustered(12_000, 32, 24, seed=43)
    q = clustered(700, 32, 24, seed=44)
    idx, st = build_pair(oracle, base, metric, 64, 8, refine > 0)
    for qs in (q, q[:3]):
        print(k, refine, qs.shape[0], compare_search(oracle, idx, st, qs, k, 16, refine))


@pytest.mark.parametrize("metric,k,refine", [("l2", 32, 0), ("l2", 33, 0), ("l2", 40, 0), ("ip", 49, 0),
                                             ("ip", 64, 0), ("cosine", 10, 5)])
def test_ivfpq_mid_candidate_sets(oracle, metric, k, refine):
    """Candidate sets of 49..64 stream through four-wave blocks with 192-entry wave queues (cut at
    128, to exactly the candidate count at the end), 48 (L2 k = 32 with its re-score margin) through
    128-entry ones: the same results as the oracle for whole queries, a sliced small batch and a
    filter."""
    base = clustered(12_000, 32, 24, seed=43)
    q = clustered(700, 32, 24, seed=44)
    idx, st = build_pair(oracle, base, metric, 64, 8, refine > 0)
    for qs in (q, q[:3]):
        print(k, refine, qs.shape[0], compare_search(oracle, idx, st, qs, k, 16, refine))
    allowed = np.arange(0, 12_000, 5, dtype=np.uint64)
    print("filtered", compare_search(oracle, idx, st, q, k, 16, refine, allowed))


@pytest.mark.parametrize("metric,k,refine", [("l2", 1000, 0), ("ip", 2000, 0), ("l2", 100, 16), ("cosine", 50, 40),
                                             ("l2", 3000, 2)])
def test_ivfpq_candidate_sets_above_1024(oracle, metric, k, refine):
    """k * refine_factor (plus the L2 re-score margin) above 1024 (the reference has no limit,
    src/ivfpq_index.cc:303-308): the block-buffer scan with an LDS candidate buffer sized to the
    selection; equal to the oracle, also for k above the probed count (empty slots)."""
    base = clustered(30_000, 32, 24, seed=43)
    q = clustered(40, 32, 24, seed=44)
    idx, st = build_pair(oracle, base, metric, 64, 8, refine > 0)
    print(k, refine, compare_search(oracle, idx, st, q, k, 32, refine))
    print(k, refine, "nprobe 2", compare_search(oracle, idx, st, q[:5], k, 2, refine))


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
@pytest.mark.parametrize("dim,m", [(45, 15), (70, 14), (23, 23)])
def test_ivfpq_refine_tail_dims(oracle, metric, dim, m):
    """Re-ranking with the stored vectors at dims whose exact sums run the 8-wide loop and a scalar
    tail with separately rounded and fused steps (45 = 32 + 8 + 4 + 1, 70 = 64 + 4 + 2, 23 = 16 + 4 + 3):
    refine 3 re-ranks on one wave (a lane per candidate), refine 8 on the eight-wave block (eight
    lanes per candidate); distances bit-identical to the oracle."""
    base = clustered(6_000, dim, 24, seed=49 + dim)
    q = clustered(200, dim, 24, seed=50 + dim)
    idx, st = build_pair(oracle, base, metric, 32, m, True, iters=3)
    for refine in (3, 8):
        for nprobe in (2, 12):
            print(refine, nprobe, compare_search(oracle, idx, st, q, 10, nprobe, refine))


@pytest.mark.parametrize("metric,k,refine", [("l2", 12_000, 0), ("ip", 20_000, 0), ("cosine", 5_000, 3)])
def test_ivfpq_candidate_sets_beyond_lds(oracle, metric, k, refine):
    """Candidate sets whose buffer does not fit LDS beside the query table (L2 k = 12,000 keeps
    18,000 for the re-score; inner product 20,000; cosine 15,000 before refine): the block-buffer
    scan keeps each work-group's buffer in global memory; equal to the oracle."""
    base = clustered(30_000, 32, 24, seed=51)
    q = clustered(12, 32, 24, seed=52)
    idx, st = build_pair(oracle, base, metric, 16, 8, refine > 0, iters=3)
    print(k, refine, compare_search(oracle, idx, st, q, k, 16, refine))
    print(k, refine, compare_search(oracle, idx, st, q, k, 5, refine))


@pytest.mark.parametrize("metric,dim,m,nlist,refine", [("l2", 512, 256, 16, 0), ("ip", 384, 192, 16, 0),
                                                       ("cosine", 512, 256, 16, 3), ("l2", 256, 256, 1100, 2)])
def test_ivfpq_more_than_128_subspaces(oracle, metric, dim, m, nlist, refine):
    """m above 128 (the reference has no limit on m, src/ivfpq_index.cc:95-103): the per-query table
    no longer fits LDS, so the block-buffer scan keeps it in global memory and sums each code 128
    sub-spaces at a time, in order. L2 with the precomputed table (its exact re-score too), inner
    product, cosine with refine, and L2 with residual tables (nlist 1100 x m 256 exceeds the
    precomputed table's 256 MiB budget)."""
    base = clustered(5_000, dim, 12, seed=60 + m)
    q = clustered(60, dim, 12, seed=61 + m)
    idx, st = build_pair(oracle, base, metric, nlist, m, refine > 0, iters=3)
    if metric == "l2":
        assert (st.precomputed is None) == (nlist == 1100)
    for nprobe in (2, 9):
        print(nprobe, compare_search(oracle, idx, st, q, 10, nprobe, refine))


@pytest.mark.parametrize("dim,m", [(120, 30), (56, 14), (21, 7), (124, 31)])
def test_ivfpq_partial_code_dwords(oracle, dim, m):
    """m not a multiple of four (the last code dword carries pad bytes) with the precomputed L2
    table: the streaming scan's exact re-score adds the list's m table rows only, never the rows of
    the list stored after it; the last list's table ends the allocation."""
    base = clustered(6_000, dim, 24, seed=47 + m)
    q = clustered(300, dim, 24, seed=48 + m)
    idx, st = build_pair(oracle, base, "l2", 24, m, False, iters=3)
    for nprobe in (1, 5, 24):
        print(compare_search(oracle, idx, st, q, 10, nprobe))


@pytest.mark.parametrize("metric,dim,m", [("l2", 3072, 96), ("cosine", 4096, 128), ("ip", 2560, 64)])
def test_ivfpq_wide_vectors(oracle, metric, dim, m):
    """Vectors wider than 2048 dims (the reference has no limit): training, encoding and search
    (residual and precomputed tables, refine) equal to the oracle."""
    base = clustered(3_000, dim, 12, seed=45)
    q = clustered(30, dim, 12, seed=46)
    idx, st = build_pair(oracle, base, metric, 16, m, metric != "ip", iters=4)
    print(compare_search(oracle, idx, st, q, 10, 8, 2 if metric != "ip" else 0))


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
def test_ivfpq_saturated_refine(oracle, metric):
    """refine_factor 2^63: k * refine_factor wraps, the reference saturates it at the stored count and
    re-ranks every probed vector exactly (tests/test_regressions.cc:101-118); past the device path's
    candidate buffer this runs as an exact scan of the probed lists."""
    base = clustered(2_000, 8, 10, 21)
    idx, st = build_pair(oracle, base, metric, 16, 4, True)
    q = base[:50]
    for nprobe in (4, 16):
        for k in (2, 10):
            print(nprobe, k, compare_search(oracle, idx, st, q, k, nprobe, 1 << 63))
    labels, _ = idx.search(base[:1], 2, nprobe=16, refine_factor=1 << 63)
    if metric == "l2":
        assert labels[0, 0] == 0  # refine over everything is exact
    allowed = np.arange(0, 2_000, 3, dtype=np.uint64)
    print("filtered", compare_search(oracle, idx, st, q, 10, 16, 1 << 63, allowed))


def test_ivfpq_filter_matches_oracle(oracle):
    base = clustered(8_000, 16, 30, 8)
    q = clustered(60, 16, 30, 9)
    idx, st = build_pair(oracle, base, "l2", 32, 8, True)
    rng = np.random.default_rng(1)
    for frac in (0.5, 0.1, 0.005):
        allowed = np.sort(rng.choice(8_000, max(1, int(8_000 * frac)), replace=False)).astype(np.uint64)
        print(frac, compare_search(oracle, idx, st, q, 10, 32, 2, allowed))


@pytest.mark.parametrize("metric,refine", [("l2", 0), ("l2", 4), ("ip", 0), ("cosine", 3)])
def test_ivfpq_filtered_codes_as_their_own_store(oracle, metric, refine):
    """A filtered search scans the admitted codes gathered into a store of their own (per-list
    counts, offsets, codes, t1 terms and stored vectors) and maps the refs back: the oracle's
    answer at densities from no admitted code to every code, for a batch of whole queries, a sliced
    small batch, k = 10 and k = 100, and nprobe 1 and 16 (lists with no admitted code included)."""
    base = clustered(12_000, 32, 24, seed=47)
    q = clustered(300, 32, 24, seed=48)
    idx, st = build_pair(oracle, base, metric, 64, 8, refine > 0)
    rng = np.random.default_rng(2)
    for frac in (0.0, 0.002, 0.05, 0.6, 1.0):
        n_allowed = int(round(12_000 * frac))
        allowed = np.sort(rng.choice(12_000, n_allowed, replace=False)).astype(np.uint64)
        for qs, k, nprobe in ((q, 10, 16), (q[:3], 10, 16), (q, 100, 16), (q, 10, 1)):
            print(frac, qs.shape[0], k, nprobe, compare_search(oracle, idx, st, qs, k, nprobe, refine, allowed))


def test_ivfpq_without_precomputed_table(oracle):
    """nlist * m * 256 floats above 256 MiB: per-list residual tables (src/ivfpq_index.cc:338-342)."""
    base = clustered(8_400, 32, 40, 10)
    q = clustered(50, 32, 40, 11)
    idx, st = build_pair(oracle, base, "l2", 8_200, 32, False, iters=3)
    assert st.precomputed is None
    print(compare_search(oracle, idx, st, q, 10, 32))


def test_ivfpq_unaligned_code_width(oracle):
    """m = 25 (dim 100): codes are not a multiple of 4 bytes."""
    base, q = D.unit_mix(12_000, 40)
    idx, st = build_pair(oracle, base, "cosine", 64, 25, True, iters=6)
    print(compare_search(oracle, idx, st, q, 10, 16, 8))


@pytest.mark.parametrize("dim,m", [(64, 16), (128, 64), (96, 96)])
def test_ivfpq_code_widths(oracle, dim, m):
    """16 code bytes of four dims (the bank-rotated scan), 64 bytes of two dims, and 96 bytes of one
    dim (past the widest streaming kernel)."""
    base = clustered(5_000, dim, 24, 40 + m)
    q = clustered(40, dim, 24, 41 + m)
    idx, st = build_pair(oracle, base, "l2", 24, m, False, iters=3)
    for nprobe in (3, 24):
        print(compare_search(oracle, idx, st, q, 10, nprobe))


def test_ivfpq_integer_mixture_l2(oracle):
    """The integer-valued mixture of the 1M x 128 workload, at 60k rows: nlist 256, m 32."""
    base, q = D.int_mix(60_000, 200)
    idx, st = build_pair(oracle, base, "l2", 256, 32, False, iters=6)
    for nprobe in (4, 32):
        print(compare_search(oracle, idx, st, q, 10, nprobe))


def test_ivfpq_incremental_adds_and_labels(oracle):
    base = clustered(5_000, 16, 20, 12)
    idx = quiver.IvfPqIndex(16, nlist=16, m=4, train_iterations=5)
    idx.train(base)
    labels = np.arange(5_000, dtype=np.uint64) * 7 + 3
    for b in range(0, 5_000, 1_300):
        idx.add(base[b:b + 1_300], labels=labels[b:b + 1_300])
    assert len(idx) == 5_000
    cent, cb = idx.centroids, idx.codebook
    assign, codes, _ = oracle.ivfpq_encode(cent, cb, "l2", base)
    st = IvfPqState("l2", cent, cb, oracle.ivfpq_precompute(cent, cb)).set_lists(assign, codes, labels)
    off, lab, got_codes = idx.lists()
    assert np.array_equal(off, st.offsets) and np.array_equal(lab, st.labels)
    assert np.array_equal(got_codes, st.codes)
    print(compare_search(oracle, idx, st, base[:30], 5, 16))


def test_set_trained_uses_given_state(oracle):
    """An index given trained state (as loading does) encodes and searches like the oracle."""
    base = clustered(4_000, 16, 20, 13)
    cent, cb, pre = oracle.ivfpq_train(base, "l2", 32, 8, 5, 99)
    idx = quiver.IvfPqIndex(16, "l2", nlist=32, m=8)
    idx.set_trained(cent, cb)
    assert idx.is_trained
    idx.add(base)
    assign, codes, _ = oracle.ivfpq_encode(cent, cb, "l2", base)
    st = IvfPqState("l2", cent, cb, pre).set_lists(assign, codes, np.arange(4_000, dtype=np.uint64))
    print(compare_search(oracle, idx, st, base[:40], 10, 8))


def test_untrained_and_empty():
    idx = quiver.IvfPqIndex(8, nlist=4, m=2)
    with pytest.raises(ValueError, match="trained"):
        idx.add(np.zeros((1, 8)))
    labels, dist = idx.search(np.zeros((2, 8)), k=3)
    assert (labels == -1).all() and np.isinf(dist).all()
    idx.train(np.random.default_rng(0).standard_normal((300, 8)).astype(np.float32))
    with pytest.raises(ValueError, match="already trained"):
        idx.train(np.random.default_rng(0).standard_normal((300, 8)).astype(np.float32))
    labels, dist = idx.search(np.zeros((2, 8)), k=3)
    assert (labels == -1).all()


@pytest.mark.parametrize("metric,refine", [("l2", 0), ("ip", 0), ("l2", 3)])
def test_every_round_improves_on_the_last(oracle, metric, refine):
    """One list whose codes come ever closer to the query in scan order: every round's candidates
    beat all earlier ones, so every wave's queue takes a full round of appends after each cut."""
    rng = np.random.default_rng(14)
    dim, n = 16, 12_288
    direction = rng.standard_normal(dim).astype(np.float32)
    direction /= np.linalg.norm(direction)
    t = np.linspace(60.0, 0.0, n, dtype=np.float32)
    base = (t[:, None] * direction[None, :] + 0.01 * rng.standard_normal((n, dim))).astype(np.float32)
    if metric == "ip":
        base = -base  # larger <q, x> later in the list
    q = (np.zeros((4, dim)) + 0.001 * rng.standard_normal((4, dim))).astype(np.float32)
    q[:, 0] += 1.0
    idx, st = build_pair(oracle, base, metric, 1, 8, refine > 0, iters=4)
    print(compare_search(oracle, idx, st, q, 10, 1, refine))


@pytest.mark.parametrize("refine", [0, 3])
def test_uncertified_ranking_is_rescanned_exactly(oracle, refine):
    """L2 with the precomputed table ranks by base + (term1 + sum qtab) and re-scores the best
    keep + margin with the reference's sum base + sum (pre + qtab) (src/ivfpq_index.cc:334-346).
    A hundred copies of one vector next to query 0 share a list and a code, more than the selection
    holds (keep + max(6, keep / 2): 16 for k = 10, 45 with refine 3), so the approximate and exact
    sums of the whole selection differ only by rounding: the keep-th exact sum is not below the
    last approximate one minus the rounding bound, the ranking is not certified, and query 0 is
    rescanned with exact sums (in a batch of whole queries and alone, as a sliced query). Every
    result equals the oracle's."""
    base = clustered(10_000, 32, 50, 61)
    q = clustered(300, 32, 50, 62)
    base[:100] = q[0] + np.float32(0.01)
    idx, st = build_pair(oracle, base, "l2", 64, 16, refine > 0)
    for qs in (q, q[:1]):
        print(qs.shape[0], compare_search(oracle, idx, st, qs, 10, 8, refine))
        assert Qvh().ivf_last_fallbacks(idx._index._device_handle) >= 1


@pytest.mark.parametrize("refine", [0, 4])
def test_real_valued_l2_rescans_are_rare(oracle, refine):
    """L2 with the precomputed table ranks by an approximate sum and re-scores its best keep +
    max(6, keep/2) in the reference's arithmetic; a query whose selection that margin cannot certify
    is rescanned exactly. On real-valued Gaussian data (not the integer mixture the margin was tuned
    on) the rescans must stay rare: at most 1% of 4,000 queries at k = 10, with and without refine,
    and the results equal the oracle's either way."""
    rng = np.random.default_rng(77)
    base = rng.standard_normal((60_000, 64)).astype(np.float32)
    q = rng.standard_normal((4_000, 64)).astype(np.float32)
    idx, st = build_pair(oracle, base, "l2", 256, 16, refine > 0, train_n=20_000, iters=6)
    for nprobe in (4, 16):
        stats = compare_search(oracle, idx, st, q, 10, nprobe, refine)
        fb = Qvh().ivf_last_fallbacks(idx._index._device_handle)
        print(f"nprobe={nprobe} refine={refine}: {fb} of {q.shape[0]} queries rescanned", stats)
        assert fb <= q.shape[0] // 100


def _given_state_pair(oracle, cent, cb, metric, base):
    """Product index installed with the given trained state and filled with `base`, and the oracle's
    state from the same arrays."""
    idx = quiver.IvfPqIndex(cent.shape[1], metric, nlist=cent.shape[0], m=cb.shape[0])
    idx.set_trained(cent, cb)
    idx.add(base)
    pre = oracle.ivfpq_precompute(cent, cb) if metric == "l2" else None
    assign, codes, _ = oracle.ivfpq_encode(cent, cb, metric, base)
    st = IvfPqState(metric, cent, cb, pre).set_lists(assign, codes, np.arange(base.shape[0], dtype=np.uint64))
    off, lab, got_codes = idx.lists()
    assert np.array_equal(off, st.offsets) and np.array_equal(lab, st.labels)
    assert np.array_equal(got_codes, st.codes)
    return idx, st


@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_coarse_bands_beyond_the_register_sort(oracle, metric):
    """Batches of 1,024 queries or more score the centroids on the matrix unit and re-score, in the
    reference's order, only the lists within the rounding bound of the nprobe-th approximate score
    (src/ivfpq_index.cc:285-300). Two centroid layouts force its rare paths, with 1,024 queries at
    one point (plus noise far below the score spacing):
    (a) 186 near lists sit in 31 of the 64 lane strides (list l is held by lane l % 64), every other
        list far away, so the nprobe-th smallest lane minimum lies far above the nprobe-th score and
        admits more candidates than the register sort holds: the nprobe-th score is found by
        selection instead;
    (b) 200 copies of one centroid tie exactly at the nearest score, a band larger than the register
        sort: every list of the query is re-scored exactly and ties go to the smaller list id.
    Probes and results equal the oracle's."""
    rng = np.random.default_rng(401)
    dim, nlist, m = 32, 512, 8
    q0 = (3.0 * rng.standard_normal(dim)).astype(np.float32)
    unit = rng.standard_normal((nlist, dim))
    unit /= np.linalg.norm(unit, axis=1, keepdims=True)
    cb = rng.standard_normal((m, 256, dim // m)).astype(np.float32)
    lists = np.arange(nlist)
    near = (lists % 64 < 31) & (lists // 64 < 6)
    assert near.sum() == 186
    layouts = {}
    if metric == "l2":
        r = np.full(nlist, 50.0)
        r[near] = 1.0 + 0.25 * rng.permutation(186)
        layouts["lanes"] = (q0[None, :] + r[:, None] * unit).astype(np.float32)
        tied = np.full(nlist, 50.0)
        tied[:200] = 1.0
        u = np.array(unit)
        u[:200] = unit[0]
        layouts["ties"] = (q0[None, :] + tied[:, None] * u).astype(np.float32)
    else:
        s = np.full(nlist, -1.0)
        s[near] = 2.0 + 0.05 * rng.permutation(186)
        layouts["lanes"] = (s[:, None] * q0[None, :] + 0.01 * unit).astype(np.float32)
        s = np.full(nlist, -1.0)
        s[:200] = 3.0
        c = s[:, None] * q0[None, :] + 0.01 * unit
        c[:200] = c[0]
        layouts["ties"] = c.astype(np.float32)
    q = (q0[None, :] + 1e-4 * rng.standard_normal((1024, dim))).astype(np.float32)
    for name, cent in layouts.items():
        base = (q0[None, :] + 2.0 * rng.standard_normal((6000, dim))).astype(np.float32)
        idx, st = _given_state_pair(oracle, cent, cb, metric, base)
        for nprobe in (16, 32, 64):
            print(f"case: {metric} {name} nprobe={nprobe}", flush=True)
            print(compare_search(oracle, idx, st, q, 10, nprobe))
