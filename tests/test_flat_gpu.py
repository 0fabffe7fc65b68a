"""Flat exact search on the GPU vs the oracle (the C restatement of FlatIndex::search_batch,
src/flat_index.cc:69-140), on the same seeded inputs.

The device returns distances re-scored in the reference's own arithmetic, so they must be
bit-identical to the oracle's for the same rows, and the (distance, row) order makes the rows
identical too: assert_same_topk allows label differences only inside groups of exactly equal
distance at the k-th boundary, and checks that boundary members really carry that distance.
"""

import numpy as np
import pytest

import quiver_amd as quiver
from oracle.oracle import rows_bitmap
from parity import assert_same_topk
from quiver_amd import datasets as D
from qvh_ctypes import Qvh

pytestmark = pytest.mark.gpu


def _true_dist(oracle, stored, queries, metric):
    def f(qi, labels):
        return oracle.flat_pair_dist(stored, queries, np.full(labels.size, qi), labels, metric)
    return f


def _device_path_matches_host_path(idx, queries, k, allowed):
    """The same filtered search with torch device queries (the admitted rows as a device list) and
    with host queries (the rows listed on the host): identical rows and bit-identical distances.
    The device bitmap form is compared with both in test_device_filters_gpu.py."""
    import torch

    hl, hd = idx.search(queries, k, filter=allowed)
    dl, dd = idx.search(torch.from_numpy(np.ascontiguousarray(queries)).to("cuda:0"), k, filter=allowed)
    assert np.array_equal(dl.cpu().numpy(), hl)
    assert np.array_equal(dd.cpu().numpy().view(np.uint32), hd.view(np.uint32))


def _check(oracle, base, queries, k, metric, allowed=None, labels=None):
    print(f"case: n={base.shape[0]} dim={base.shape[1]} nq={queries.shape[0]} k={k} "
          f"metric={metric} filtered={allowed is not None}", flush=True)
    idx = quiver.FlatIndex(base.shape[1], metric)
    idx.add(base, labels=labels)
    got_l, got_d = idx.search(queries, k, filter=allowed)
    stored = oracle.normalize(base) if metric == "cosine" else base
    bm = None
    if allowed is not None:
        lab = np.arange(base.shape[0], dtype=np.uint64) if labels is None else labels
        bm = rows_bitmap(np.flatnonzero(np.isin(lab, allowed)), base.shape[0])
    rows, dist = oracle.flat_search(stored, queries, k, metric, bm)
    if labels is None:
        exp_l = rows.astype(np.int64)
        exp_l[rows == np.uint32(0xFFFFFFFF)] = -1
    else:
        exp_l = np.where(rows == np.uint32(0xFFFFFFFF), np.uint64(2**64 - 1),
                         labels[np.minimum(rows, base.shape[0] - 1)]).view(np.int64)
    stats = assert_same_topk(got_l, got_d, exp_l, dist,
                             None if labels is not None else _true_dist(oracle, stored, queries, metric))
    return stats


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
@pytest.mark.parametrize("filtered", [False, True])
def test_flat_gaussian_10k_matches_oracle(oracle, metric, filtered):
    """10,000 x 128 N(0,1), 100 queries, k=10 (the reference's CPU-runnable case)."""
    base, q = D.flat_small()
    allowed = D.allowed_ids(base.shape[0], 0.1, seed=5) if filtered else None
    stats = _check(oracle, base, q, 10, metric, allowed)
    print(stats)


@pytest.mark.parametrize("metric", ["l2", "ip"])
@pytest.mark.parametrize("k", [1, 10, 11])
def test_integer_stores_short_lists(oracle, metric, k):
    """On a store of small integers, a batch of small-integer queries has exact GEMM-form distances
    and scans with 10-entry lane lists for k <= 10 (no margin, nothing to certify: no fallback); a
    batch holding any real-valued query takes the 16-entry lists with the margin instead (the
    device picks between the two launches). Integer, real-valued and mixed batches, and filtered
    searches through host and device buffers, against the oracle, with ties (integer data has many)
    resolved by row."""
    base, q_int = D.int_mix(40_000, 150)
    q_real = q_int[:100] + np.random.default_rng(3).standard_normal((100, base.shape[1])).astype(np.float32) * 0.37
    q_mixed = np.concatenate([q_int[100:], q_real[:3]])
    idx = quiver.FlatIndex(base.shape[1], metric)
    idx.add(base)
    for name, q in (("integer", q_int), ("real", q_real), ("mixed", q_mixed)):
        print(name, _check(oracle, base, q, k, metric))
        idx.search(q, k)
        fallbacks = Qvh().last_fallbacks(idx._index._device_handle)
        print(name, "fallbacks", fallbacks)
        if name == "integer":
            assert fallbacks == 0
        else:
            # the margin certifies all but near-ties (here the rounding bound is ~180 on squared
            # distances of ~1e5 between dense integer rows); without it nearly every query would fall back
            assert fallbacks <= 0.1 * q.shape[0], fallbacks
    rng = np.random.default_rng(4)
    for n_allowed in (4_000, 24_000):
        allowed = np.sort(rng.choice(40_000, n_allowed, replace=False)).astype(np.uint64)
        print(_check(oracle, base, q_int, k, metric, allowed))
        _device_path_matches_host_path(idx, q_int, k, allowed)


@pytest.mark.parametrize("fraction", [0.005, 0.3, 0.49, 0.7, 0.97, 1.0])
@pytest.mark.parametrize("metric", ["l2", "cosine"])
def test_filter_densities(oracle, fraction, metric):
    """A filter runs over the list of admitted rows at any density, through host and device buffers
    alike (a filter admitting every row runs as no filter). Both give the oracle's answer."""
    base, q = D.unit_mix(30_000, 50)
    allowed = D.allowed_ids(base.shape[0], fraction, seed=17)
    print(_check(oracle, base, q, 10, metric, allowed))
    idx = quiver.FlatIndex(base.shape[1], metric)
    idx.add(base)
    _device_path_matches_host_path(idx, q, 10, allowed)


def test_cosine_rows_are_normalized_like_the_reference(oracle):
    base, _ = D.flat_small()
    idx = quiver.FlatIndex(128, "cosine")
    idx.add(base[:500])
    exp = oracle.normalize(base[:500])
    got = np.stack([idx.get_vector(i) for i in range(500)])
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_normalize_entry_point_is_bit_exact(oracle):
    rng = np.random.default_rng(7)
    for d in (1, 3, 4, 7, 13, 31, 100, 128, 257):
        x = (rng.standard_normal((300, d)) * rng.uniform(1e-3, 1e3, (300, 1))).astype(np.float32)
        x[0] = 0.0  # zero vector stays zero
        x[1, 0] = 3e19  # squares overflow float: the double-precision branch
        got = Qvh().normalize(x)
        exp = oracle.normalize(x)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), d


@pytest.mark.parametrize("dim", [1, 5, 13, 16, 24, 33, 50, 64, 70, 85, 100, 117, 127, 128])
def test_awkward_dimensions(oracle, dim):
    """Rows padded to a multiple of 8 up to 128 dims (at least 16): every register-scan width from
    16 to 128 in steps of 8 is met (33 -> 40, 50 -> 56, 70 -> 72, 85 -> 88, 100 -> 104, 117 -> 120)."""
    rng = np.random.default_rng(dim)
    base = rng.standard_normal((3000, dim)).astype(np.float32)
    q = rng.standard_normal((37, dim)).astype(np.float32)
    for metric in ("l2", "ip"):
        _check(oracle, base, q, 7, metric)


@pytest.mark.parametrize("dim", [50, 100, 117])
@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
def test_eight_padded_widths_full_blocks(oracle, dim, metric):
    """Rows padded to 56, 104 and 120 floats under whole 256-query blocks of the MFMA scan (the
    full-tile form, several row splits), unfiltered and with a 60% filter."""
    rng = np.random.default_rng(300 + dim)
    base = rng.standard_normal((40_000, dim)).astype(np.float32)
    q = rng.standard_normal((400, dim)).astype(np.float32)
    print(_check(oracle, base, q, 10, metric))
    allowed = np.sort(rng.choice(40_000, 24_000, replace=False)).astype(np.uint64)
    print(_check(oracle, base, q, 10, metric, allowed))


@pytest.mark.parametrize("dim", [129, 200, 257, 384, 768, 1000, 1024])
@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
def test_dimensions_above_the_register_width(oracle, dim, metric):
    """dim > 128: the chunked MFMA scan (32-dim chunks of rows and queries staged through LDS) over
    20k rows in several splits; k = 10 with the shared bound, a 10% filter (listed rows), a 60%
    filter (bitmap) and k = 40 (unshared lists, wide merge); the merge re-scores in the reference's
    order, so distances are bit-identical."""
    rng = np.random.default_rng(dim)
    base = rng.standard_normal((20_000, dim)).astype(np.float32)
    q = rng.standard_normal((300, dim)).astype(np.float32)
    print(_check(oracle, base, q, 10, metric))
    allowed = np.sort(rng.choice(20_000, 2_000, replace=False)).astype(np.uint64)
    print(_check(oracle, base, q, 7, metric, allowed))
    allowed = np.sort(rng.choice(20_000, 12_000, replace=False)).astype(np.uint64)
    print(_check(oracle, base, q[:100], 5, metric, allowed))
    print(_check(oracle, base, q[:50], 40, metric))


def test_wide_rows_integer_data_and_ties(oracle):
    """Integer-valued 256-d rows with duplicated rows (exact ties resolve to the smaller row) on the
    chunked scan, and a batch of 17 queries (above the few-query kernel's batch limit of 8)."""
    rng = np.random.default_rng(77)
    base = rng.integers(0, 16, (30_000, 256)).astype(np.float32)
    base[15_000:15_500] = base[:500]
    q = base[rng.choice(30_000, 400, replace=False)] + rng.integers(-1, 2, (400, 256)).astype(np.float32)
    print(_check(oracle, base, q, 10, "l2"))
    print(_check(oracle, base, q[:17], 10, "l2"))


@pytest.mark.parametrize("k", [33, 64, 100, 256, 300, 1024])
@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
def test_large_k(oracle, k, metric):
    """33 <= k <= 256: the MFMA scan with unshared 32-entry lists and the wide merge; larger k: the
    general exact kernel (queue cuts at k). Ties by row either way."""
    base, q = D.int_mix(20_000, 30)
    print(_check(oracle, base, q, k, metric))
    allowed = D.allowed_ids(base.shape[0], 0.02, seed=9)
    print(_check(oracle, base, q, k, metric, allowed))


@pytest.mark.parametrize("metric", ["l2", "cosine"])
def test_large_k_crowded_lists_fall_back_exactly(oracle, metric):
    """200 near-copies of query 0 in consecutive rows: its 100 nearest crowd one split's 32-entry
    lists, so the wide merge hands that query to the exact kernel while the others stay on the
    MFMA path (40 queries: above the few-query kernel's 8); every result still equals the
    oracle's."""
    base, q = D.int_mix(40_000, 40)
    base = base.copy()
    noise = np.random.default_rng(3).integers(-1, 2, (200, base.shape[1]))
    base[5_000:5_200] = np.clip(q[0] + noise, 0, 255)
    stored = oracle.normalize(base) if metric == "cosine" else base
    idx = quiver.FlatIndex(base.shape[1], metric)
    idx.add(base)
    for k in (100, 40):
        print(f"case: crowded lists k={k} metric={metric}", flush=True)
        got_l, got_d = idx.search(q, k)
        if k == 100:  # more than the ~4 crowded lists' 4 x 32 entries can give: query 0 falls back
            assert Qvh().last_fallbacks(idx._index._device_handle) >= 1
        rows, dist = oracle.flat_search(stored, q, k, metric)
        print(assert_same_topk(got_l, got_d, rows.astype(np.int64), dist, _true_dist(oracle, stored, q, metric)))
    idx.search(q[1:], 100)
    assert Qvh().last_fallbacks(idx._index._device_handle) == 0  # no crowded query: no fallback


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
def test_k_above_1024_sorts_every_row(oracle, metric):
    """k above 1024 (the reference has no limit, src/flat_index.cc:84-107): every admitted row is
    scored and the keys sorted on the device. Integer mixture (many exact ties, resolved by row),
    k = 1025 and 5000, a 10% filter (listed rows), a 70% filter (bitmap), and k above the row
    count (empty slots)."""
    base, q = D.int_mix(20_000, 12)
    print(_check(oracle, base, q, 1025, metric))
    print(_check(oracle, base, q[:3], 5000, metric, D.allowed_ids(base.shape[0], 0.1, seed=4)))
    print(_check(oracle, base, q[:3], 2000, metric, D.allowed_ids(base.shape[0], 0.7, seed=6)))
    print(_check(oracle, base[:3000], q[:2], 4000, metric))


@pytest.mark.parametrize("k", [1, 2, 10, 16, 17, 32])
def test_k_values(oracle, k):
    base, q = D.flat_small()
    _check(oracle, base[:4000], q[:50], k, "l2")


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
@pytest.mark.parametrize("nq,k,n", [(1, 10, 700_000), (3, 1, 50_000), (8, 100, 200_000), (2, 1024, 30_000),
                                    (5, 10, 2_048), (1, 10, 2_047), (3, 200, 500_000), (1, 256, 30_000)])
def test_small_batches_split_rows(oracle, metric, nq, k, n):
    """Batches of at most eight queries split each query's rows over up to 1024 work-groups and
    merge the sorted partial lists (2,047 rows: too few to split, one work-group per query). k up
    to 256 merges by selection below the k-th list head; k = 256 over 32 lists gathers more keys
    than the buffer holds and takes the sequential merge; k = 1024 always does."""
    base = D.gaussian(n, 16, seed=31)
    q = D.gaussian(nq, 16, seed=32)
    print(_check(oracle, base, q, k, metric))


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
@pytest.mark.parametrize("dim,nq,k,n", [(32, 1, 10, 700_000), (40, 2, 64, 100_000), (47, 3, 1, 60_000),
                                        (61, 8, 33, 120_000), (100, 5, 10, 2_048), (128, 4, 20, 150_000),
                                        (159, 7, 64, 50_000), (96, 6, 16, 33_333), (64, 11, 10, 80_000),
                                        (128, 12, 64, 40_000), (128, 3, 100, 200_000), (64, 8, 128, 60_000),
                                        (100, 2, 100, 50_000)])
def test_few_query_coalesced_scan(oracle, metric, dim, nq, k, n):
    """At most eight queries with 32 <= dim <= 159 and k <= 64: eight lanes per row replay the
    reference's accumulation order (32-element blocks, 8-element blocks, the rounded and fused
    tail: dims 40, 47 and 61 take every branch); each launch reads a row once for up to eight
    queries (11 and 12 queries: the row-split MFMA scan). k up to 128 for dims that are multiples
    of 32 (256-entry queues); dim 100 with k = 100 takes the split exact kernel."""
    base = D.gaussian(n, dim, seed=33)
    q = D.gaussian(nq, dim, seed=34)
    print(_check(oracle, base, q, k, metric))


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
@pytest.mark.parametrize("nq", [9, 16, 32, 64, 100])
def test_small_batches_on_256_row_splits(oracle, metric, nq):
    """Up to 32 queries: the ring scan over 73 splits of 4,096 rows; 33 to 128: one block of the
    MFMA scan in its row-split form (the two waves of a 32-query group take the two halves of each
    tile, and the odd wave's lists join the even wave's through LDS) over up to 256 splits. Either
    way the merge takes two lane lists per query and split. Integer data adds exact ties across
    splits, waves and tile halves."""
    base = D.gaussian(300_000, 128, seed=35)
    q = D.gaussian(nq, 128, seed=36)
    print(_check(oracle, base, q, 10, metric))
    ib, iq = D.int_mix(300_000, nq)
    print(_check(oracle, ib, iq, 10, metric))


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
@pytest.mark.parametrize("k", [22, 32, 43, 44])
def test_wide_k_shared_bound(oracle, metric, k):
    """k from 22 to 43 (the wide merge's k + max(16, k / 2) keys at most 64): the register scan's
    32-entry lane lists share a bound of rank ceil(R / 2) across the lane pair and the row splits;
    k = 44 keeps no shared bound. Real-valued and integer data (exact ties across splits), a full
    query block and a partial one, against the oracle."""
    base = D.gaussian(300_000, 96, seed=71)
    q = D.gaussian(300, 96, seed=72)
    print(_check(oracle, base, q, k, metric))
    if metric == "l2":
        ib, iq = D.int_mix(300_000, 300)
        print(_check(oracle, ib, iq, k, metric))


@pytest.mark.parametrize("metric", ["l2", "cosine"])
@pytest.mark.parametrize("nq", [384, 768, 1280, 1792])
def test_mid_batches_whole_round_splits(oracle, metric, nq):
    """Batches of 2, 3, 5 and 7 query blocks take the smallest row-split count whose work-groups
    fill whole rounds of the CUs (on 256 CUs: 128, 168, 152 and 72 splits of 300,000 rows, none a
    power of two but the first), with the bound slots shared by every list of a query. Integer data
    adds exact ties across splits."""
    base = D.gaussian(300_000, 128, seed=37)
    q = D.gaussian(nq, 128, seed=38)
    print(_check(oracle, base, q, 10, metric))
    if metric == "l2":
        ib, iq = D.int_mix(300_000, nq)
        print(_check(oracle, ib, iq, 10, metric))


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
@pytest.mark.parametrize("dim,nq,k,n", [(128, 5, 10, 1_000_003), (128, 32, 10, 300_000), (128, 31, 1, 70_001),
                                        (96, 17, 21, 65_632), (64, 8, 11, 4_200), (32, 5, 16, 100),
                                        (128, 2, 10, 33), (64, 4, 10, 4_097)])
def test_ring_scan(oracle, metric, dim, nq, k, n):
    """The ring scan (4 to 32 unfiltered queries, or fewer over rows too few to split; rows of
    whole 32-dim quarters; k up to 21): 1,000,003 rows make 255 splits of 3,936 rows, the last of
    259 (a 3-row block); 4,200 rows four splits whose waves stream 9, 8, 8 and 8 blocks; 100 rows
    one split of four blocks, the last of 4 rows; 33 rows leave two waves without a block; 4,097
    rows end on a 1-row block. k = 21 takes the 32-entry lists, k = 1, 10 and 11 the 16-entry ones."""
    base = D.gaussian(n, dim, seed=51)
    q = D.gaussian(nq, dim, seed=52)
    print(_check(oracle, base, q, k, metric))


@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_ring_scan_integer_store(oracle, metric):
    """Integer store and queries: the ring scan's GEMM-form distances are exact (every bound 0), so
    its lists certify without the margin; one real-valued query in the batch has a bound above 0
    and its selection is certified against it. Exact ties across splits and waves resolve to the
    smaller row. (One query: the few-query kernel.)"""
    base, q = D.int_mix(200_000, 32)
    print(_check(oracle, base, q, 10, metric))
    q2 = q.copy()
    q2[7, 3] += np.float32(0.25)
    print(_check(oracle, base, q2, 10, metric))
    print(_check(oracle, base, q[:1], 10, metric))


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
@pytest.mark.parametrize("fraction", [0.6, 0.95])
def test_small_batches_split_rows_filtered_and_ties(oracle, fraction, metric):
    """Integer data (many exactly equal distances across splits) with a row filter above half
    density, through host and device buffers."""
    base, q = D.int_mix(300_000, 12)
    allowed = D.allowed_ids(base.shape[0], fraction, seed=41)
    print(_check(oracle, base, q[:4], 10, metric, allowed))
    print(_check(oracle, base, q, 10, metric, allowed))
    print(_check(oracle, base, q[:1], 50, metric))
    idx = quiver.FlatIndex(base.shape[1], metric)
    idx.add(base)
    for qs in (q[:4], q):
        _device_path_matches_host_path(idx, qs, 10, allowed)


def test_integer_data_exact_ties(oracle):
    """Integer-valued mixture (config 2's distribution): distances are exact integers, ties are
    common; ties resolve to the smaller row."""
    base, q = D.int_mix(200_000, 300)
    stats = _check(oracle, base, q, 10, "l2")
    print(stats)


@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_overflowing_distances_fill_the_tail(oracle, metric):
    """Only rows 0-5 have finite distances. Rows at 3e19 overflow to +inf; rows at 3e38 also
    overflow the dot product, so the scan's expanded form sees inf - inf = NaN. The k - 6 slots
    after the finite rows hold what the reference puts there (+inf distances, smallest rows
    first), so those candidates must survive the scan's prune test while lists are not full."""
    rng = np.random.default_rng(17)
    base = rng.standard_normal((6000, 32)).astype(np.float32)
    base[6:3000] *= np.float32(3e19)
    base[3000:] = np.sign(base[3000:]) * np.float32(3e38)
    q = (2.0 * rng.standard_normal((64, 32))).astype(np.float32)
    _check(oracle, base, q, 10, metric)
    _check(oracle, base[::-1].copy(), q, 10, metric)


def test_fewer_rows_than_k_and_selective_filter(oracle):
    rng = np.random.default_rng(3)
    base = rng.standard_normal((10, 8)).astype(np.float32)
    labels = np.arange(100, 110, dtype=np.uint64)
    idx = quiver.FlatIndex(8)
    idx.add(base, labels=labels)
    got_l, got_d = idx.search(base[:1], k=50)
    assert (got_l[0, :10] >= 100).all() and (got_l[0, 10:] == -1).all()
    assert np.isinf(got_d[0, 10:]).all()
    got_l, got_d = idx.search(base[:1], k=5, filter=[103, 107])
    assert set(got_l[0, :2].tolist()) == {103, 107} and (got_l[0, 2:] == -1).all()
    _check(oracle, base, base, 5, "l2", allowed=np.array([103, 107], np.uint64), labels=labels)


def test_empty_filter_and_unknown_labels():
    rng = np.random.default_rng(4)
    base = rng.standard_normal((200, 8)).astype(np.float32)
    idx = quiver.FlatIndex(8)
    idx.add(base)
    got_l, got_d = idx.search(base[:3], k=4, filter=[])
    assert (got_l == -1).all() and np.isinf(got_d).all()
    got_l, _ = idx.search(base[:3], k=4, filter=[10**12])
    assert (got_l == -1).all()


def test_known_answers_cosine_and_inner_product():
    """tests/test_flat.cc:37-52 of the reference."""
    base = np.array([[1, 0, 0, 0], [0, 2, 0, 0], [1, 1, 0, 0]], np.float32)
    q = np.array([[3, 0.1, 0, 0]], np.float32)
    cos = quiver.FlatIndex(4, "cosine")
    cos.add(base)
    l, d = cos.search(q, 3)
    assert l[0, 0] == 0
    assert abs(d[0, 0] - (1.0 - 3.0 / np.sqrt(9.01))) < 1e-5
    ip = quiver.FlatIndex(4, "ip")
    ip.add(base)
    l, d = ip.search(q, 3)
    assert l[0, 0] == 2 and abs(d[0, 0] - (1.0 - 3.1)) < 1e-5


def test_incremental_adds_and_labels(oracle):
    rng = np.random.default_rng(9)
    base = rng.standard_normal((5000, 32)).astype(np.float32)
    idx = quiver.FlatIndex(32)
    for b in range(0, 5000, 1237):  # several appends, growing the device store
        idx.add(base[b:b + 1237], labels=np.arange(b, min(b + 1237, 5000), dtype=np.uint64) * 3)
    assert len(idx) == 5000
    q = rng.standard_normal((20, 32)).astype(np.float32)
    got_l, got_d = idx.search(q, 10)
    rows, dist = oracle.flat_search(base, q, 10, "l2")
    assert np.array_equal(got_l, rows.astype(np.int64) * 3)
    assert np.array_equal(got_d.view(np.uint32), dist.view(np.uint32))


def test_c_abi_rows_match_python_path(oracle):
    base, q = D.flat_small()
    f = Qvh().flat(128, "l2")
    f.append(base)
    assert f.size() == base.shape[0]
    rows, dist = f.search(q, 10)
    exp_r, exp_d = oracle.flat_search(base, q, 10, "l2")
    assert np.array_equal(rows, exp_r) and np.array_equal(dist.view(np.uint32), exp_d.view(np.uint32))
    f.close()


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
@pytest.mark.parametrize("count,k", [(1, 10), (37, 10), (600, 10), (600, 50), (20_000, 10)])
def test_search_over_listed_rows(oracle, metric, count, k):
    """HnswIndex::search_exact's scan over the node ids a selective filter admits
    (src/hnsw_index.cc:722-739): exact top-k over a row list given in any order, with repeats."""
    print(f"case: listed rows count={count} k={k} metric={metric}", flush=True)
    base, q = D.unit_mix(30_000, 40)
    rng = np.random.default_rng(count * 7 + k)
    rows = rng.choice(base.shape[0], count, replace=False).astype(np.uint32)
    listed = np.concatenate([rows, rows[: count // 3]])
    rng.shuffle(listed)
    f = Qvh().flat(base.shape[1], metric)
    stored = f.append(base)
    st, got_rows, got_d = f.search_rows(q, k, listed)
    assert st == 0, f.q.error()
    exp_rows, exp_d = oracle.flat_search(stored, q, k, metric, rows_bitmap(np.sort(rows), base.shape[0]))

    def labels(r):
        out = r.astype(np.int64)
        out[r == np.uint32(0xFFFFFFFF)] = -1
        return out

    print(assert_same_topk(labels(got_rows), got_d, labels(exp_rows), exp_d, _true_dist(oracle, stored, q, metric)))


def test_search_over_listed_rows_edges():
    base, q = D.unit_mix(1_000, 5)
    f = Qvh().flat(base.shape[1], "l2")
    f.append(base)
    st, rows, dist = f.search_rows(q, 4, np.zeros(0, np.uint32))  # nothing admitted
    assert st == 0 and np.all(rows == np.uint32(0xFFFFFFFF)) and np.all(np.isinf(dist))
    st, rows, dist = f.search_rows(q, 4, np.array([999, 3], np.uint32))  # fewer rows than k
    assert st == 0 and set(rows[0][:2]) == {3, 999} and np.all(rows[:, 2:] == np.uint32(0xFFFFFFFF))
    st, _, _ = f.search_rows(q, 4, np.array([5, 1_000], np.uint32))  # row 1000 is not stored
    assert st == -22 and "not stored" in f.q.error()


@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_near_ties_within_rounding_fall_back_exactly(oracle, metric):
    """Rows q0 + P(v) for 40 permutations P of one vector v all lie at the same true distance from
    query 0, so their GEMM-form and exact distances differ only by rounding: the merge cannot
    certify query 0's selection (its k-th exact distance is not below the 16th GEMM-form distance
    minus the rounding bound) and hands it to the exact kernel. The other queries are certified.
    Every result equals the oracle's (src/flat_index.cc:84-97)."""
    rng = np.random.default_rng(23)
    dim = 64
    base = (4.0 * rng.standard_normal((60_000, dim))).astype(np.float32)
    q = (4.0 * rng.standard_normal((40, dim))).astype(np.float32)
    v = (0.7 * rng.standard_normal(dim)).astype(np.float32)
    for i in range(40):
        base[1_000 + 97 * i] = q[0] + v[rng.permutation(dim)]
    idx = quiver.FlatIndex(dim, metric)
    idx.add(base)
    got_l, got_d = idx.search(q, 10)
    fallbacks = Qvh().last_fallbacks(idx._index._device_handle)
    rows, dist = oracle.flat_search(base, q, 10, metric)
    print("fallbacks", fallbacks,
          assert_same_topk(got_l, got_d, rows.astype(np.int64), dist, _true_dist(oracle, base, q, metric)))
    if metric == "l2":
        assert 1 <= fallbacks <= 3, fallbacks  # query 0 (and nothing like the others)


@pytest.mark.parametrize("dim", [64, 1024])
@pytest.mark.parametrize("allowed_frac", [None, 0.3, 0.8])
def test_many_uncertified_queries(oracle, dim, allowed_frac):
    """20 queries, each with 40 planted rows at one true distance (as above), cannot be certified:
    the first eight listed re-run over row splits with a select merge, the other twelve on one
    work-group each; also under a 30% filter (listed rows) and an 80% filter (bitmap). Results
    equal the oracle's."""
    rng = np.random.default_rng(29 + dim)
    n = 80_000 if dim == 64 else 40_000
    base = (4.0 * rng.standard_normal((n, dim))).astype(np.float32)
    q = (4.0 * rng.standard_normal((60, dim))).astype(np.float32)
    for qi in range(20):
        v = (0.7 * rng.standard_normal(dim)).astype(np.float32)
        for i in range(40):
            base[500 + 1_900 * qi + 37 * i] = q[qi] + v[rng.permutation(dim)]
    allowed = None
    if allowed_frac is not None:
        allowed = np.sort(rng.choice(n, int(n * allowed_frac), replace=False)).astype(np.uint64)
    print(f"case: uncertified dim={dim} allowed={allowed_frac}", flush=True)
    idx = quiver.FlatIndex(dim, "l2")
    idx.add(base)
    got_l, got_d = idx.search(q, 10, filter=allowed)
    fallbacks = Qvh().last_fallbacks(idx._index._device_handle)
    bm = None if allowed is None else rows_bitmap(allowed.astype(np.int64), n)
    rows, dist = oracle.flat_search(base, q, 10, "l2", bm)
    exp_l = rows.astype(np.int64)
    exp_l[rows == np.uint32(0xFFFFFFFF)] = -1
    print("fallbacks", fallbacks, assert_same_topk(got_l, got_d, exp_l, dist, _true_dist(oracle, base, q, "l2")))
    if allowed is None:
        assert fallbacks >= 9, fallbacks


def test_integer_rows_certify_exactly(oracle):
    """Small-integer rows and queries whose (||q|| + max ||x||)^2 stays below 2^24: both distance forms
    are exact, the rounding bound is 0 and no query falls back, at the size of the 1M workload's
    batches (10,000 queries over 60,000 rows)."""
    base, q = D.int_mix(60_000, 10_000)
    idx = quiver.FlatIndex(128)
    idx.add(base)
    got_l, got_d = idx.search(q, 10)
    assert Qvh().last_fallbacks(idx._index._device_handle) == 0
    rows, dist = oracle.flat_search(base, q[:500], 10)
    print(assert_same_topk(got_l[:500], got_d[:500], rows.astype(np.int64), dist, _true_dist(oracle, base, q, "l2")))


@pytest.mark.parametrize("dim", [16, 64])
@pytest.mark.parametrize("k", [63, 64])
def test_few_splits_large_k_merge_by_selection(oracle, dim, k):
    """Small batches over 3,000 rows split into fewer lists than k (the exact kernel's 8 splits for
    dim 16, the few-query kernel's 2 for dim 64): the selection merge then gathers every real key
    of every list, nsplit * k < k * k <= 4096, and needs no overflow path for k <= 64."""
    base = D.gaussian(3_000, dim, seed=35)
    q = D.gaussian(3, dim, seed=36)
    for metric in ("l2", "ip"):
        print(_check(oracle, base, q, k, metric))
