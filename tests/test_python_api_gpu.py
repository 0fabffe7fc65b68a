"""The Python surface of FlatIndex and IvfPqIndex (quiver_amd/__init__.py) against the behaviours the
reference's Python tests pin (python/tests/test_quiver.py, cited per test), for the two classes this
package keeps (the HNSW index is out of scope). Answers are checked against exact float64 search;
bit-level parity with the oracle lives in test_flat_gpu.py and test_ivfpq_gpu.py.
"""

import threading

import numpy as np
import pytest

import quiver_amd as quiver

pytestmark = pytest.mark.gpu


def exact_knn(base, queries, k, metric="l2"):
    b, q = base.astype(np.float64), np.atleast_2d(queries).astype(np.float64)
    if metric == "l2":
        score = (q * q).sum(1)[:, None] - 2 * q @ b.T + (b * b).sum(1)[None, :]
    else:
        score = -(q @ b.T)
    return np.argsort(score, axis=1, kind="stable")[:, :k]


def mean_recall(truth, labels):
    return float(np.mean([np.intersect1d(t, g).size / len(t) for t, g in zip(truth, labels)]))


def blobs(n, dim, clusters, seed, spread=3.0):
    rng = np.random.default_rng(seed)
    centers = spread * np.random.default_rng(1000 + clusters).standard_normal((clusters, dim))
    return (centers[rng.integers(0, clusters, n)] + rng.standard_normal((n, dim))).astype(np.float32)


def trained_ivf(dim=16, n=3000, **kw):
    x = blobs(n, dim, 12, 9)
    index = quiver.IvfPqIndex(dim, nlist=kw.pop("nlist", 16), m=kw.pop("m", 4), train_iterations=4, **kw)
    index.train(x)
    index.add(x)
    return index, x


# ---- inputs: lists, float64, one vector (test_quiver.py:35-40) ----------------------------------

@pytest.mark.parametrize("kind", ["flat", "ivfpq"])
def test_python_lists_float64_and_one_vector(kind):
    if kind == "flat":
        index = quiver.FlatIndex(3)
        index.add([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]])
        labels, dist = index.search([1.0, 2.0, 3.1], k=1)
    else:
        index, x = trained_ivf(dim=4, n=600, nlist=4, m=2)
        labels, dist = index.search(x[7].astype(np.float64).tolist(), k=1, nprobe=4)
    assert labels.shape == (1, 1) and labels.dtype == np.int64 and dist.dtype == np.float32
    if kind == "flat":
        assert labels.tolist() == [[0]]


# ---- empty result slots (test_quiver.py:42-46) ----------------------------------------------------

def test_missing_results_are_minus_one_and_inf():
    flat = quiver.FlatIndex(4)
    flat.add(np.eye(4, dtype=np.float32))
    labels, dist = flat.search(np.ones(4), k=6)
    assert labels[0, 4:].tolist() == [-1, -1] and np.isinf(dist[0, 4:]).all()
    assert sorted(labels[0, :4].tolist()) == [0, 1, 2, 3]
    ivf, x = trained_ivf(dim=4, n=300, nlist=2, m=2)
    labels, dist = ivf.search(x[:2], k=400, nprobe=2)  # more than the 300 stored
    assert (labels[:, 300:] == -1).all() and np.isinf(dist[:, 300:]).all()


# ---- labels and filters (test_quiver.py:49-59, 146-158, 161-167) --------------------------------

@pytest.mark.parametrize("labels,error,match", [
    (np.array([0, 1, 2, 3, 2**64 - 1], dtype=np.uint64), ValueError, r"2\*\*63"),
    ([0, 1, 2, 3, 2**63], ValueError, r"2\*\*63"),
    ([0, 1, 2, 3, -1], ValueError, "non-negative"),
    (np.array([0.0, 1, 2, 3, 4]), TypeError, "integers"),
    ([0, 1, 2, 3, True], TypeError, "integers"),
    ([0, 1, 2], ValueError, "3 labels for 5 vectors"),
])
def test_rejected_labels(labels, error, match):
    x = np.random.default_rng(2).standard_normal((5, 4)).astype(np.float32)
    with pytest.raises(error, match=match):
        quiver.FlatIndex(4).add(x, labels=labels)


def test_largest_label_round_trips():
    x = np.random.default_rng(2).standard_normal((5, 4)).astype(np.float32)
    index = quiver.FlatIndex(4)
    index.add(x, labels=[0, 1, 2, 3, 2**63 - 1])
    assert index.search(x[4], k=1)[0][0, 0] == 2**63 - 1


def test_filter_admits_only_its_labels_and_cosine_rows_are_unit():
    x = blobs(3000, 24, 10, 1)
    index = quiver.FlatIndex(24, metric="cosine")
    index.add(x, labels=np.arange(3000) * 10)
    allowed = np.arange(0, 30000, 30)
    labels, _ = index.search(x[:50], k=5, filter=allowed)
    assert np.isin(labels, allowed).all()
    np.testing.assert_allclose(np.linalg.norm(index.get_vector(3)), 1.0, rtol=1e-5)


@pytest.mark.parametrize("flt", [[], set(), {1, 2}, (i for i in [1, 2]), range(3), np.array([1, 2]), 2])
def test_filter_takes_any_iterable_of_labels(flt):
    x = np.random.default_rng(3).standard_normal((20, 4)).astype(np.float32)
    index = quiver.FlatIndex(4)
    index.add(x)
    labels, _ = index.search(x[:1], k=2, filter=flt)
    assert set(labels[0][labels[0] >= 0].tolist()) <= {0, 1, 2}


# ---- argument errors (test_quiver.py:62-75, 170-178) ---------------------------------------------

def test_argument_errors_raise_value_error():
    flat = quiver.FlatIndex(8)
    with pytest.raises(ValueError, match="dimension"):
        flat.add(np.zeros((2, 7)))
    with pytest.raises(ValueError, match="unknown metric"):
        quiver.FlatIndex(8, metric="hamming")
    with pytest.raises(ValueError):
        quiver.FlatIndex.load("/does/not/exist.qvr")
    with pytest.raises(ValueError):
        quiver.IvfPqIndex.load("/does/not/exist.qvr")
    with pytest.raises(ValueError, match="trained"):
        quiver.IvfPqIndex(8, nlist=4, m=2).add(np.zeros((3, 8)))
    with pytest.raises(ValueError, match="divisible"):
        quiver.IvfPqIndex(10, m=3)
    with pytest.raises(ValueError, match="NaN"):
        flat.add(np.full((1, 8), np.nan))


@pytest.mark.parametrize("kind", ["flat", "ivfpq"])
def test_huge_k_is_an_error_not_a_crash(kind):
    x = np.random.default_rng(4).standard_normal((300, 4)).astype(np.float32)
    if kind == "flat":
        index = quiver.FlatIndex(4)
    else:
        index = quiver.IvfPqIndex(4, nlist=2, m=2)
        index.train(x)
    index.add(x)
    with pytest.raises(ValueError, match="too large"):
        index.search(x[:3], k=2**64 // 3 + 1)
    with pytest.raises((ValueError, OverflowError)):
        index.search(x[:4], k=2**62)


# ---- exactness, recall and files (test_quiver.py:116-143) ---------------------------------------

def test_flat_search_is_exact_and_survives_a_file_round_trip(tmp_path):
    x = blobs(3000, 24, 10, 5)
    q = blobs(50, 24, 10, 6)
    index = quiver.FlatIndex(24)
    index.add(x)
    labels, dist = index.search(q, k=10)
    np.testing.assert_array_equal(labels, exact_knn(x, q, 10))
    assert np.all(np.diff(dist, axis=1) >= 0)
    index.save(tmp_path / "flat.qvr")
    loaded = quiver.FlatIndex.load(tmp_path / "flat.qvr")
    assert len(loaded) == 3000
    np.testing.assert_array_equal(loaded.search(q, k=10)[0], labels)


@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_ivfpq_recall_and_file_round_trip(tmp_path, metric):
    """Recall floors of test_quiver.py:126-143 (L2) and tests/test_regressions.cc:133-158 (inner
    product with cells assigned by inner product)."""
    dim = 32 if metric == "l2" else 16
    x = blobs(6000, dim, 40, 11)
    q = blobs(60, dim, 40, 12)
    index = quiver.IvfPqIndex(dim, metric=metric, nlist=64 if metric == "l2" else 32, m=16 if metric == "l2" else 8,
                              store_vectors=True)
    index.train(x)
    index.add(x)
    assert index.is_trained and len(index) == 6000
    labels, _ = index.search(q, k=10, nprobe=16, refine_factor=4 if metric == "l2" else 8)
    assert mean_recall(exact_knn(x, q, 10, metric), labels) >= 0.9
    index.save(tmp_path / "ivf.qvr")
    loaded = quiver.IvfPqIndex.load(tmp_path / "ivf.qvr")
    np.testing.assert_array_equal(loaded.search(q, k=5)[0], index.search(q, k=5)[0])


# ---- threads (test_quiver.py:92-113, 180-199) ---------------------------------------------------

def test_flat_searches_while_another_thread_adds():
    x = blobs(3000, 24, 10, 7)
    q = blobs(40, 24, 10, 8)
    index = quiver.FlatIndex(24)
    index.add(x[:1000])
    failures = []

    def searcher():
        try:
            for _ in range(30):
                labels, _ = index.search(q, k=5, num_threads=1)
                if not (labels >= 0).all():
                    failures.append("empty slot")
        except Exception as e:  # pragma: no cover
            failures.append(repr(e))

    readers = [threading.Thread(target=searcher) for _ in range(4)]
    for t in readers:
        t.start()
    for start in range(1000, 3000, 250):
        index.add(x[start:start + 250], labels=np.arange(start, start + 250))
    for t in readers:
        t.join()
    assert not failures and len(index) == 3000


def test_ivfpq_add_and_search_in_parallel_threads_finish():
    index, x = trained_ivf(dim=16, n=20000, nlist=32, m=4)
    q = np.random.default_rng(13).standard_normal((20000, 16)).astype(np.float32)
    finished = []
    jobs = [lambda: index.search(q, k=10, nprobe=32), lambda: index.add(x[:5000]),
            lambda: index.add(x[:100], num_threads=1)]
    threads = [threading.Thread(target=lambda f=f: (f(), finished.append(1))) for f in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert len(finished) == 3 and len(index) == 25100
