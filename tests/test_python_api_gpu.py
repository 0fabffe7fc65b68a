"""The reference's Python tests of the flat and IVF-PQ indexes (python/tests/test_quiver.py), run
against this package: the same calls, arguments, expected results and errors. The HNSW cases of that
file have flat-index counterparts here where the behaviour is shared (labels, filters, errors,
threads)."""

import threading

import numpy as np
import pytest

import quiver_amd as quiver

pytestmark = pytest.mark.gpu


def brute_force(base, queries, k):
    d = ((queries[:, None, :] - base[None, :, :]) ** 2).sum(-1)
    return np.argsort(d, axis=1)[:, :k]


@pytest.fixture(scope="module")
def data():
    rng = np.random.default_rng(0)
    return rng.standard_normal((3000, 24), dtype=np.float32), rng.standard_normal((50, 24), dtype=np.float32)


def recall(truth, got):
    return np.mean([len(set(t) & set(g)) / len(t) for t, g in zip(truth, got)])


def test_float64_lists_and_single_vectors_are_accepted():
    index = quiver.FlatIndex(3)
    index.add([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]])
    labels, _ = index.search([1.0, 2.0, 3.1], k=1)
    assert labels.tolist() == [[0]]


def test_missing_results_are_minus_one():
    index = quiver.FlatIndex(4)
    index.add(np.eye(4, dtype=np.float32))
    labels, dist = index.search(np.ones(4), k=6)
    assert labels[0, 4:].tolist() == [-1, -1] and np.isinf(dist[0, 4:]).all()


def test_labels_and_filter(data):
    base, queries = data
    index = quiver.FlatIndex(24, metric="cosine")
    index.add(base, labels=np.arange(len(base)) * 10)
    allowed = np.arange(0, len(base) * 10, 30)
    labels, dist = index.search(queries, k=5, filter=allowed)
    assert np.isin(labels, allowed).all()
    assert dist.dtype == np.float32 and np.all(np.diff(dist, axis=1) >= 0)


def test_errors():
    for make in (lambda: quiver.FlatIndex(8), lambda: quiver.IvfPqIndex(8, nlist=2, m=2)):
        index = make()
        with pytest.raises(ValueError, match="dimension"):
            index.add(np.zeros((2, 7)))
    index = quiver.FlatIndex(8)
    index.add(np.zeros((1, 8)), labels=[5])
    index.add(np.ones((1, 8)), labels=[5])  # the flat index keeps duplicate labels (src/flat_index.cc:48-66)
    assert index.search(np.zeros(8), k=2)[0].tolist() == [[5, 5]]
    with pytest.raises(ValueError):
        index.add(np.zeros((1, 8)), labels=[-1])
    with pytest.raises(ValueError):
        quiver.FlatIndex(8, metric="hamming")
    with pytest.raises(ValueError):
        quiver.IvfPqIndex(8, metric="hamming")
    with pytest.raises(ValueError):
        quiver.FlatIndex.load("/does/not/exist.qvr")
    with pytest.raises(ValueError):
        quiver.IvfPqIndex.load("/does/not/exist.qvr")
    with pytest.raises(ValueError):
        index.add(np.full((1, 8), np.nan))  # non-finite vectors (tests/test_regressions.cc:87-99)


def test_concurrent_python_threads(data):
    base, queries = data
    index = quiver.FlatIndex(24)
    index.add(base[:1000])
    errors = []

    def reader():
        try:
            for _ in range(50):
                labels, _ = index.search(queries, k=5, num_threads=1)
                assert (labels >= 0).all()
        except Exception as e:  # pragma: no cover
            errors.append(e)

    threads = [threading.Thread(target=reader) for _ in range(4)]
    for t in threads:
        t.start()
    for i in range(1000, 3000, 100):
        index.add(base[i:i + 100], labels=np.arange(i, i + 100))
    for t in threads:
        t.join()
    assert not errors and len(index) == 3000


def test_flat_index_is_exact(data, tmp_path):
    base, queries = data
    flat = quiver.FlatIndex(24)
    flat.add(base)
    labels, _ = flat.search(queries, k=10)
    np.testing.assert_array_equal(labels, brute_force(base, queries, 10))
    flat.save(str(tmp_path / "flat.qvr"))
    assert len(quiver.FlatIndex.load(str(tmp_path / "flat.qvr"))) == len(base)


def test_ivfpq(tmp_path):
    rng = np.random.default_rng(1)
    centers = rng.standard_normal((40, 32)).astype(np.float32) * 3
    base = (centers[rng.integers(0, 40, 6000)] + rng.standard_normal((6000, 32))).astype(np.float32)
    queries = (centers[rng.integers(0, 40, 50)] + rng.standard_normal((50, 32))).astype(np.float32)
    index = quiver.IvfPqIndex(32, nlist=64, m=16, store_vectors=True)
    with pytest.raises(ValueError):
        index.add(base)  # must train first
    index.train(base)
    index.add(base)
    assert index.is_trained and len(index) == 6000
    labels, _ = index.search(queries, k=10, nprobe=16, refine_factor=4)
    assert recall(brute_force(base, queries, 10), labels) >= 0.9
    index.save(str(tmp_path / "ivf.qvr"))
    loaded = quiver.IvfPqIndex.load(str(tmp_path / "ivf.qvr"))
    np.testing.assert_array_equal(loaded.search(queries, k=5)[0], index.search(queries, k=5)[0])


def test_ivfpq_inner_product_recall():
    """Max-inner-product probing with cells assigned by inner product (tests/test_regressions.cc:133-158)."""
    rng = np.random.default_rng(4)
    centers = rng.standard_normal((30, 16)).astype(np.float32) * 3
    base = (centers[rng.integers(0, 30, 6000)] + rng.standard_normal((6000, 16))).astype(np.float32)
    queries = (centers[rng.integers(0, 30, 100)] + rng.standard_normal((100, 16))).astype(np.float32)
    truth = np.argsort(-(queries @ base.T), axis=1)[:, :10]
    index = quiver.IvfPqIndex(16, metric="ip", nlist=32, m=8, store_vectors=True)
    index.train(base)
    index.add(base)
    labels, _ = index.search(queries, k=10, nprobe=16, refine_factor=8)
    assert recall(truth, labels) >= 0.9


def test_label_range_and_sentinel():
    x = np.random.default_rng(2).standard_normal((5, 4)).astype(np.float32)
    index = quiver.FlatIndex(4)
    with pytest.raises(ValueError, match="2\\*\\*63"):
        index.add(x, labels=np.array([0, 1, 2, 3, 2**64 - 1], dtype=np.uint64))
    with pytest.raises(ValueError, match="2\\*\\*63"):
        index.add(x, labels=[0, 1, 2, 3, 2**63])
    index.add(x, labels=[0, 1, 2, 3, 2**63 - 1])
    assert index.search(x[4], k=1)[0][0, 0] == 2**63 - 1


@pytest.mark.parametrize("flt", [[], set(), {1, 2}, (i for i in [1, 2]), range(3), np.array([1, 2])])
def test_filter_accepts_any_iterable(flt):
    x = np.random.default_rng(3).standard_normal((20, 4)).astype(np.float32)
    f = quiver.FlatIndex(4)
    f.add(x)
    labels, _ = f.search(x[:1], k=2, filter=flt)
    assert set(labels[0][labels[0] >= 0]) <= {0, 1, 2}


def test_huge_k_is_rejected_not_a_crash():
    x = np.random.default_rng(4).standard_normal((300, 4)).astype(np.float32)
    for index in (quiver.FlatIndex(4), quiver.IvfPqIndex(4, nlist=2, m=2)):
        if isinstance(index, quiver.IvfPqIndex):
            index.train(x)  # training takes at least max(nlist, 256) vectors
        index.add(x)
        with pytest.raises(ValueError, match="too large"):
            index.search(x[:3], k=2**64 // 3 + 1)
        with pytest.raises((ValueError, OverflowError)):
            index.search(x[:4], k=2**62)


def test_ivfpq_concurrent_add_and_search_do_not_deadlock():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((20000, 16)).astype(np.float32)
    index = quiver.IvfPqIndex(16, nlist=32, m=4, train_iterations=3)
    index.train(x)
    index.add(x)
    q = rng.standard_normal((20000, 16)).astype(np.float32)
    done = []

    def run(fn):
        fn()
        done.append(1)

    threads = [threading.Thread(target=run, args=(f,)) for f in (
        lambda: index.search(q, k=10, nprobe=32),
        lambda: index.add(x[:5000]),
        lambda: index.add(x[:100], num_threads=1))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert len(done) == 3 and len(index) == 25100
