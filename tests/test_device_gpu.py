"""Device-resident query batches from Python: torch (ROCm) tensors in GPU memory go straight to the
device search (FlatIndex/IvfPqIndex.search_batch_device) and the results stay on the device. The
reference's bindings take host arrays only (python/quiver_ext.cc:24-25); its search_batch
(src/flat_index.cc:126-140, src/ivfpq_index.cc:421-437) defines the answer.

The main cases check the device-tensor results against the oracle directly: distances bit-identical,
labels identical up to equal-distance groups at the k-th boundary. The edge cases (empty index,
conversions, streams) compare with the host-buffer path, itself checked against the oracle.
"""

import numpy as np
import pytest

import quiver_amd as quiver
from oracle.oracle import IvfPqState, rows_bitmap
from parity import assert_same_topk

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible to torch")
    return torch.device("cuda", quiver._quiver._device_index())


def _same(host, dev):
    hl, hd = host
    dl, dd = dev
    assert dl.dtype == torch.int64 and dd.dtype == torch.float32
    assert np.array_equal(hl, dl.cpu().numpy())
    assert np.array_equal(hd.view(np.uint32), dd.cpu().numpy().view(np.uint32))


def _data(n, dim, nq, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, dim)).astype(np.float32),
            rng.standard_normal((nq, dim)).astype(np.float32))


def _oracle_match(dev_result, exp_labels, exp_dist):
    """Device-tensor results against the oracle's labels (uint64, all ones = empty) and distances."""
    dl, dd = dev_result
    assert dl.dtype == torch.int64 and dd.dtype == torch.float32
    return assert_same_topk(dl.cpu().numpy(), dd.cpu().numpy(), exp_labels, exp_dist)


def _flat_expected(oracle, stored, q, k, metric, labels, allowed=None):
    bm = None
    if allowed is not None:
        bm = rows_bitmap(np.flatnonzero(np.isin(labels, allowed)), labels.size)
    rows, dist = oracle.flat_search(stored, q, k, metric, bm)
    exp = np.full(rows.shape, np.uint64(2**64 - 1), dtype=np.uint64)
    ok = rows != np.uint32(0xFFFFFFFF)
    exp[ok] = labels[rows[ok].astype(np.int64)]
    return exp, dist


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
def test_flat_device_queries_match_oracle(oracle, metric):
    dev = _gpu()
    base, q = _data(20_000, 64, 300, 1)
    print(f"case: flat {metric} n=20000 dim=64 nq=300", flush=True)
    labels = np.arange(20_000, dtype=np.uint64) * 3 + 7
    idx = quiver.FlatIndex(64, metric)
    idx.add(base, labels=labels)
    stored = oracle.normalize(base) if metric == "cosine" else base
    qd = torch.from_numpy(q).to(dev)
    for k in (1, 10, 32, 100):  # MFMA scan with KL 16 and 32, the wide merge
        print(k, _oracle_match(idx.search(qd, k), *_flat_expected(oracle, stored, q, k, metric, labels)))
    allowed = np.arange(7, 60_000, 9, dtype=np.uint64)
    print(_oracle_match(idx.search(qd, 10, filter=allowed),
                        *_flat_expected(oracle, stored, q, 10, metric, labels, allowed)))
    for nq in (1, 5):  # the few-query scan (a 1-D tensor is one query)
        one = idx.search(qd[0], 5) if nq == 1 else idx.search(qd[:nq], 5)
        exp_l, exp_d = _flat_expected(oracle, stored, q[:nq], 5, metric, labels)
        if nq == 1:
            one = (one[0].reshape(1, -1), one[1].reshape(1, -1))
        print(nq, _oracle_match(one, exp_l, exp_d))


def test_flat_device_edge_cases():
    dev = _gpu()
    idx = quiver.FlatIndex(16, "l2")
    q = torch.zeros((3, 16), device=dev)
    labels, dist = idx.search(q, 4)  # empty index
    assert labels.shape == (3, 4) and bool((labels == -1).all()) and bool(torch.isinf(dist).all())
    base, hq = _data(5, 16, 3, 2)
    idx.add(base)
    _same(idx.search(hq, 8), idx.search(torch.from_numpy(hq).to(dev), 8))  # fewer rows than k
    idx.add(base + 1.0)  # the cached label table follows the index
    _same(idx.search(hq, 8), idx.search(torch.from_numpy(hq).to(dev), 8))
    with pytest.raises(ValueError):
        idx.search(torch.full((2, 16), float("nan"), device=dev), 3)
    with pytest.raises(ValueError):
        idx.search(torch.zeros((2, 15), device=dev), 3)
    with pytest.raises(ValueError):
        idx.search(torch.zeros((2, 16), device=dev), 0)
    # float64 and non-contiguous inputs are converted like host arrays are
    q64 = torch.from_numpy(hq.astype(np.float64)).to(dev)
    _same(idx.search(hq, 3), idx.search(q64, 3))
    wide = torch.from_numpy(np.repeat(hq, 2, axis=1)).to(dev)[:, ::2]
    _same(idx.search(hq, 3), idx.search(wide, 3))


def test_flat_device_search_runs_on_the_current_stream():
    dev = _gpu()
    base, q = _data(50_000, 128, 256, 3)
    idx = quiver.FlatIndex(128, "l2")
    idx.add(base)
    host = idx.search(q, 10)
    s = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(s):
        qd = torch.from_numpy(q).to(dev, non_blocking=False)
        res = idx.search(qd, 10)
    s.synchronize()
    _same(host, res)


@pytest.mark.parametrize("metric,store,refine", [("l2", False, 0), ("l2", True, 4), ("cosine", True, 8),
                                                 ("ip", False, 0)])
def test_ivfpq_device_queries_match_oracle(oracle, metric, store, refine):
    dev = _gpu()
    base, q = _data(12_000, 32, 200, 4)
    print(f"case: ivfpq {metric} store={store} refine={refine}", flush=True)
    labels = np.arange(12_000, dtype=np.uint64) * 5 + 1
    idx = quiver.IvfPqIndex(32, metric, nlist=64, m=8, store_vectors=store, train_iterations=5)
    idx.train(base)
    cent, cb, pre = oracle.ivfpq_train(base, metric, 64, 8, 5, 1234)
    assert np.array_equal(idx.centroids.view(np.uint32), cent.view(np.uint32))
    assert np.array_equal(idx.codebook.view(np.uint32), cb.view(np.uint32))
    idx.add(base, labels=labels)
    assign, codes, stored = oracle.ivfpq_encode(cent, cb, metric, base)
    st = IvfPqState(metric, cent, cb, pre).set_lists(assign, codes, labels, stored if store else None)
    qd = torch.from_numpy(q).to(dev)

    def check(nprobe, allowed=None):
        bm = None if allowed is None else rows_bitmap(np.flatnonzero(np.isin(st.labels, allowed)), st.labels.size)
        refs, dist = oracle.ivfpq_search(st, q, 10, nprobe, refine, bm)
        got = idx.search(qd, 10, nprobe=nprobe, refine_factor=refine, filter=allowed)
        print(nprobe, allowed is not None, _oracle_match(got, st.ref_to_label(refs), dist))

    for nprobe in (1, 8, 64):
        check(nprobe)
    check(16, np.arange(1, 60_000, 25, dtype=np.uint64))


def test_ivfpq_device_untrained_and_growing():
    dev = _gpu()
    idx = quiver.IvfPqIndex(16, "l2", nlist=8, m=4, train_iterations=3)
    q = torch.zeros((2, 16), device=dev)
    labels, dist = idx.search(q, 3)  # untrained: empty results, as on the host
    assert bool((labels == -1).all()) and bool(torch.isinf(dist).all())
    base, hq = _data(3_000, 16, 20, 5)
    idx.train(base)
    idx.add(base[:1_000])
    qd = torch.from_numpy(hq).to(dev)
    _same(idx.search(hq, 5, nprobe=8), idx.search(qd, 5, nprobe=8))
    idx.add(base[1_000:])  # the cached CSR tables follow the index
    _same(idx.search(hq, 5, nprobe=8), idx.search(qd, 5, nprobe=8))


@pytest.mark.parametrize("kind", ["flat", "flat_small", "ivfpq"])
def test_calls_on_two_streams_share_the_handle_safely(kind):
    """Device searches of one handle on two streams, the second growing the handle's workspace,
    then a host search: each call is ordered after the handle's earlier work on the device, so
    every result equals the host path's."""
    dev = _gpu()
    base, _ = _data(30_000, 32, 1, 6)
    rng = np.random.default_rng(7)
    qa = rng.standard_normal((300, 32)).astype(np.float32)
    qb = rng.standard_normal((6_000, 32)).astype(np.float32)
    if kind == "flat_small":  # the few-query scan: 5 queries, then 16 (two launches, more partial lists)
        qa, qb = qa[:5], qb[:16]
    print(f"case: two streams {kind}", flush=True)
    if kind in ("flat", "flat_small"):
        idx = quiver.FlatIndex(32, "l2")
        idx.add(base)
        search = lambda q: idx.search(q, 10)  # noqa: E731
    else:
        idx = quiver.IvfPqIndex(32, "l2", nlist=64, m=8, train_iterations=4)
        idx.train(base)
        idx.add(base)
        search = lambda q: idx.search(q, 10, nprobe=16)  # noqa: E731
    want_a, want_b = search(qa), search(qb)
    s1, s2 = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    with torch.cuda.stream(s1):
        got_a = search(torch.from_numpy(qa).to(dev))
    with torch.cuda.stream(s2):
        got_b = search(torch.from_numpy(qb).to(dev))
    again_a = search(qa)  # host call on the handle's own stream
    torch.cuda.synchronize(dev)
    _same(want_a, got_a)
    _same(want_b, got_b)
    assert np.array_equal(want_a[0], again_a[0])
