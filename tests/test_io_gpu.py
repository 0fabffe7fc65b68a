"""`.qvr` interchange with the compiled reference, on the GPU.

An index the reference built and saved loads here straight into the device layouts and returns
the reference's own search results (bit-identical distances, labels up to exact-distance ties);
saving it again reproduces the reference's file byte for byte. An index built here and saved
loads in the reference, which then answers like the device does.
"""

import numpy as np
import pytest

import quiver_amd as quiver
from parity import assert_same_topk

pytestmark = pytest.mark.gpu


def clustered(n, dim, seed):
    rng = np.random.default_rng(seed)
    centers = (2.0 * np.random.default_rng(500).standard_normal((40, dim))).astype(np.float32)
    return (centers[rng.integers(0, 40, n)] + rng.standard_normal((n, dim))).astype(np.float32)


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
def test_flat_reference_file_round_trip(tmp_path, reference, metric):
    print(f"case: flat {metric}", flush=True)
    base, q = clustered(3_000, 40, 1), clustered(60, 40, 2)
    labels = (np.arange(3_000, dtype=np.uint64) * 5 + 11)
    ref = reference.flat(40, metric)
    ref.add(base, labels)
    theirs = tmp_path / "theirs.qvr"
    ref.save(theirs)

    ours = quiver.FlatIndex.load(theirs)
    assert len(ours) == 3_000 and ours.metric == metric
    exp_l, exp_d = ref.search(q, 10)
    got_l, got_d = ours.search(q, 10)
    print(assert_same_topk(got_l, got_d, exp_l, exp_d))
    allowed = labels[::7]
    exp_l, exp_d = ref.search(q, 10, allowed=allowed)
    got_l, got_d = ours.search(q, 10, filter=allowed)
    print(assert_same_topk(got_l, got_d, exp_l, exp_d))

    again = tmp_path / "again.qvr"
    ours.save(again)
    assert again.read_bytes() == theirs.read_bytes()


def test_flat_saved_here_loads_in_reference(tmp_path, reference):
    base, q = clustered(2_000, 24, 3), clustered(30, 24, 4)
    ours = quiver.FlatIndex(24, "cosine")
    ours.add(base)
    path = tmp_path / "ours.qvr"
    ours.save(path)
    ref = reference.flat_load(path)
    exp_l, exp_d = ref.search(q, 7)
    got_l, got_d = ours.search(q, 7)
    print(assert_same_topk(got_l, got_d, exp_l, exp_d))


@pytest.mark.parametrize("metric,store,refine", [("l2", False, 0), ("l2", True, 4), ("cosine", True, 8),
                                                 ("ip", False, 0)])
def test_ivfpq_reference_file_round_trip(tmp_path, reference, metric, store, refine):
    print(f"case: ivfpq {metric} store={store} refine={refine}", flush=True)
    base, q = clustered(6_000, 32, 5), clustered(80, 32, 6)
    ref = reference.ivfpq(32, metric, nlist=32, m=8, train_iterations=6, store_vectors=store)
    ref.train(base)
    labels = np.arange(6_000, dtype=np.uint64)[::-1].copy() + 100
    ref.add(base, labels)
    theirs = tmp_path / "theirs.qvr"
    ref.save(theirs)

    ours = quiver.IvfPqIndex.load(theirs)
    assert ours.is_trained and len(ours) == 6_000
    # IvfPqIndex::list_sizes / memory_bytes (src/ivfpq_index.cc:446-463) equal the reference's
    assert np.array_equal(np.asarray(ours.list_sizes(), dtype=np.uint64), ref.list_sizes(32))
    assert ours.memory_bytes == ref.memory_bytes
    for nprobe in (1, 8, 32):
        exp_l, exp_d = ref.search(q, 10, nprobe=nprobe, refine_factor=refine)
        got_l, got_d = ours.search(q, 10, nprobe=nprobe, refine_factor=refine)
        print(nprobe, assert_same_topk(got_l, got_d, exp_l, exp_d))
    allowed = labels[::3]
    exp_l, exp_d = ref.search(q, 10, nprobe=8, refine_factor=refine, allowed=allowed)
    got_l, got_d = ours.search(q, 10, nprobe=8, refine_factor=refine, filter=allowed)
    print("filter", assert_same_topk(got_l, got_d, exp_l, exp_d))

    again = tmp_path / "again.qvr"
    ours.save(again)
    assert again.read_bytes() == theirs.read_bytes()


def test_ivfpq_saved_here_loads_in_reference(tmp_path, reference):
    base, q = clustered(5_000, 16, 7), clustered(40, 16, 8)
    ours = quiver.IvfPqIndex(16, "l2", nlist=16, m=4, store_vectors=True, train_iterations=5)
    ours.train(base)
    ours.add(base)
    path = tmp_path / "ours.qvr"
    ours.save(path)
    ref = reference.ivfpq_load(path)
    assert len(ref) == 5_000
    assert np.array_equal(np.asarray(ours.list_sizes(), dtype=np.uint64), ref.list_sizes(16))
    assert ours.memory_bytes == ref.memory_bytes
    for nprobe, refine in ((4, 0), (16, 3)):
        exp_l, exp_d = ref.search(q, 10, nprobe=nprobe, refine_factor=refine)
        got_l, got_d = ours.search(q, 10, nprobe=nprobe, refine_factor=refine)
        print(nprobe, assert_same_topk(got_l, got_d, exp_l, exp_d))


def test_loaded_index_keeps_growing(tmp_path, reference):
    """add() after load appends to the loaded lists exactly as the reference does."""
    base = clustered(4_000, 16, 9)
    ref = reference.ivfpq(16, "l2", nlist=16, m=4, train_iterations=4)
    ref.train(base)
    ref.add(base[:2_500])
    path = tmp_path / "part.qvr"
    ref.save(path)
    ours = quiver.IvfPqIndex.load(path)
    ours.add(base[2_500:])
    ref.add(base[2_500:])
    full_ref, full_ours = tmp_path / "full_ref.qvr", tmp_path / "full_ours.qvr"
    ref.save(full_ref)
    ours.save(full_ours)
    assert full_ours.read_bytes() == full_ref.read_bytes()
