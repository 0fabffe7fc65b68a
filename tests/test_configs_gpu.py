"""The benchmark workloads at their full sizes, on the GPU, against the oracle and the compiled
reference's golden vectors.

Each test runs the whole query batch on the device (the batch shape fixes the scan's row splits,
shared bounds, slicing and query order) and checks every query of it against the oracle on the same
inputs (src/flat_index.cc:69-140, src/ivfpq_index.cc:144-381), the last, partially filled query
block of the scans included:

* 1,000,000 x 128 integer mixture, flat L2, k = 10 (10,000 queries; also batches of 1, 8, 16, 32
  and 128 queries: the few-query kernels and the row-split scan);
* 1,183,514 x 100 unit-norm mixture, flat cosine, k = 10: unfiltered, 10% and 0.5% allowed ids;
* IVF-PQ L2 on the 1M mixture, nlist 2048, m 32, trained on the 100,000-row sample: trained
  state, cells, codes and list order against the SHA-256 of the compiled reference's own run
  (tests/golden/ivfpq_1m.json), its first 200 searches at nprobe 32 bit for bit, and the nprobe
  sweep {1, 4, 8, 16, 32, 64} against the oracle on the same state;
* IVF-PQ cosine on the 1.18M set, nlist 2048, m 25, stored vectors, refine 8, nprobe 16 and 64:
  training against the oracle's, the cells and codes of all 1,183,514 rows against the oracle's
  encode, stored vectors, searches.
"""

import json
import os

import numpy as np
import pytest

import quiver_amd as quiver
from golden import inputs as G
from oracle.oracle import IvfPqState, rows_bitmap
from parity import assert_same_topk
from quiver_amd import datasets as D
from qvh_ctypes import Qvh

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_CACHE = {}


def _frozen(*arrays):
    for a in arrays:
        a.flags.writeable = False
    return arrays


def int_mix_full():
    if "int" not in _CACHE:
        _CACHE["int"] = _frozen(*D.int_mix())
    return _CACHE["int"]


def unit_mix_full(oracle):
    """(base, queries, base as the reference stores it for cosine: simd::normalize of each row)."""
    if "unit" not in _CACHE:
        base, q = D.unit_mix()
        _CACHE["unit"] = _frozen(base, q, oracle.normalize(base))
    return _CACHE["unit"]


def _true_dist(oracle, stored, queries, metric):
    def f(qi, labels):
        return oracle.flat_pair_dist(stored, queries, np.full(labels.size, qi), labels, metric)
    return f


def _rows_to_labels(rows):
    out = rows.astype(np.int64)
    out[rows == np.uint32(0xFFFFFFFF)] = -1
    return out


def test_flat_l2_int_mixture_1m(oracle):
    base, q = int_mix_full()
    print(f"case: flat l2 {base.shape} nq={q.shape[0]} k=10", flush=True)
    idx = quiver.FlatIndex(128)
    idx.add(base)
    got_l, got_d = idx.search(q, 10)
    # integer rows and queries: both distance forms are exact, so every selection is certified
    assert Qvh().last_fallbacks(idx._index._device_handle) == 0
    rows, dist = oracle.flat_search(base, q, 10)
    print(assert_same_topk(got_l, got_d, _rows_to_labels(rows), dist, _true_dist(oracle, base, q, "l2")))
    # the few-query kernels (up to 16) and the row-split MFMA scan (up to 128) over the same rows
    for nq in (1, 8, 16, 32, 128):
        print(f"case: flat l2 1M nq={nq}", flush=True)
        gl, gd = idx.search(q[:nq], 10)
        print(assert_same_topk(gl, gd, _rows_to_labels(rows[:nq]), dist[:nq], _true_dist(oracle, base, q, "l2")))


@pytest.mark.parametrize("fraction", [None, 0.1, 0.005])
def test_flat_cosine_unit_mixture_filtered(oracle, fraction):
    base, q, stored = unit_mix_full(oracle)
    n = base.shape[0]
    print(f"case: flat cosine {base.shape} nq={q.shape[0]} k=10 allowed={fraction}", flush=True)
    if "flat_cos" not in _CACHE:
        idx = quiver.FlatIndex(100, "cosine")
        idx.add(base)
        _CACHE["flat_cos"] = idx
    idx = _CACHE["flat_cos"]
    allowed = None if fraction is None else D.allowed_ids(n, fraction)
    got_l, got_d = idx.search(q, 10, filter=allowed)
    print("fallbacks", Qvh().last_fallbacks(idx._index._device_handle))
    bm = None if allowed is None else rows_bitmap(allowed.astype(np.int64), n)
    rows, dist = oracle.flat_search(stored, q, 10, "cosine", bm)
    print(assert_same_topk(got_l, got_d, _rows_to_labels(rows), dist, _true_dist(oracle, stored, q, "cosine")))


def _ivf_state(metric, cent, cb, pre, off, labels, codes, vectors=None):
    st = IvfPqState(metric, cent, cb, pre)
    st.offsets = np.ascontiguousarray(off, dtype=np.uint64)
    st.labels = np.ascontiguousarray(labels, dtype=np.uint64)
    st.codes = np.ascontiguousarray(codes, dtype=np.uint8)
    st.vectors = vectors
    return st


def test_ivfpq_l2_int_mixture_1m_matches_reference(oracle):
    with open(os.path.join(GOLDEN, "ivfpq_1m.json")) as f:
        g = json.load(f)
    base, q = int_mix_full()
    assert D.sha256(base) == g["base_sha"] and D.sha256(q) == g["query_sha"]
    sample = G.int_mix_sample(base.shape[0])
    assert G.sha(sample.astype(np.int64)) == g["sample_sha"]
    print("case: IVF-PQ l2 1M nlist 2048 m 32: train on the 100k sample, add all", flush=True)
    idx = quiver.IvfPqIndex(128, "l2", nlist=2048, m=32, train_iterations=20)
    idx.train(base[sample])
    cent, cb = idx.centroids, idx.codebook
    assert G.sha(cent) == g["centroids_sha"], "coarse centroids differ from the reference's"
    assert G.sha(cb) == g["codebook_sha"], "PQ codebook differs from the reference's"
    idx.add(base)
    off, labels, codes = idx.lists()
    assert G.sha(off) == g["offsets_sha"], "list offsets (cells) differ from the reference's"
    assert G.sha(labels) == g["labels_sha"], "list order differs from the reference's"
    assert G.sha(codes) == g["codes_sha"], "PQ codes differ from the reference's"
    got_l, got_d = idx.search(q, 10, nprobe=g["search_nprobe"])
    assert Qvh().ivf_last_fallbacks(idx._index._device_handle) == 0
    exp_l = np.array(g["search_labels"], dtype=np.int64).view(np.uint64)
    exp_d = np.array(g["search_dist_bits"], dtype=np.uint32).view(np.float32)
    print("reference's first 200:", assert_same_topk(got_l[:200], got_d[:200], exp_l, exp_d))
    st = _ivf_state("l2", cent, cb, oracle.ivfpq_precompute(cent, cb), off, labels, codes)
    for nprobe in (1, 4, 8, 16, 32, 64):
        print(f"case: IVF-PQ l2 1M nprobe={nprobe}", flush=True)
        got_l, got_d = idx.search(q, 10, nprobe=nprobe)
        refs, dist = oracle.ivfpq_search(st, q, 10, nprobe)
        print(nprobe, "fallbacks", Qvh().ivf_last_fallbacks(idx._index._device_handle),
              assert_same_topk(got_l, got_d, st.ref_to_label(refs), dist))


def test_ivfpq_cosine_refine_unit_mixture(oracle):
    base, q, stored = unit_mix_full(oracle)
    n = base.shape[0]
    sample = np.random.default_rng(31).permutation(n)[:100_000]
    print("case: IVF-PQ cosine 1.18M nlist 2048 m 25 store_vectors: train on a 100k sample", flush=True)
    idx = quiver.IvfPqIndex(100, "cosine", nlist=2048, m=25, store_vectors=True, train_iterations=20)
    idx.train(base[sample])
    cent, cb, _ = oracle.ivfpq_train(base[sample], "cosine", 2048, 25, 20, 1234)
    assert np.array_equal(idx.centroids.view(np.uint32), cent.view(np.uint32)), "centroids differ"
    assert np.array_equal(idx.codebook.view(np.uint32), cb.view(np.uint32)), "codebook differs"
    print("case: add all 1,183,514", flush=True)
    idx.add(base)
    off, labels, codes = idx.lists()
    assert np.array_equal(np.sort(labels), np.arange(n, dtype=np.uint64))
    pos = np.empty(n, dtype=np.int64)
    pos[labels.astype(np.int64)] = np.arange(n)
    print("case: cells and codes of all 1,183,514 rows against the oracle's encode", flush=True)
    assign, exp_codes, _ = oracle.ivfpq_encode(cent, cb, "cosine", base)
    cell = np.searchsorted(off.astype(np.int64), pos, side="right") - 1
    assert np.array_equal(cell, assign.astype(np.int64)), "cells differ"
    assert np.array_equal(codes[pos], exp_codes), "PQ codes differ"
    # list order: within each list, rows in input order (src/ivfpq_index.cc:263-269)
    assert np.array_equal(labels.astype(np.int64), np.argsort(assign, kind="stable")), "list order differs"
    vectors = idx.list_vectors()
    assert np.array_equal(vectors.view(np.uint32), stored[labels.astype(np.int64)].view(np.uint32))
    st = _ivf_state("cosine", cent, cb, None, off, labels, codes, vectors)
    for nprobe in (16, 64):
        print(f"case: IVF-PQ cosine refine 8 nprobe={nprobe}", flush=True)
        got_l, got_d = idx.search(q, 10, nprobe=nprobe, refine_factor=8)
        refs, dist = oracle.ivfpq_search(st, q, 10, nprobe, 8)
        print(nprobe, assert_same_topk(got_l, got_d, st.ref_to_label(refs), dist))
