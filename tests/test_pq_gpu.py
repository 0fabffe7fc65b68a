"""ProductQuantizer and nearest_centroid on the GPU (qvh_pq_*, qvh_nearest_centroid) against the
compiled reference's golden vectors and the oracle (src/product_quantizer.cc:14-27,155-217): codes,
tables and ADC sums bit-identical, decode exact."""

import numpy as np
import pytest

from golden import inputs as G
from qvh_ctypes import Qvh

pytestmark = pytest.mark.gpu


def _golden(name):
    import os
    return np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name), allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_nearest_centroid_matches_reference_and_oracle(oracle):
    g = _golden("nearest.npz")
    q = Qvh()
    for i, (x, cent) in enumerate(G.nearest_centroid_cases()):
        print(f"case: nearest_centroid {i}: n={x.shape[0]} k={cent.shape[0]} dim={x.shape[1]}", flush=True)
        got = q.nearest_centroid(x, cent)
        assert np.array_equal(got, g[f"case{i}_out"]), i
    rng = np.random.default_rng(5)
    x = rng.standard_normal((500, 100)).astype(np.float32)
    cent = rng.standard_normal((1000, 100)).astype(np.float32)  # more centroids than the block's threads
    assert np.array_equal(q.nearest_centroid(x, cent), oracle.nearest_centroid(x, cent))


def test_pq_matches_reference_golden_vectors():
    """The reference's trained codebook (kmeans.npz): encode, L2 and IP tables, adc_batch."""
    g = _golden("kmeans.npz")
    px, pq_q = G.pq_points()
    cb = g["pq_codebook"]
    m, _, dsub = cb.shape
    pq = Qvh().pq(m * dsub, m, cb)
    assert np.array_equal(pq.encode(px[:500]), g["pq_codes"])
    assert np.array_equal(bits(pq.tables(pq_q)), bits(g["pq_l2_tables"]))
    assert np.array_equal(bits(pq.tables(pq_q, inner_product=True)), bits(g["pq_ip_tables"]))
    assert np.array_equal(bits(pq.adc(g["pq_l2_tables"][0], g["pq_codes"])), bits(g["pq_adc_batch"]))
    assert np.array_equal(bits(pq.adc(g["pq_l2_tables"][0], g["pq_codes"])), bits(g["pq_adc_single"]))
    rec = pq.decode(g["pq_codes"])
    exp = np.concatenate([cb[j, g["pq_codes"][:, j]] for j in range(m)], axis=1)
    assert np.array_equal(bits(rec), bits(exp))


@pytest.mark.parametrize("dim,m", [(128, 32), (100, 25), (96, 8), (30, 30)])
def test_pq_matches_oracle(oracle, dim, m):
    rng = np.random.default_rng(dim + m)
    x = rng.standard_normal((3_000, dim)).astype(np.float32)
    cb = oracle.pq_train(x, m, iterations=6, seed=7)
    pq = Qvh().pq(dim, m, cb)
    codes = pq.encode(x)
    assert np.array_equal(codes, oracle.pq_encode(cb, x))
    queries = rng.standard_normal((7, dim)).astype(np.float32)
    l2 = pq.tables(queries)
    ip = pq.tables(queries, inner_product=True)
    for i in range(7):
        el2, eip = oracle.pq_tables(cb, queries[i])
        assert np.array_equal(bits(l2[i]), bits(el2)) and np.array_equal(bits(ip[i]), bits(eip))
        assert np.array_equal(bits(pq.adc(l2[i], codes)), bits(oracle.pq_adc(el2, codes)))
