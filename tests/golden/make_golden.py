#!/usr/bin/env python3
"""Writes the golden vectors under tests/golden/ from the COMPILED REFERENCE.

The reference library is oracle/_ref/libquiver_ref.so, built from the reference sources in place
by `make -C oracle ref` (only where those sources exist). Inputs are regenerated from seeded
generators (quiver_amd/datasets.py, numpy default_rng) and pinned by SHA-256; each fixture holds
inputs where they are small, and the reference's outputs.

    python tests/golden/make_golden.py            # small fixtures (seconds)
    python tests/golden/make_golden.py --full     # + the 1M-row IVF-PQ workload hashes (minutes)
    python tests/golden/make_golden.py --only nearest   # one fixture

Fixtures:
  kernels.npz     l2sqr / dot for dims 1..70, normalize bits (incl. zero and overflow rows)
  flat_c1.npz     flat search, 10,000 x 128 N(0,1) base, 100 queries, k=10: L2 / IP / cosine,
                  without and with a 10% allowed-id filter; fewer-than-k and label cases
  kmeans.npz      k-means (plain, duplicate points with empty-cluster splits, subsampled),
                  PQ train / encode / L2 + IP tables / ADC
  ivfpq_small.npz IVF-PQ train + add + search (n=4000, dim 32, nlist 32, m 8): centroids,
                  codebook, CSR lists, search outputs at nprobe 1/8/32, L2 (+refine), cosine
                  (+refine), inner product, and the refine-saturation case
  nearest.npz     nearest_centroid over seeded points and centroids (AVX2 tail branches,
                  duplicated centroids, overflowing distances)
  ivfpq_1m.json   (--full) SHA-256 of the trained state and lists of the 1,000,000 x 128 integer
                  mixture at nlist 2048, m 32 (trained on default_rng(31)'s first 100,000 rows),
                  and search outputs of the first 200 queries at nprobe 32
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import qvr  # noqa: E402
from oracle.oracle import Reference  # noqa: E402
from quiver_amd import datasets as D  # noqa: E402
from tests.golden.inputs import (IVF_CASES, IVF_ITERS, IVF_M, IVF_NLIST, IVF_NPROBES,  # noqa: E402
                                 NORMALIZE_DIMS, few_rows, flat_filter, int_mix_sample, ivf_points,
                                 kernel_pairs, kmeans_points, nearest_centroid_cases, normalize_rows,
                                 pq_points, sha)


def kernels(ref: Reference):
    a, b = kernel_pairs()
    l2 = np.array([ref.l2sqr(a[i, :i + 1], b[i, :i + 1]) for i in range(70)], np.float32)
    dot = np.array([ref.dot(a[i, :i + 1], b[i, :i + 1]) for i in range(70)], np.float32)
    out = dict(pairs_sha=np.array(sha(a) + sha(b)), kern_l2=l2, kern_dot=dot)
    for d in NORMALIZE_DIMS:
        x = normalize_rows(d)
        out[f"norm_sha_{d}"] = np.array(sha(x))
        out[f"norm_out_{d}"] = ref.normalize(x)
    return out


def flat_c1(ref: Reference):
    base, q = D.flat_small()
    allowed = flat_filter(base.shape[0])
    out = dict(base_sha=np.array(D.sha256(base)), query_sha=np.array(D.sha256(q)))
    for metric in ("l2", "ip", "cosine"):
        idx = ref.flat(base.shape[1], metric)
        idx.add(base)
        out[f"{metric}_labels"], out[f"{metric}_dist"] = idx.search(q, 10)
        out[f"{metric}_f_labels"], out[f"{metric}_f_dist"] = idx.search(q, 10, allowed=allowed)
    # fewer rows than k, custom labels, a two-label filter (tests/test_flat.cc:54-72 shape)
    small = few_rows()
    idx = ref.flat(8, "l2")
    idx.add(small, np.arange(100, 110, dtype=np.uint64))
    out["few_labels"], out["few_dist"] = idx.search(small[:3], 50)
    out["few_f_labels"], out["few_f_dist"] = idx.search(small[:3], 5, allowed=np.array([103, 107], np.uint64))
    return out


def kmeans_pq(ref: Reference):
    x, dup = kmeans_points()
    out = dict(km_sha=np.array(sha(x) + sha(dup)))
    out["km_plain"] = ref.kmeans(x, 40, 8, seed=3)
    out["km_split"] = ref.kmeans(dup, 16)
    out["km_sub"] = ref.kmeans(x, 8, 5, max_points_per_centroid=100, seed=7)
    px, pq_q = pq_points()
    cb = ref.pq_train(px, 4, iterations=10, seed=5)
    out.update(pq_sha=np.array(sha(px) + sha(pq_q)), pq_codebook=cb)
    out["pq_codes"] = ref.pq_encode(cb, px[:500])
    tabs = [ref.pq_tables(cb, pq_q[i]) for i in range(5)]
    out["pq_l2_tables"] = np.stack([t[0] for t in tabs])
    out["pq_ip_tables"] = np.stack([t[1] for t in tabs])
    b, s = ref.pq_adc(cb, out["pq_l2_tables"][0], out["pq_codes"])
    out["pq_adc_batch"], out["pq_adc_single"] = b, s
    return out


def nearest(ref: Reference):
    out = {}
    for i, (x, cent) in enumerate(nearest_centroid_cases()):
        out[f"case{i}_sha"] = np.array(sha(x) + sha(cent))
        out[f"case{i}_out"] = ref.nearest_centroid(x, cent)
    return out


def ivfpq_small(ref: Reference, tmp: str):
    base, q = ivf_points()
    out = dict(ivf_sha=np.array(sha(base) + sha(q)))
    for name, metric, store, refine in IVF_CASES:
        idx = ref.ivfpq(32, metric, nlist=IVF_NLIST, m=IVF_M, train_iterations=IVF_ITERS, store_vectors=store)
        idx.train(base)
        idx.add(base)
        path = os.path.join(tmp, f"{name}.qvr")
        idx.save(path)
        st = qvr.read_ivfpq(path)
        if name == "l2":
            out["l2_centroids"], out["l2_codebook"] = st["centroids"], st["codebook"]
        out[f"{name}_state_sha"] = np.array(sha(st["centroids"]) + sha(st["codebook"]))
        out[f"{name}_offsets"] = st["offsets"]
        out[f"{name}_order"] = st["labels"].astype(np.uint16)  # default labels = input row
        out[f"{name}_codes"] = st["codes"]
        for nprobe in IVF_NPROBES:
            out[f"{name}_p{nprobe}_labels"], out[f"{name}_p{nprobe}_dist"] = idx.search(
                q, 10, nprobe=nprobe, refine_factor=refine)
        if name == "l2r":  # k * refine_factor wraps to 0 (tests/test_regressions.cc:101-118)
            out["sat_labels"], out["sat_dist"] = idx.search(q[:10], 2, nprobe=32, refine_factor=1 << 63)
    return out


def ivfpq_1m(ref: Reference, tmp: str):
    base, q = D.int_mix()
    sample = int_mix_sample(base.shape[0])
    idx = ref.ivfpq(128, "l2", nlist=2048, m=32, train_iterations=20)
    idx.train(base[sample])
    idx.add(base)
    path = os.path.join(tmp, "big.qvr")
    idx.save(path)
    st = qvr.read_ivfpq(path)
    labels, dist = idx.search(q[:200], 10, nprobe=32)
    return {
        "base_sha": D.sha256(base), "query_sha": D.sha256(q), "sample_sha": sha(sample.astype(np.int64)),
        "centroids_sha": sha(st["centroids"]), "codebook_sha": sha(st["codebook"]),
        "offsets_sha": sha(st["offsets"]), "labels_sha": sha(st["labels"]), "codes_sha": sha(st["codes"]),
        "search_nprobe": 32, "search_labels": labels.astype(np.int64).tolist(),
        "search_dist_bits": dist.view(np.uint32).astype(np.int64).tolist(),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--full", action="store_true")
    ap.add_argument("--only", choices=["nearest"], help="write only this fixture")
    args = ap.parse_args()
    ref = Reference()
    print("reference SIMD path:", ref.simd_isa)
    if args.only == "nearest":
        np.savez_compressed(os.path.join(HERE, "nearest.npz"), **nearest(ref))
        return
    np.savez_compressed(os.path.join(HERE, "nearest.npz"), **nearest(ref))
    np.savez_compressed(os.path.join(HERE, "kernels.npz"), **kernels(ref))
    np.savez_compressed(os.path.join(HERE, "flat_c1.npz"), **flat_c1(ref))
    np.savez_compressed(os.path.join(HERE, "kmeans.npz"), **kmeans_pq(ref))
    with tempfile.TemporaryDirectory() as tmp:
        np.savez_compressed(os.path.join(HERE, "ivfpq_small.npz"), **ivfpq_small(ref, tmp))
        if args.full:
            with open(os.path.join(HERE, "ivfpq_1m.json"), "w") as f:
                json.dump(ivfpq_1m(ref, tmp), f)
    for name in sorted(os.listdir(HERE)):
        print(name, os.path.getsize(os.path.join(HERE, name)))


if __name__ == "__main__":
    main()
