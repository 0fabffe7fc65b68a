"""Child process of test_alloc_fault_gpu.py: runs a fixed sequence of index operations with the
device allocation numbered QVH_FAULT_ALLOC failing (core.hip's fault hook). The operation that
meets the failure must raise ValueError carrying the injected message and leave its index as it
was before the call: the same size, labels and inverted lists (read from host-side state, which
allocates nothing on the device), and searches that equal the oracle's on what the index holds.
Prints "fault at <step>" or "no fault", then "state ok"; exits non-zero on any violation."""

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

import quiver_amd as quiver  # noqa: E402
from oracle.oracle import IvfPqState, Oracle  # noqa: E402
from parity import assert_same_topk  # noqa: E402


def main():
    rng = np.random.default_rng(0)
    base = rng.standard_normal((6_000, 16)).astype(np.float32)
    q = rng.standard_normal((40, 16)).astype(np.float32)
    flat = quiver.FlatIndex(16)
    ivf = quiver.IvfPqIndex(16, nlist=16, m=4, train_iterations=3)

    def flat_state():
        return len(flat), np.asarray(flat._index._labels()).copy()

    def ivf_state():
        if not ivf.is_trained:
            return (False,)
        off, labels, codes = ivf.lists()
        return True, off.copy(), labels.copy(), codes.copy()

    steps = [
        ("flat add 1", "flat", lambda: flat.add(base[:2_000])),
        ("flat search", "flat", lambda: flat.search(q, 10)),
        ("flat add 2", "flat", lambda: flat.add(base[2_000:])),
        ("flat search 2", "flat", lambda: flat.search(q[:5], 10)),
        ("ivf train", "ivf", lambda: ivf.train(base)),
        ("ivf add 1", "ivf", lambda: ivf.add(base[:3_000])),
        ("ivf search", "ivf", lambda: ivf.search(q, 10, nprobe=8)),
        ("ivf add 2", "ivf", lambda: ivf.add(base[3_000:])),
    ]
    oracle = Oracle()
    for name, which, op in steps:
        before = flat_state() if which == "flat" else ivf_state()
        try:
            op()
            continue
        except ValueError as e:
            if "injected allocation failure" not in str(e):
                raise
        print("fault at", name, flush=True)
        if which == "flat":
            size, labels = flat_state()
            assert size == before[0] and np.array_equal(labels, before[1]), name
            if size:  # the device mirror still answers for exactly those rows
                got_l, got_d = flat.search(q, 10)
                rows, dist = oracle.flat_search(base[:size], q, 10)
                assert_same_topk(got_l, got_d, rows.astype(np.int64), dist)
        else:
            after = ivf_state()
            assert len(after) == len(before) and all(np.array_equal(a, b) for a, b in zip(after[1:], before[1:])), name
            if after[0] and len(ivf):
                cent, cb = ivf.centroids, ivf.codebook
                st = IvfPqState("l2", cent, cb, oracle.ivfpq_precompute(cent, cb))
                st.offsets, st.labels, st.codes = after[1], after[2], after[3]
                got_l, got_d = ivf.search(q, 10, nprobe=8)
                refs, dist = oracle.ivfpq_search(st, q, 10, 8)
                assert_same_topk(got_l, got_d, st.ref_to_label(refs), dist)
        print("state ok", flush=True)
        return
    print("no fault", flush=True)
    print("state ok", flush=True)


if __name__ == "__main__":
    main()
