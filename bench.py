#!/usr/bin/env python3
"""Benchmark of the Quiver search path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workloads (one "step" = one batched search of the whole query set; queries, index and outputs
resident in HBM):
  flat   exact L2, k=10, 1,000,000 x 128 fp32 base (integer-valued 64-component mixture,
         quiver_amd/datasets.py), 10,000 queries from the same mixture.
  ivfpq  the same base and queries in an IVF-PQ index: nlist 2048, m 32 x 8 bits, L2, residual
         PQ trained on 100,000 rows of a seeded permutation (numpy default_rng(31)); k=10,
         nprobe 32 (swept over 1..64, each point the median of back-to-back searches, untimed by
         the step clock).

Prints ONE JSON line. `value` is the flat workload's queries per second (query prep + fused MFMA
scan + merge/exact re-score), timed over K steps with the device synchronized on both sides;
the "ivfpq" object carries the same fields for the IVF-PQ workload, "flat_small_batches" the
flat search time of 1, 8, 32 and 128 of the same queries, and "flat_wide_rows" a 500,000 x 768
flat search (the chunked MFMA scan for rows wider than 128). `roofline` is each
workload's dominant kernel measured with HIP events on the stream it runs on: the flat scan's
algorithmic 2*n*d*nq FLOP per launch against the dense FP32 matrix peak (157.3 TFLOP/s), the
IVF-PQ list scan's algorithmic code bytes (sum over queries and probed lists of len * m) against
HBM peak (8 TB/s). `host_api` is the reference's own way of timing (bench/ann_bench.cc:351-357,
378): search_batch through the C++ classes with host buffers in and out, best of 3, which adds the
PCIe transfers. `cpu_baseline` is the reference's own CPU search (its sources compiled by
oracle/Makefile; the C restatement in oracle/ when that library is absent) timed on every CPU this
process may use (`host`: hardware_concurrency, affinity, cgroup quota) and on one thread, over a
bounded sample of the same queries; for IVF-PQ it loads the index built here from a .qvr file, so
both sides search identical trained state and lists.
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "batched QPS @k=10: flat 1M×128 L2 and IVF-PQ nprobe=32; % of MFMA/HBM peak"
FP32_MFMA_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0


class Hip:
    """The few HIP runtime calls the bench needs for device-resident buffers."""

    def __init__(self):
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        self.lib = L = C.CDLL(os.path.join(rocm, "lib", "libamdhip64.so"))
        L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        L.hipFree.argtypes = [C.c_void_p]
        L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        L.hipDeviceSynchronize.argtypes = []

    def malloc(self, nbytes: int) -> C.c_void_p:
        p = C.c_void_p()
        rc = self.lib.hipMalloc(C.byref(p), nbytes)
        if rc != 0:
            raise RuntimeError(f"hipMalloc({nbytes}) failed: {rc}")
        return p

    def h2d(self, dst, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        assert self.lib.hipMemcpy(dst, arr.ctypes.data_as(C.c_void_p), arr.nbytes, 1) == 0

    def d2h(self, arr: np.ndarray, src):
        assert self.lib.hipMemcpy(arr.ctypes.data_as(C.c_void_p), src, arr.nbytes, 2) == 0

    def sync(self):
        assert self.lib.hipDeviceSynchronize() == 0

    def copy_d2d(self, dst, src, nbytes: int):
        assert self.lib.hipMemcpy(dst, src, nbytes, 3) == 0


class Qvh:
    def __init__(self):
        self.lib = L = C.CDLL(os.path.join(ROOT, "quiver_amd", "lib", "libqvh.so"))
        L.qvh_last_error.restype = C.c_char_p
        L.qvh_flat_create.argtypes = [C.c_uint32, C.c_int, C.POINTER(C.c_void_p)]
        L.qvh_flat_append.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]
        L.qvh_flat_search_device.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint32,
                                             C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.qvh_flat_sync.argtypes = [C.c_void_p]
        L.qvh_flat_set_timing.argtypes = [C.c_void_p, C.c_int]
        L.qvh_flat_last_timing.argtypes = [C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_float),
                                           C.POINTER(C.c_float), C.POINTER(C.c_uint32)]
        L.qvh_flat_destroy.argtypes = [C.c_void_p]
        L.qvh_ivfpq_search_device.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint32, C.c_uint32,
                                              C.c_uint64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.qvh_ivfpq_sync.argtypes = [C.c_void_p]
        L.qvh_ivfpq_set_timing.argtypes = [C.c_void_p, C.c_int]
        L.qvh_ivfpq_last_timing.argtypes = [C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_float),
                                            C.POINTER(C.c_uint64)]
        L.qvh_device_info.argtypes = [C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t,
                                      C.POINTER(C.c_int)]

    def check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {self.lib.qvh_last_error().decode()}")

    def device(self):
        name = C.create_string_buffer(128)
        arch = C.create_string_buffer(64)
        cus = C.c_int()
        self.check(self.lib.qvh_device_info(name, 128, arch, 64, C.byref(cus)), "device")
        return name.value.decode(), arch.value.decode(), cus.value


def host_cores():
    """CPUs this process may use: the affinity mask, bounded by a cgroup v2 CPU quota if one is set
    (cpu.max), next to std::thread::hardware_concurrency() (os.cpu_count()), which is what the
    reference's ThreadPool(0) sizes itself to."""
    visible = os.cpu_count() or 1
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else visible
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
            if q != "max":
                quota = float(q) / float(period)
    except (OSError, ValueError):
        pass
    usable = affinity if quota is None else max(1, min(affinity, int(quota)))
    return {"hardware_concurrency": visible, "affinity": affinity, "cgroup_cpus": quota, "usable": usable}


COPY_CALIBRATION_BYTES = 256 << 20

# flat: the 1M x 128 L2 headline; ivfpq: IVF-PQ L2 on the same data; cosine: the 1.18M x 100 cosine
# flat search with allowed-id filters; wide: 500k x 768 L2; ivfcos: IVF-PQ cosine with refine 8.
WORKLOADS = ("flat", "ivfpq", "cosine", "wide", "ivfcos")


def load_traffic(name: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary profiles/<name>.md (its
    line "traffic_bytes_per_launch: N"), if present."""
    path = os.path.join(ROOT, "profiles", f"{name}.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    return None


def copy_calibration(hip: Hip):
    """One device-to-device copy of COPY_CALIBRATION_BYTES: the plain copy kernel whose
    FETCH_SIZE / WRITE_SIZE counters scale the others to bytes."""
    a = hip.malloc(COPY_CALIBRATION_BYTES)
    b = hip.malloc(COPY_CALIBRATION_BYTES)
    hip.copy_d2d(b, a, COPY_CALIBRATION_BYTES)
    hip.sync()
    hip.lib.hipFree(a)
    hip.lib.hipFree(b)


def bench_flat(args, hip: Hip, qvh: Qvh):
    from quiver_amd import datasets as D

    n, dim, nq, k = 1_000_000, 128, 10_000, 10
    base, queries = D.int_mix(n, nq)
    h = C.c_void_p()
    qvh.check(qvh.lib.qvh_flat_create(dim, 0, C.byref(h)), "create")
    qvh.check(qvh.lib.qvh_flat_append(h, base.ctypes.data_as(C.c_void_p), n, None), "append")
    d_q = hip.malloc(queries.nbytes)
    hip.h2d(d_q, queries)
    d_rows = hip.malloc(nq * k * 4)
    d_dist = hip.malloc(nq * k * 4)
    qvh.check(qvh.lib.qvh_flat_set_timing(h, 1), "timing")

    def step():
        qvh.check(qvh.lib.qvh_flat_search_device(h, d_q, nq, k, None, d_rows, d_dist, None), "search")

    for _ in range(args.warmup):
        step()
    qvh.check(qvh.lib.qvh_flat_sync(h), "sync")
    hip.sync()
    stages = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
        p, s, m, ns = C.c_float(), C.c_float(), C.c_float(), C.c_uint32()
        qvh.check(qvh.lib.qvh_flat_last_timing(h, C.byref(p), C.byref(s), C.byref(m), C.byref(ns)),
                  "timing")
        stages.append((p.value, s.value, m.value, ns.value))
    qvh.check(qvh.lib.qvh_flat_sync(h), "sync")
    hip.sync()
    elapsed = time.perf_counter() - t0

    rows = np.empty((nq, k), np.uint32)
    dist = np.empty((nq, k), np.float32)
    hip.d2h(rows, d_rows)
    hip.d2h(dist, d_dist)
    assert (rows != 0xFFFFFFFF).all() and (np.diff(dist, axis=1) >= 0).all(), "malformed results"

    st = np.array(stages, dtype=np.float64)
    scan_ms = float(st[:, 1].mean())
    flops = 2.0 * n * dim * nq
    achieved = flops / (scan_ms * 1e-3) / 1e12
    ms_per_step = elapsed / args.steps * 1e3
    result = {
        "value": nq / (ms_per_step * 1e-3),
        "ms_per_step": ms_per_step,
        "stage_ms": {"prep": float(st[:, 0].mean()), "scan": scan_ms, "merge": float(st[:, 2].mean())},
        "nsplit": int(st[0, 3]),
        "roofline": {"bound": "mfma", "kernel": "flat_scan_kernel<128,10>", "achieved": achieved,
                     "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / FP32_MFMA_PEAK_TFLOPS,
                     "traffic": load_traffic("flat_scan_int_mix_1m_pmc")},
        "config": {"workload": "flat exact L2 k=10: 1,000,000 x 128 fp32 integer-valued mixture, "
                               "10,000 queries batched", "n": n, "dim": dim, "nq": nq, "k": k},
    }
    # The reference's timing (bench/ann_bench.cc:351-357,378): FlatIndex::search_batch from host
    # buffers to host buffers, best of 3 after a warm-up, through the C++ class (Python binding).
    import quiver_amd as quiver

    host_index = quiver.FlatIndex(dim, "l2")
    host_index.add(base)
    host_index.search(queries, k)
    best = min(_timed(lambda: host_index.search(queries, k)) for _ in range(3))
    result["host_api"] = {"qps": nq / best, "ms": best * 1e3,
                          "note": "FlatIndex::search_batch, host numpy buffers in and out (PCIe included)"}
    del host_index
    if not args.no_extra:
        # Small batches (the first query: the few-query kernel; 8 and 32: the ring scan; 128: the
        # row-split MFMA scan): device time of one search from its stage events, and the caller's
        # wall time of search + sync.
        small = {}
        for b in (1, 8, 32, 128):
            dev, wall = [], []
            for _ in range(21):
                t = time.perf_counter()
                qvh.check(qvh.lib.qvh_flat_search_device(h, d_q, b, k, None, d_rows, d_dist, None), "search")
                qvh.check(qvh.lib.qvh_flat_sync(h), "sync")
                wall.append(time.perf_counter() - t)
                p, s, m, ns = C.c_float(), C.c_float(), C.c_float(), C.c_uint32()
                qvh.check(qvh.lib.qvh_flat_last_timing(h, C.byref(p), C.byref(s), C.byref(m), C.byref(ns)),
                          "timing")
                dev.append(p.value + s.value + m.value)
            small[f"nq{b}"] = {"device_us": float(np.median(dev[1:])) * 1e3,
                               "wall_us": float(np.median(wall[1:])) * 1e6}
        result["small_batches"] = small
    qvh.lib.qvh_flat_destroy(h)
    for p in (d_q, d_rows, d_dist):
        hip.lib.hipFree(p)
    return result, base, queries


def _timed(fn) -> float:
    t = time.perf_counter()
    fn()
    return time.perf_counter() - t


def bench_ivfpq(args, hip: Hip, qvh: Qvh, base, queries):
    import quiver_amd as quiver

    n, dim = base.shape
    nq, k, nlist, m, nprobe = queries.shape[0], 10, 2048, 32, 32
    sample = np.random.default_rng(31).permutation(n)[:100_000]
    idx = quiver.IvfPqIndex(dim, "l2", nlist=nlist, m=m)
    t0 = time.perf_counter()
    idx.train(base[sample])
    train_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    idx.add(base)
    add_s = time.perf_counter() - t0
    h = C.c_void_p(idx._index._device_handle)
    d_q = hip.malloc(queries.nbytes)
    hip.h2d(d_q, queries)
    d_refs = hip.malloc(nq * k * 8)
    d_dist = hip.malloc(nq * k * 4)
    qvh.check(qvh.lib.qvh_ivfpq_set_timing(h, 2), "timing")

    def search(probes):
        qvh.check(qvh.lib.qvh_ivfpq_search_device(h, d_q, nq, k, probes, 0, None, d_refs, d_dist, None),
                  "search")

    def timing(with_bytes=True):
        a, b, nb = C.c_float(), C.c_float(), C.c_uint64()
        qvh.check(qvh.lib.qvh_ivfpq_last_timing(h, C.byref(a), C.byref(b), C.byref(nb) if with_bytes else None),
                  "timing")
        return a.value, b.value, nb.value

    # Each sweep point: one search that also counts the probed code bytes (level 2), then five
    # back-to-back searches with stage events only (level 1); the stage times are the median of the
    # last four, so a point is measured at the same steady state as the timed loop below.
    sweep = {}
    for p in sorted(set(args.sweep) | {nprobe}):
        qvh.check(qvh.lib.qvh_ivfpq_set_timing(h, 2), "timing")
        search(p)
        qvh.check(qvh.lib.qvh_ivfpq_sync(h), "sync")
        nbytes = timing()[2]
        qvh.check(qvh.lib.qvh_ivfpq_set_timing(h, 1), "timing")
        runs = []
        for _ in range(5):
            search(p)
            runs.append(timing(with_bytes=False))
        sel, scan = (float(np.median([r[i] for r in runs[1:]])) for i in (0, 1))
        sweep[str(p)] = {"select_ms": sel, "scan_ms": scan, "code_bytes": nbytes,
                         "scan_hbm_frac": nbytes / (scan * 1e-3) / (HBM_PEAK_GBS * 1e9)}

    # The timed steps record stage events only (level 1): the code-byte count is a separate kernel.
    qvh.check(qvh.lib.qvh_ivfpq_set_timing(h, 1), "timing")
    for _ in range(args.warmup):
        search(nprobe)
    qvh.check(qvh.lib.qvh_ivfpq_sync(h), "sync")
    hip.sync()
    stages = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        search(nprobe)
        stages.append(timing(with_bytes=False))
    qvh.check(qvh.lib.qvh_ivfpq_sync(h), "sync")
    hip.sync()
    elapsed = time.perf_counter() - t0

    refs = np.empty((nq, k), np.uint64)
    dist = np.empty((nq, k), np.float32)
    hip.d2h(refs, d_refs)
    hip.d2h(dist, d_dist)
    assert (refs != np.uint64(2**64 - 1)).all() and (np.diff(dist, axis=1) >= 0).all(), "malformed results"

    # Host buffers in and out through IvfPqIndex::search_batch (bench/ann_bench.cc:351-357,378).
    idx.search(queries, k, nprobe=nprobe)
    best = min(_timed(lambda: idx.search(queries, k, nprobe=nprobe)) for _ in range(3))
    host_api = {"qps": nq / best, "ms": best * 1e3,
                "note": "IvfPqIndex::search_batch, host numpy buffers in and out (PCIe included)"}
    larger_k = {}
    if not args.no_extra:
        # Small batches (sliced queries): device time of the select and scan stages, and the
        # caller's wall time of search + sync.
        small = {}
        for b in (1, 100):
            dev, wall = [], []
            for _ in range(21):
                t = time.perf_counter()
                qvh.check(qvh.lib.qvh_ivfpq_search_device(h, d_q, b, k, nprobe, 0, None, d_refs, d_dist, None),
                          "search")
                qvh.check(qvh.lib.qvh_ivfpq_sync(h), "sync")
                wall.append(time.perf_counter() - t)
                sel_, scan_, _ = timing(with_bytes=False)
                dev.append(sel_ + scan_)
            small[f"nq{b}"] = {"device_us": float(np.median(dev[1:])) * 1e3,
                               "wall_us": float(np.median(wall[1:])) * 1e6}
        larger_k["small_batches"] = small
        # The same queries at nprobe 32 with k = 100 (150 candidates re-scored per query).
        k2 = 100
        d_refs2, d_dist2 = hip.malloc(nq * k2 * 8), hip.malloc(nq * k2 * 4)
        scans = []
        for _ in range(4):
            qvh.check(qvh.lib.qvh_ivfpq_search_device(h, d_q, nq, k2, nprobe, 0, None, d_refs2, d_dist2, None),
                      "search")
            scans.append(timing(with_bytes=False))
        qvh.check(qvh.lib.qvh_ivfpq_sync(h), "sync")
        sel2, scan2 = (float(np.median([t[i] for t in scans[1:]])) for i in (0, 1))
        larger_k["k100"] = {"select_ms": sel2, "scan_ms": scan2, "qps": nq / ((sel2 + scan2) * 1e-3)}
        for p in (d_refs2, d_dist2):
            hip.lib.hipFree(p)
    for p in (d_q, d_refs, d_dist):
        hip.lib.hipFree(p)

    st = np.array(stages, dtype=np.float64)
    scan_ms = float(st[:, 1].mean())
    code_bytes = int(sweep[str(nprobe)]["code_bytes"])
    achieved = code_bytes / (scan_ms * 1e-3) / 1e9
    ms_per_step = elapsed / args.steps * 1e3
    return idx, {
        "value": nq / (ms_per_step * 1e-3),
        "unit": "queries/s",
        "ms_per_step": ms_per_step,
        "stage_ms": {"select": float(st[:, 0].mean()), "scan": scan_ms},
        "host_api": host_api,
        "roofline": {"bound": "hbm", "kernel": "ivf_stream_kernel<8, true, 128, false, 4>", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": load_traffic("ivf_stream_int_mix_1m_nprobe32_pmc"),
                     "code_bytes_per_launch": code_bytes},
        "nprobe_sweep": sweep,
        **larger_k,
        "build": {"train_s": train_s, "add_s": add_s, "encode_vectors_per_s": n / add_s},
        "config": {"workload": "IVF-PQ L2 k=10 nprobe=32: 1,000,000 x 128 fp32 integer-valued mixture, "
                               "nlist 2048, m 32, trained on a 100,000-row sample; 10,000 queries batched",
                   "n": n, "dim": dim, "nq": nq, "k": k, "nlist": nlist, "m": m, "nprobe": nprobe},
    }


def bench_flat_filtered(args, qvh: Qvh):
    """1,183,514 x 100 unit-norm mixture, cosine, k=10, 10,000 queries, through the host-buffer API
    (FlatIndex.search: queries and filter from host memory), unfiltered and with allowed-id sets of
    10% and 0.5%; the stage times come from the same handle's HIP events."""
    import quiver_amd as quiver
    from quiver_amd import datasets as D

    base, q = D.unit_mix()
    n, dim, k = base.shape[0], base.shape[1], 10
    idx = quiver.FlatIndex(dim, "cosine")
    idx.add(base)
    h = C.c_void_p(idx._index._device_handle)
    qvh.check(qvh.lib.qvh_flat_set_timing(h, 1), "timing")
    out = {}
    for name, frac in (("none", None), ("10%", 0.10), ("0.5%", 0.005)):
        allowed = None if frac is None else D.allowed_ids(n, frac)
        admitted = n if allowed is None else allowed.size
        idx.search(q, k, filter=allowed)
        times, scans = [], []
        for _ in range(3):
            t0 = time.perf_counter()
            idx.search(q, k, filter=allowed)
            times.append(time.perf_counter() - t0)
            p_, s_, m_, ns = C.c_float(), C.c_float(), C.c_float(), C.c_uint32()
            qvh.check(qvh.lib.qvh_flat_last_timing(h, C.byref(p_), C.byref(s_), C.byref(m_), C.byref(ns)), "timing")
            scans.append(s_.value)
        scan_ms = float(np.mean(scans))
        tflops = 2.0 * admitted * dim * q.shape[0] / (scan_ms * 1e-3) / 1e12
        out[name] = {"qps_host_api": q.shape[0] / float(np.mean(times)), "admitted_rows": int(admitted),
                     "scan_ms": scan_ms, "scan_tflops_admitted": tflops,
                     "frac_of_fp32_mfma_peak": tflops / FP32_MFMA_PEAK_TFLOPS}
    return {"config": {"workload": "flat exact cosine k=10: 1,183,514 x 100 unit-norm 256-component mixture, "
                                   "10,000 queries, host-buffer API, allowed-id filters", "n": n, "dim": dim,
                       "nq": int(q.shape[0]), "k": k},
            "filters": out}


def bench_flat_wide(args, hip: Hip, qvh: Qvh):
    """Rows wider than the register-resident scan (the chunked MFMA scan): 500,000 x 768 N(0,1)
    fp32, L2, k=10, 10,000 queries, device-resident, median of 3 after one warm-up."""
    n, dim, nq, k = 500_000, 768, 10_000, 10
    rng = np.random.default_rng(768)
    base = rng.standard_normal((n, dim), dtype=np.float32)
    queries = rng.standard_normal((nq, dim), dtype=np.float32)
    h = C.c_void_p()
    qvh.check(qvh.lib.qvh_flat_create(dim, 0, C.byref(h)), "create")
    qvh.check(qvh.lib.qvh_flat_append(h, base.ctypes.data_as(C.c_void_p), n, None), "append")
    del base
    d_q = hip.malloc(queries.nbytes)
    hip.h2d(d_q, queries)
    d_rows = hip.malloc(nq * k * 4)
    d_dist = hip.malloc(nq * k * 4)
    qvh.check(qvh.lib.qvh_flat_set_timing(h, 1), "timing")
    stages, walls = [], []
    for i in range(4):
        t0 = time.perf_counter()
        qvh.check(qvh.lib.qvh_flat_search_device(h, d_q, nq, k, None, d_rows, d_dist, None), "search")
        qvh.check(qvh.lib.qvh_flat_sync(h), "sync")
        wall = time.perf_counter() - t0
        p_, s_, m_, ns = C.c_float(), C.c_float(), C.c_float(), C.c_uint32()
        qvh.check(qvh.lib.qvh_flat_last_timing(h, C.byref(p_), C.byref(s_), C.byref(m_), C.byref(ns)), "timing")
        if i:
            stages.append((p_.value, s_.value, m_.value))
            walls.append(wall)
    qvh.check(qvh.lib.qvh_flat_destroy(h), "destroy")
    for ptr in (d_q, d_rows, d_dist):
        hip.lib.hipFree(ptr)
    st = np.median(np.array(stages), axis=0)
    tflops = 2.0 * n * dim * nq / (st[1] * 1e-3) / 1e12
    return {"config": {"workload": "flat exact L2 k=10: 500,000 x 768 N(0,1) fp32, 10,000 queries batched (chunked "
                                   "MFMA scan)", "n": n, "dim": dim, "nq": nq, "k": k},
            "qps": nq / float(np.median(walls)),
            "stage_ms": {"prep": float(st[0]), "scan": float(st[1]), "merge": float(st[2])},
            "scan_tflops": tflops, "frac_of_fp32_mfma_peak": tflops / FP32_MFMA_PEAK_TFLOPS}


def bench_ivfpq_cosine_refine(args, hip: Hip, qvh: Qvh):
    """IVF-PQ cosine with exact re-ranking on the same 1,183,514 x 100 set: nlist 2048, m 25,
    stored vectors, refine_factor 8 (80 candidates re-ranked), k=10, nprobe 16 and 64."""
    import quiver_amd as quiver
    from quiver_amd import datasets as D

    base, q = D.unit_mix()
    n, dim, k, nq = base.shape[0], base.shape[1], 10, q.shape[0]
    sample = np.random.default_rng(31).permutation(n)[:100_000]
    idx = quiver.IvfPqIndex(dim, "cosine", nlist=2048, m=25, store_vectors=True)
    t0 = time.perf_counter()
    idx.train(base[sample])
    train_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    idx.add(base)
    add_s = time.perf_counter() - t0
    h = C.c_void_p(idx._index._device_handle)
    d_q = hip.malloc(q.nbytes)
    hip.h2d(d_q, q)
    d_refs = hip.malloc(nq * k * 8)
    d_dist = hip.malloc(nq * k * 4)
    out = {}
    for nprobe in (16, 64):
        qvh.check(qvh.lib.qvh_ivfpq_set_timing(h, 2), "timing")
        qvh.check(qvh.lib.qvh_ivfpq_search_device(h, d_q, nq, k, nprobe, 8, None, d_refs, d_dist, None), "search")
        a, b, nb = C.c_float(), C.c_float(), C.c_uint64()
        qvh.check(qvh.lib.qvh_ivfpq_last_timing(h, C.byref(a), C.byref(b), C.byref(nb)), "timing")
        qvh.check(qvh.lib.qvh_ivfpq_set_timing(h, 1), "timing")
        steps = []
        qvh.check(qvh.lib.qvh_ivfpq_sync(h), "sync")
        t0 = time.perf_counter()
        for _ in range(5):
            qvh.check(qvh.lib.qvh_ivfpq_search_device(h, d_q, nq, k, nprobe, 8, None, d_refs, d_dist, None), "search")
            sa, sb = C.c_float(), C.c_float()
            qvh.check(qvh.lib.qvh_ivfpq_last_timing(h, C.byref(sa), C.byref(sb), None), "timing")
            steps.append((sa.value, sb.value))
        qvh.check(qvh.lib.qvh_ivfpq_sync(h), "sync")
        elapsed = time.perf_counter() - t0
        st = np.array(steps)
        scan_ms = float(st[:, 1].mean())
        # The re-ranking reads each query's k * refine_factor candidates' stored vectors (dim fp32
        # each) beside the codes: algorithmic bytes of the same scan stage.
        refine_bytes = nq * k * 8 * dim * 4
        out[str(nprobe)] = {"qps": nq * 5 / elapsed, "select_ms": float(st[:, 0].mean()), "scan_ms": scan_ms,
                            "code_bytes": nb.value, "refine_bytes": refine_bytes,
                            "scan_hbm_frac": nb.value / (scan_ms * 1e-3) / (HBM_PEAK_GBS * 1e9),
                            "scan_hbm_frac_with_refine":
                                (nb.value + refine_bytes) / (scan_ms * 1e-3) / (HBM_PEAK_GBS * 1e9)}
    for ptr in (d_q, d_refs, d_dist):
        hip.lib.hipFree(ptr)
    return {"config": {"workload": "IVF-PQ cosine k=10 refine_factor 8: 1,183,514 x 100 unit-norm mixture, "
                                   "nlist 2048, m 25, stored vectors, trained on a 100,000-row sample; "
                                   "10,000 queries", "n": n, "dim": dim, "nq": nq, "k": k, "nlist": 2048, "m": 25,
                       "refine_factor": 8},
            "build": {"train_s": train_s, "add_s": add_s}, "nprobe": out}


def cpu_baseline_ivfpq(idx, queries, k, nprobe, seconds, threads):
    """QPS of the reference CPU IVF-PQ search on the index built here (loaded from a .qvr file)."""
    from oracle.oracle import IvfPqState, Oracle, Reference

    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "ivfpq.qvr")
        idx.save(path)
        try:
            ref = Reference()
            kind = "reference"
            ix = ref.ivfpq_load(path)
            run = lambda q: ix.search(q, k, nprobe=nprobe, threads=threads)
        except FileNotFoundError:
            orc = Oracle()
            kind = "port"
            cent, cb = idx.centroids, idx.codebook
            off, labels, codes = idx.lists()
            st = IvfPqState("l2", cent, cb, orc.ivfpq_precompute(cent, cb))
            st.offsets, st.labels, st.codes, st.vectors = off, labels, codes, None
            run = lambda q: orc.ivfpq_search(st, q, k, nprobe, 0, None, threads=threads)
        batch = 256
        done = 0
        t0 = time.perf_counter()
        while done == 0 or time.perf_counter() - t0 < seconds:
            b = done % queries.shape[0]
            run(queries[b:b + batch])
            done += min(batch, queries.shape[0] - b)
        elapsed = time.perf_counter() - t0
    return {"value": done / elapsed, "unit": "queries/s", "cores": threads, "kind": kind,
            "sample": f"{done} queries (the 10,000-query set cycled in batches of {batch}) at nprobe {nprobe} "
                      f"against the same 1,000,000-vector index loaded from .qvr ({elapsed:.1f} s, "
                      f"ThreadPool({threads}), grain 1)"}


def cpu_baseline_flat(base, queries, k, seconds, threads):
    """QPS of the reference CPU flat search over a bounded prefix of the query batch."""
    from oracle.oracle import Oracle, Reference

    try:
        ref = Reference()
        kind = "reference"
        idx = ref.flat(base.shape[1], "l2")
        idx.add(base)
        run = lambda q: idx.search(q, k, threads=threads)
    except FileNotFoundError:
        orc = Oracle()
        kind = "port"
        run = lambda q: orc.flat_search(base, q, k, "l2", threads=threads)
    batch = 2 * threads
    done = 0
    t0 = time.perf_counter()
    while done < queries.shape[0] and (time.perf_counter() - t0 < seconds or done == 0):
        run(queries[done:done + batch])
        done = min(done + batch, queries.shape[0])
    elapsed = time.perf_counter() - t0
    return {"value": done / elapsed, "unit": "queries/s", "cores": threads, "kind": kind,
            "sample": f"first {done} of {queries.shape[0]} queries against all {base.shape[0]} rows "
                      f"({elapsed:.1f} s, ThreadPool({threads}), grain 1)"}


def with_one_thread(full, one):
    """The multithreaded baseline with the one-thread run beside it (the reference reports both)."""
    out = dict(full)
    out["one_thread"] = {"value": one["value"], "sample": one["sample"]}
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=250)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="CPU baseline threads (default: every CPU the process may use, cgroup quota included)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the filtered cosine flat and the cosine IVF-PQ refine workloads")
    ap.add_argument("--copy-calibration", action="store_true",
                    help=f"first run one {COPY_CALIBRATION_BYTES >> 20} MiB device copy (for rocprofv3 --pmc scaling)")
    ap.add_argument("--workloads", default=",".join(WORKLOADS),
                    help="comma-separated subset of " + ",".join(WORKLOADS) + " (for profiling one workload; "
                         "the JSON line always carries flat, whose numbers are `value`)")
    ap.add_argument("--sweep", default="1,4,8,16,32,64", help="nprobe points of the IVF-PQ sweep")
    args = ap.parse_args()
    args.workloads = set(w for w in args.workloads.split(",") if w)
    unknown = args.workloads - set(WORKLOADS)
    if unknown:
        ap.error(f"unknown workloads {sorted(unknown)}")
    if args.no_extra:
        args.workloads &= {"flat", "ivfpq"}
    args.sweep = [int(p) for p in args.sweep.split(",") if p]
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build's search path runs on a single MI355X and "
              f"has no multi-GPU mode (asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)

    hip, qvh = Hip(), Qvh()
    name, arch, cus = qvh.device()
    t_start = time.perf_counter()

    def done(stage):  # one progress line per finished stage (stderr; stdout carries the JSON line)
        print(f"[bench] {stage} done at {time.perf_counter() - t_start:.1f} s", file=sys.stderr, flush=True)

    if args.copy_calibration:
        copy_calibration(hip)
    flat, base, queries = bench_flat(args, hip, qvh)
    done("flat")
    idx, ivf = None, None
    if "ivfpq" in args.workloads:
        idx, ivf = bench_ivfpq(args, hip, qvh, base, queries)
        done("ivfpq")
    extra = {}
    if not args.no_extra:
        extra["flat_small_batches"] = flat["small_batches"]
    if "cosine" in args.workloads:
        extra["flat_cosine_filtered"] = bench_flat_filtered(args, qvh)
        done("flat_cosine_filtered")
    if "wide" in args.workloads:
        extra["flat_wide_rows"] = bench_flat_wide(args, hip, qvh)
        done("flat_wide_rows")
    if "ivfcos" in args.workloads:
        extra["ivfpq_cosine_refine"] = bench_ivfpq_cosine_refine(args, hip, qvh)
        done("ivfpq_cosine_refine")
    cpu = None
    if ivf is not None:
        ivf["cpu_baseline"] = None
    cores = host_cores()
    if not args.no_cpu:
        threads = args.cpu_threads or cores["usable"]
        cpu = with_one_thread(cpu_baseline_flat(base, queries, 10, args.cpu_seconds, threads),
                              cpu_baseline_flat(base, queries, 10, args.cpu_seconds / 3, 1))
        cpu["host"] = cores
        done("cpu_baseline flat")
        if ivf is not None:
            ivf["cpu_baseline"] = with_one_thread(
                cpu_baseline_ivfpq(idx, queries, 10, 32, args.cpu_seconds / 3, threads),
                cpu_baseline_ivfpq(idx, queries, 10, 32, args.cpu_seconds / 3, 1))
            done("cpu_baseline ivfpq")
    line = {
        "metric": METRIC,
        "value": flat["value"],
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": flat["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded, quiver_amd/datasets.py)",
        "config": flat["config"],
        "roofline": flat["roofline"],
        "cpu_baseline": cpu,
        "stage_ms": flat["stage_ms"],
        "host_api": flat["host_api"],
        "nsplit": flat["nsplit"],
        "ivfpq": ivf,
        **extra,
        "device": {"name": name, "arch": arch, "compute_units": cus},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
