# SPDX-License-Identifier: Apache-2.0
"""Flat-search benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C2] [--nq N] [--storage f32]

A step is one exact search of the configuration's whole query batch against the
whole database, with queries, database and outputs already resident in HBM (the
device-pointer C ABI entry point; the host-pointer entry adds PCIe copies and is
not what `value` measures). Default workload: BASELINE.json configs[1] (C2):
L2, nb = 1,000,000 x d = 128 GMM(1,024 centres, sigma 0.3), nq = 10,000, k = 100,
seed 1. Prints ONE JSON line on stdout; progress goes to stderr.

roofline: the dominant kernel is scan_filter (fused MFMA distance tile +
threshold filter over the full database, one launch per step). achieved =
2 * nq * nb * d algorithmic FLOP per launch / its mean duration, timed with HIP
events on the launch stream over a second pass of the same K searches (the
timed pass itself carries no instrumentation), against the dense MFMA peak
of the storage type (fp32 157.3, fp16/bf16 2516.6 TFLOP/s) -- or, where the
algorithmic bytes (database in its storage type + queries + results) at 8 TB/s
take longer than the FLOP at peak (C4 fp32 nq <= 16, C4 fp16 at every nq),
those bytes per launch against 8 TB/s. roofline.step_frac is the same work
over ms_per_step: the whole search (every launch, gap and synchronisation)
against the roofline.

--storage f16 / bf16 runs the reduced-precision variant (database and queries
rounded to that type, fp32 accumulation; mflat_flat_create_ex).

cpu_baseline: the oracle's restatement of the reference CPU path (cpuSearch,
src/FlatIndex.mm:259-290; serial, as the reference) timed on a bounded prefix of
the same query batch against the full database, on one host core.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "metal-flat_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_F16_MFMA_TFLOPS = 2516.6   # dense fp16 / bf16
PEAK_HBM_GBS = 8000.0

# Bytes per launch of the dominant kernel through L2's memory side, from rocprofv3
# FETCH_SIZE + WRITE_SIZE runs scaled by a plain-copy calibration (x2.0, x1.0), as
# committed under profiles/. Keyed by (config, nq, storage); reported as
# roofline.traffic for the configuration it was measured on, null otherwise.
MEASURED_TRAFFIC_BYTES = {
    ("C1", 1_000, "f32"): 61.9e6,
    ("C2", 10_000, "f32"): 4.636e9,
    ("C2", 10_000, "f16"): 2.090e9,
    ("C2", 10_000, "bf16"): 2.084e9,
    ("C3", 10_000, "f32"): 239.84e9,
    ("C3", 10_000, "bf16"): 22.0e9,
    ("C4", 1, "f32"): 3.881e9,
    ("C4", 1, "f16"): 1.961e9,
    ("C4", 16, "f32"): 3.882e9,
    ("C4", 16, "f16"): 1.963e9,
    ("C4", 64, "f32"): 3.890e9,
    ("C4", 64, "f16"): 1.970e9,
    ("C5", 2_000_000, "f32"): 30.7e9,
    # IVF fine scan (both launches of a search), C2's data, nlist 1000, nprobe 62
    ("IVF", 1000, 62, "f32"): 4.66e9,
    # IVF-PQ ADC full pass, C2's data, nlist 1000, nprobe 62, m_sub 16 (lookup tables, codes, cross tables)
    ("IVFPQ", 1000, 62, 16): 10.61e9,
}

WORKLOADS = {
    "C1": ("C1: flat L2, nb=100,000 x d=128 integer-valued U{0..255}, nq=1,000, k=10, seed 0", 0, 10),
    "C2": ("C2: flat L2, nb=1,000,000 x d=128 GMM(1024 centres, sigma 0.3), nq=10,000, k=100, seed 1", 0, 100),
    "C3": ("C3: flat inner product, nb=1,000,000 x d=768 unit N(0,I), nq=10,000, k=100, seed 2", 1, 100),
    "C4": ("C4: flat L2, nb=10,000,000 x d=96 U[-1,1], nq={nq}, k=10, seed 3", 0, 10),
    "C5": ("C5: k-means assignment (k=1), 2,000,000 points x d=128 GMM(4096, sigma 0.5) vs 65,536 centroids, seed 4", 0, 1),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_data(cfg, nq_override):
    import datagen

    if cfg == "C1":
        return datagen.sift_like()
    if cfg == "C2":
        return datagen.gmm()
    if cfg == "C3":
        return datagen.unit_normal()
    if cfg == "C4":
        return datagen.uniform_pm1(nq=nq_override or 64)
    if cfg == "C5":
        return datagen.kmeans_assign()
    raise SystemExit(f"unknown config {cfg}")


def host_threads():
    """Host cores this process may use (the GPU box grants 16 per GPU)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def cpu_baseline(x, q, k, metric, gpu_ids, storage=0, threads=1, seconds_target=12.0):
    """Times the oracle on `threads` host cores (1 = the reference's serial
    cpuSearch; more = parallel over queries, as the reference's bench,
    bench/bench.mm:134-156) on a prefix of the queries sized to ~10-15 s.
    Reduced-precision storage: the oracle runs on the identically rounded inputs."""
    import numpy as np
    import oracle

    if storage:
        x, q, metric = oracle.storage_inputs(x, q[:4096], metric, storage)

    nb, d = x.shape
    # per-query cost ~ nb*d sequential fp32 steps; calibrate on one query per thread
    t0 = time.perf_counter()
    oracle.flat_search(x, q[:threads], k, metric=metric, threads=threads)
    one = max(time.perf_counter() - t0, 1e-6) / threads
    n = int(max(1, min(q.shape[0], seconds_target / one)))
    t0 = time.perf_counter()
    oi, od = oracle.flat_search(x, q[:n], k, metric=metric, threads=threads)
    dt = time.perf_counter() - t0
    recall = float(np.mean([len(set(oi[r].tolist()) & set(gpu_ids[r].tolist())) / k for r in range(n)]))
    swaps, far = near_tie_swaps(x, q[:n], oi, od, gpu_ids[:n], metric)
    where = "one host core" if threads == 1 else f"{threads} host threads (queries split across them)"
    return {
        "value": n / dt,
        "unit": "queries/s",
        "cores": threads,
        "kind": "port",
        "sample": f"first {n} of the {q.shape[0]} queries against all {nb} rows (d={d}, k={k}), "
                  f"{dt:.1f} s on {where}; GPU/oracle id agreement on the sample {recall:.5f} "
                  f"({swaps} differing ids, {far} of them outside the 1e-5 near-tie gap of the k-th value)",
    }


def near_tie_swaps(x, q, oi, od, gi, metric):
    """Ids the GPU returned that the oracle did not, and how many of them lie
    outside the near-tie gap (1e-5 relative of the oracle's k-th value, plus for
    L2 2^-20 (||q||^2 + ||x||^2)): float64 distances of those rows only."""
    import numpy as np

    swaps = far = 0
    k = oi.shape[1]
    for r in range(oi.shape[0]):
        extra = set(gi[r].tolist()) - set(oi[r].tolist())
        swaps += len(extra)
        if not extra:
            continue
        qq = q[r].astype(np.float64)
        kth = float(od[r, k - 1])
        for i in extra:
            if i < 0:
                far += 1
                continue
            xx = x[i].astype(np.float64)
            v = float(np.sum((xx - qq) ** 2)) if metric == 0 else float(xx @ qq)
            floor = 2.0 ** -20 * (float(qq @ qq) + float(xx @ xx)) if metric == 0 else 1e-6
            if not abs(v - kth) <= 1e-5 * abs(kth) + floor:
                far += 1
    return swaps, far


def kmeans_bench(iters):
    """ms per device k-means iteration (assignment of every training point + the
    centroid update) on C5's 2,000,000 x 128 points with 65,536 cells, taken as
    (T(iters) - T(0)) / iters so the upload, seeding and final assignment cancel."""
    import datagen
    import mflat

    mflat.load()
    cents, pts = datagen.kmeans_assign()
    nlist = cents.shape[0]
    del cents
    log(f"[bench] kmeans: {pts.shape[0]} x {pts.shape[1]} points, {nlist} cells, {iters} iterations")
    mflat.kmeans_train(pts[:100_000], 1024, 1, 256)   # warm-up (kernel loading)
    t = []
    for it in (0, iters):
        t0 = time.perf_counter()
        mflat.kmeans_train(pts, nlist, it, 256)
        t.append(time.perf_counter() - t0)
        log(f"[bench] kmeans iters={it}: {t[-1]:.3f}s")
    per = (t[1] - t[0]) * 1000.0 / iters
    flop = 2.0 * pts.shape[0] * nlist * pts.shape[1]
    print(json.dumps({"metric": "ms per device k-means iteration (assign + update)", "value": round(per, 3),
                      "unit": "ms", "higher_is_better": False, "n_gpus": 1, "iters": iters,
                      "config": {"workload": "C5 points (2,000,000 x 128 GMM(4096, sigma 0.5)), 65,536 cells, "
                                             "max 256 points per cell (all points train), seed 4"},
                      "assign_tflops_equiv": round(flop / (per / 1000.0) / 1e12, 2),
                      "total_s": {"iters_0": round(t[0], 3), f"iters_{iters}": round(t[1], 3)}}), flush=True)


def ivf_bench(args):
    """IVF search (mflat_ivf_*) on C2's database and queries (or, --config C3,
    C3's: d = 768 inner product, which runs 32-query work items only): nlist and nprobe by
    the reference bench's rule (bench/bench.mm:96-101: nlist = max(64, sqrt(N)),
    nprobe = max(1, nlist / 16)) unless given, k = C2's 100. A step is one search
    of the whole query batch (device pointers, inputs resident in HBM); the build
    (k-means + cell-major layout) is timed once, apart. roofline: the fine-scan
    launches (ivf_scan family: the bounded pass over every probed cell, in
    128- and 32-query work items, and its retries) against the fp32 MFMA peak,
    with algorithmic FLOP = 2 d x the rows of every query's probed cells. cpu_baseline: the oracle's searchCpu restatement
    over the same probed cells on a bounded query prefix."""
    import numpy as np
    import datagen
    import hipmem
    import mflat
    import oracle

    mflat.load()
    c3 = args.config == "C3"
    if args.config not in ("C2", "C3"):
        raise SystemExit("--ivf runs on C2's or C3's data")
    x, q = datagen.unit_normal() if c3 else datagen.gmm()
    metric = mflat.MFLAT_METRIC_INNER_PRODUCT if c3 else mflat.MFLAT_METRIC_L2
    mname = "inner product" if c3 else "L2"
    if args.nq:
        q = q[: args.nq]
    nb, d = x.shape
    nq = q.shape[0]
    k = 100
    nlist = args.nlist or max(64, int(np.sqrt(nb)))
    nprobe = args.nprobe or max(1, nlist // 16)
    storage = mflat.STORAGE_NAMES[args.storage]
    log(f"[bench] ivf: nb={nb} d={d} nq={nq} k={k} nlist={nlist} nprobe={nprobe} storage={args.storage}")
    idx = mflat.IvfIndex(d, metric, nlist, storage)
    t0 = time.perf_counter()
    idx.build(x)
    build_s = time.perf_counter() - t0
    log(f"[bench] ivf build {build_s:.2f}s")
    _, start, rid = idx.coarse()
    probed = idx.probe(q, nprobe)
    sizes = np.diff(start.astype(np.int64))
    rows = int(sizes[probed].sum())
    flop = 2.0 * d * rows

    qd = hipmem.DeviceArray.from_numpy(q)
    ids = hipmem.DeviceArray((nq, k), np.int32)
    dist = hipmem.DeviceArray((nq, k), np.float32)
    for i in range(args.warmup):
        idx.search_device(qd, k, nprobe, ids, dist)
    hipmem.synchronize()
    mflat.profile_reset()
    mflat.profile_enable(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        idx.search_device(qd, k, nprobe, ids, dist)
    hipmem.synchronize()
    elapsed = time.perf_counter() - t0
    mflat.profile_enable(False)
    kern = {}
    for fam in ("ivf_scan", "ivf_bound", "scan_filter", "scan_sample", "select", "norms", "prep"):
        ms, n = mflat.profile_read(fam)
        if n:
            kern[fam] = {"total_ms": round(ms, 4), "launches": n, "mean_ms": round(ms / n, 4)}
    gi = ids.numpy()
    log(f"[bench] ivf {args.steps} steps in {elapsed:.3f}s")

    peak = PEAK_FP32_MFMA_TFLOPS if storage == mflat.MFLAT_STORAGE_F32 else PEAK_F16_MFMA_TFLOPS
    ach = flop * args.steps / (kern["ivf_scan"]["total_ms"] / 1000.0) / 1e12
    flat = mflat.FlatIndex(d, metric)
    flat.add(x)
    fi, _, _ = flat.search(q, k)
    flat.close()
    recall = float(np.mean([len(set(gi[r].tolist()) & set(fi[r].tolist())) / k for r in range(nq)]))
    out = {
        "metric": f"QPS, IVF {mname} d={d} nb={nb} nlist={nlist} nprobe={nprobe} k={k} (1 GPU)",
        "value": round(nq * args.steps / elapsed, 2),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1000.0 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"f32": "fp32", "f16": "fp16 storage, fp32 accumulate",
                  "bf16": "bf16 storage, fp32 accumulate"}[args.storage],
        "data": "synthetic",
        "config": {"workload": (f"IVF over C3's database and queries (unit N(0,I), d=768, inner product, seed 2), "
                                if c3 else
                                f"IVF over C2's database and queries (GMM 1024 centres, sigma 0.3, seed 1), ") +
                               f"nlist={nlist}, nprobe={nprobe}, k={k}", "nb": nb, "d": d, "nq": nq, "k": k,
                   "nlist": nlist, "nprobe": nprobe, "storage": args.storage, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(ach, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(ach / peak, 4),
                     "traffic": MEASURED_TRAFFIC_BYTES.get(("IVF", nlist, nprobe, args.storage))
                     if nq == 10_000 and not c3 else None},
        "kernels": kern,
        "probed_rows_per_query": round(rows / nq, 1),
        "recall_vs_exact_flat": round(recall, 5),
        "build_s": round(build_s, 3),
    }
    if not args.no_cpu_baseline:
        payload = oracle.ivf_payload(x, rid)   # the reference keeps reorderedDb resident
        for threads, key in ((1, "cpu_baseline"), (host_threads(), "cpu_baseline_all_cores")):
            log(f"[bench] ivf cpu baseline ({threads} threads) ...")
            t0 = time.perf_counter()
            oracle.ivf_search(None, start, rid, q[:threads], k, probed[:threads], 1 if c3 else 0,
                              threads=threads, payload=payload)
            one = max(time.perf_counter() - t0, 1e-6) / threads
            n = int(max(1, min(nq, 12.0 / one)))
            t0 = time.perf_counter()
            oi, _ = oracle.ivf_search(None, start, rid, q[:n], k, probed[:n], 1 if c3 else 0, threads=threads,
                                      payload=payload)
            dt = time.perf_counter() - t0
            agree = float(np.mean([len(set(oi[r].tolist()) & set(gi[r].tolist())) / k for r in range(n)]))
            out[key] = {"value": n / dt, "unit": "queries/s", "cores": threads, "kind": "port",
                        "sample": f"first {n} of the {nq} queries over the same probed cells (searchCpu "
                                  f"restatement), {dt:.1f} s on {threads} host thread(s); GPU/oracle id "
                                  f"agreement on the sample {agree:.5f}"}
    idx.close()
    print(json.dumps(out), flush=True)


def ivfpq_bench(args):
    """IVF-PQ search (mflat_ivfpq_*) on C2's database and queries: nlist and
    nprobe by the reference bench's IVF rule, m_sub = 16 (16-byte codes for
    d = 128, the reference header's example), k = 10 (the reference's IVF-PQ
    serves k <= 64), rerank 16 k (the header's suggestion). A step is one search
    of the whole batch (device pointers). roofline: the ADC fine scan (ivf_scan
    family) is bound by LDS gathers, neither HBM nor MFMA -- M table reads of
    4 bytes per (query, probed row); achieved = those bytes / its time against
    the LDS read peak (128 B per clock per CU, 256 CUs, 2.4 GHz); traffic = its
    measured HBM bytes (FETCH_SIZE + WRITE_SIZE, scaled as for the flat scan)."""
    import numpy as np
    import datagen
    import hipmem
    import mflat
    import oracle

    mflat.load()
    x, q = datagen.gmm()
    if args.nq:
        q = q[: args.nq]
    nb, d = x.shape
    nq = q.shape[0]
    k = 10
    M = 16
    rerank = args.rerank if args.rerank >= 0 else 16 * k
    nlist = args.nlist or max(64, int(np.sqrt(nb)))
    nprobe = args.nprobe or max(1, nlist // 16)
    log(f"[bench] ivfpq: nb={nb} d={d} nq={nq} k={k} nlist={nlist} nprobe={nprobe} m_sub={M} rerank={rerank}")
    idx = mflat.IvfPqIndex(d, mflat.MFLAT_METRIC_L2, nlist, M, rerank=rerank > k)
    t0 = time.perf_counter()
    idx.build(x)
    build_s = time.perf_counter() - t0
    log(f"[bench] ivfpq build {build_s:.2f}s")
    cent, start, rid, pqc, codes = idx.coarse()
    probed = idx.probe(q, nprobe)
    rows = int(np.diff(start.astype(np.int64))[probed].sum())

    qd = hipmem.DeviceArray.from_numpy(q)
    ids = hipmem.DeviceArray((nq, k), np.int32)
    dist = hipmem.DeviceArray((nq, k), np.float32)
    for _ in range(args.warmup):
        idx.search_device(qd, k, nprobe, ids, dist, rerank=rerank)
    hipmem.synchronize()
    mflat.profile_reset()
    mflat.profile_enable(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        idx.search_device(qd, k, nprobe, ids, dist, rerank=rerank)
    hipmem.synchronize()
    elapsed = time.perf_counter() - t0
    mflat.profile_enable(False)
    kern = {}
    for fam in ("ivf_scan", "ivf_bound", "scan_filter", "select", "norms", "prep"):
        ms, n = mflat.profile_read(fam)
        if n:
            kern[fam] = {"total_ms": round(ms, 4), "launches": n, "mean_ms": round(ms / n, 4)}
    gi = ids.numpy()
    log(f"[bench] ivfpq {args.steps} steps in {elapsed:.3f}s")
    lds_bytes = 4.0 * M * rows   # table reads of the scan per search
    peak = 128.0 * 256 * 2.4e9 / 1e9
    ach = lds_bytes * args.steps / (kern["ivf_scan"]["total_ms"] / 1000.0) / 1e9
    flat = mflat.FlatIndex(d, mflat.MFLAT_METRIC_L2)
    flat.add(x)
    fi, _, _ = flat.search(q, k)
    flat.close()
    recall = float(np.mean([len(set(gi[r].tolist()) & set(fi[r].tolist())) / k for r in range(nq)]))
    out = {
        "metric": f"QPS, IVF-PQ L2 d={d} nb={nb} nlist={nlist} nprobe={nprobe} m={M} k={k} rerank={rerank} (1 GPU)",
        "value": round(nq * args.steps / elapsed, 2),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1000.0 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8 codes, fp32 tables",
        "data": "synthetic",
        "config": {"workload": f"IVF-PQ over C2's database and queries (GMM 1024 centres, sigma 0.3, seed 1), "
                               f"nlist={nlist}, nprobe={nprobe}, m_sub={M}, k={k}, rerank={rerank}",
                   "nb": nb, "d": d, "nq": nq, "k": k, "nlist": nlist, "nprobe": nprobe, "m_sub": M,
                   "rerank": rerank, "parallelism": "single GPU"},
        "roofline": {"bound": "lds", "achieved": round(ach, 2), "peak": peak, "unit": "GB/s",
                     "frac": round(ach / peak, 4),
                     "traffic": MEASURED_TRAFFIC_BYTES.get(("IVFPQ", nlist, nprobe, M)) if nq == 10_000 else None},
        "kernels": kern,
        "probed_rows_per_query": round(rows / nq, 1),
        "recall_vs_exact_flat": round(recall, 5),
        "code_bytes": int(nb * M),
        "build_s": round(build_s, 3),
    }
    if not args.no_cpu_baseline:
        for threads, key in ((1, "cpu_baseline"), (host_threads(), "cpu_baseline_all_cores")):
            log(f"[bench] ivfpq cpu baseline ({threads} threads) ...")
            t0 = time.perf_counter()
            oracle.ivfpq_search(cent, start, rid, codes, pqc, q[:threads], rerank if rerank > k else k,
                                probed[:threads], 0, threads=threads)
            one = max(time.perf_counter() - t0, 1e-6) / threads
            n = int(max(1, min(nq, 12.0 / one)))
            t0 = time.perf_counter()
            kr = rerank if rerank > k else k
            si, _ = oracle.ivfpq_search(cent, start, rid, codes, pqc, q[:n], kr, probed[:n], 0, threads=threads)
            oi = oracle.pq_rerank(x, q[:n], si, k, 0)[0] if rerank > k else si
            dt = time.perf_counter() - t0
            agree = float(np.mean([len(set(oi[r].tolist()) & set(gi[r].tolist())) / k for r in range(n)]))
            out[key] = {"value": n / dt, "unit": "queries/s", "cores": threads, "kind": "port",
                        "sample": f"first {n} of the {nq} queries over the same probed cells (searchCpu and "
                                  f"rerank restatement), {dt:.1f} s on {threads} host thread(s); GPU/oracle id "
                                  f"agreement on the sample {agree:.5f}"}
    idx.close()
    print(json.dumps(out), flush=True)


def roofline_of(flop, byts, esize, kernel_s_per_launch, step_s, traffic):
    """Roofline of one search: the bound is whichever of FLOP / dense peak and
    algorithmic bytes / HBM bandwidth takes longer; frac = that work over the
    dominant kernel's mean launch, step_frac = over the whole search."""
    peak = PEAK_FP32_MFMA_TFLOPS if esize == 4 else PEAK_F16_MFMA_TFLOPS
    if byts / (PEAK_HBM_GBS * 1e9) > flop / (peak * 1e12):
        ach = byts / kernel_s_per_launch / 1e9
        return {"bound": "hbm", "achieved": round(ach, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": traffic,
                "step_frac": round(byts / step_s / 1e9 / PEAK_HBM_GBS, 4)}
    ach = flop / kernel_s_per_launch / 1e12
    return {"bound": "mfma", "achieved": round(ach, 2), "peak": peak, "unit": "TFLOP/s",
            "frac": round(ach / peak, 4), "traffic": traffic,
            "step_frac": round(flop / step_s / 1e12 / peak, 4)}


def flat_bench(cfg, nq_override, storage_name, steps, warmup, cpu=True, host_api=True, data=None,
               cpu_threads=None, cpu_seconds=12.0):
    """One flat-search workload: K timed searches (device pointers, inputs in
    HBM, no instrumentation), then K profiled ones for the kernel means.
    Returns the bench fields of that workload (headline format)."""
    import numpy as np
    import hipmem
    import mflat

    mflat.load()
    name, metric, k = WORKLOADS[cfg]
    t0 = time.perf_counter()
    x, q = data if data is not None else make_data(cfg, nq_override)
    if nq_override and cfg != "C4":
        q = q[:nq_override]
    elif cfg == "C4" and nq_override:
        q = q[:nq_override]
    nb, d = x.shape
    nq = q.shape[0]
    log(f"[bench] {cfg}: nb={nb} d={d} nq={nq} k={k} storage={storage_name} data in {time.perf_counter() - t0:.1f}s")

    storage = mflat.STORAGE_NAMES[storage_name]
    esize = 4 if storage == mflat.MFLAT_STORAGE_F32 else 2
    idx = mflat.FlatIndex(d, metric, storage)
    if not idx.ready():
        raise SystemExit("no usable gfx950 device")
    try:
        t0 = time.perf_counter()
        idx.add(x)
        log(f"[bench] add {time.perf_counter() - t0:.2f}s")
        qd = hipmem.DeviceArray.from_numpy(q)
        ids = hipmem.DeviceArray((nq, k), np.int32)
        dist = hipmem.DeviceArray((nq, k), np.float32)

        for i in range(warmup):
            idx.search_device(qd, k, ids, dist)
        hipmem.synchronize()

        # The timed region: K searches, nothing else (no instrumentation).
        t0 = time.perf_counter()
        for i in range(steps):
            idx.search_device(qd, k, ids, dist)
        hipmem.synchronize()
        elapsed = time.perf_counter() - t0
        log(f"[bench] {steps} steps in {elapsed:.3f}s")
        # Kernel durations from a separate pass of the same searches with the
        # library's kernel timer on (HIP events around each launch on its stream).
        mflat.profile_reset()
        mflat.profile_enable(True)
        for i in range(steps):
            idx.search_device(qd, k, ids, dist)
        hipmem.synchronize()
        mflat.profile_enable(False)

        kern = {}
        for fam in ("scan_filter", "scan_sample", "scan_retry", "select", "argmin", "norms", "prep"):
            ms, n = mflat.profile_read(fam)
            if n:
                kern[fam] = {"total_ms": round(ms, 4), "launches": n, "mean_ms": round(ms / n, 4)}

        gpu_ids = ids.numpy()
        ms_per_step = elapsed * 1000.0 / steps
        flop = 2.0 * nq * nb * d
        dominant = "scan_filter" if "scan_filter" in kern else "argmin"
        # algorithmic work of a search over the dominant kernel's time per search
        # (a search may be several launches when its batch exceeds the candidate
        # workspace, e.g. C5)
        scan_s = kern[dominant]["total_ms"] / 1000.0 / steps
        # database in its storage type + queries + ids and values out
        byts = nb * d * esize + nq * d * esize + nq * k * 8
        roof = roofline_of(flop, byts, esize, scan_s, elapsed / steps,
                           MEASURED_TRAFFIC_BYTES.get((cfg, nq, storage_name)))
        out = {
            "metric": "QPS + % of MFMA/HBM roofline, flat L2 d=128 nb=1M k=100 (1 GPU)",
            "value": round(nq * steps / elapsed, 2),
            "unit": "queries/s",
            "n_gpus": 1,
            "steps": steps,
            "warmup": warmup,
            "ms_per_step": round(ms_per_step, 4),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": {"f32": "fp32", "f16": "fp16 storage, fp32 accumulate",
                      "bf16": "bf16 storage, fp32 accumulate"}[storage_name],
            "data": "synthetic",
            "config": {"workload": name.replace("{nq}", str(nq)), "nb": nb, "d": d, "nq": nq, "k": k,
                       "metric": "L2" if metric == 0 else "IP", "storage": storage_name,
                       "parallelism": "single GPU"},
            "roofline": roof,
            "kernels": kern,
        }
        if host_api:
            # The reference's own host-pointer entry point on the same batch,
            # called as a foreign binding calls it (caller-owned output buffers,
            # allocated once): includes the H2D copy of the queries and the D2H
            # copy of ids and values (PCIe), not the Python wrapper's per-call
            # output allocation and copies.
            import ctypes
            lib = mflat.load()
            qh = np.ascontiguousarray(q, dtype=np.float32)
            ids_h = np.zeros((nq, k), dtype=np.int32)
            dist_h = np.zeros((nq, k), dtype=np.float32)
            used = ctypes.c_int(-1)

            def host_call():
                st = lib.mflat_flat_search(idx._h, qh.ctypes.data, nq, k, ids_h.ctypes.data, dist_h.ctypes.data,
                                           ctypes.byref(used))
                if st != mflat.MFLAT_OK:
                    raise RuntimeError(f"mflat_flat_search status {st}")

            host_call()   # first call sizes the host-entry staging buffers
            t0 = time.perf_counter()
            for _ in range(3):
                host_call()
            host_ms = (time.perf_counter() - t0) * 1000.0 / 3
            out["host_api"] = {"entry": "mflat_flat_search (host buffers, PCIe copies included)",
                               "ms_per_step": round(host_ms, 4), "queries_per_s": round(nq * 1000.0 / host_ms, 2)}
            log(f"[bench] host entry {host_ms:.3f} ms/step")
    finally:
        idx.close()
    if cpu:
        nt = host_threads()
        if cpu_threads is None:
            log("[bench] cpu baseline (1 core) ...")
            out["cpu_baseline"] = cpu_baseline(x, q, k, metric, gpu_ids, storage, seconds_target=cpu_seconds)
            log(f"[bench] cpu baseline ({nt} threads) ...")
            out["cpu_baseline_all_cores"] = cpu_baseline(x, q, k, metric, gpu_ids, storage, threads=nt,
                                                         seconds_target=cpu_seconds)
        else:
            out["cpu_baseline"] = cpu_baseline(x, q, k, metric, gpu_ids, storage, threads=min(cpu_threads, nt),
                                               seconds_target=cpu_seconds)
        log("[bench] cpu baseline done")
    return out


# The other BASELINE.json configurations, measured in the default run beside the
# C2 headline: (key, config, query count, storage). C4 is measured at each of
# its batch sizes, with fp32 and fp16 storage; C2 and C3 also with 16-bit
# storage (their reduced-precision kernels: scan_resident, scan_wide).
EXTRA_CONFIGS = [
    ("C1", "C1", 0, "f32"),
    ("C2_f16", "C2", 0, "f16"),
    ("C2_bf16", "C2", 0, "bf16"),
    ("C3", "C3", 0, "f32"),
    ("C3_bf16", "C3", 0, "bf16"),
    ("C4_nq1", "C4", 1, "f32"),
    ("C4_nq16", "C4", 16, "f32"),
    ("C4_nq64", "C4", 64, "f32"),
    ("C4_nq1_f16", "C4", 1, "f16"),
    ("C4_nq16_f16", "C4", 16, "f16"),
    ("C4_nq64_f16", "C4", 64, "f16"),
    ("C5", "C5", 0, "f32"),
]


def extra_configs(args):
    """Each extra configuration: ms per search, the dominant kernel, its
    roofline (kernel and whole-search fractions) and a CPU baseline (the
    oracle on the host threads, ~3 s of work); a failure is recorded in its
    entry and does not drop the others or the headline."""
    out = {}
    cache = {}
    # steps per workload: about 0.1 s or more of timed searches (C1, C4 run
    # 0.3-1.3 ms a search; C2 at 16-bit storage ~3.4 ms; C3 ~20-120 ms; C5 ~250 ms)
    steps_of = {"C1": 200, "C2": 40, "C3": 5, "C4": 200, "C5": 5}
    for key, cfg, nq, storage in EXTRA_CONFIGS:
        steps = steps_of[cfg]
        try:
            if cfg not in cache:
                cache.clear()
                cache[cfg] = make_data(cfg, 64 if cfg == "C4" else 0)
            r = flat_bench(cfg, nq, storage, steps, max(1, args.warmup), cpu=not args.no_cpu_baseline,
                           host_api=False, data=cache[cfg], cpu_threads=host_threads(), cpu_seconds=3.0)
            ent = {k: r[k] for k in ("value", "unit", "ms_per_step", "steps", "dtype", "config", "roofline")}
            dom = "scan_filter" if "scan_filter" in r["kernels"] else "argmin"
            ent["dominant_kernel"] = {"family": dom, "mean_ms": r["kernels"][dom]["mean_ms"]}
            ent["kernels"] = r["kernels"]
            if "cpu_baseline" in r:
                ent["cpu_baseline"] = r["cpu_baseline"]
            out[key] = ent
        except Exception as e:   # noqa: BLE001 -- recorded, the others go on
            out[key] = {"error": f"{type(e).__name__}: {e}"}
            log(f"[bench] extra {key} failed: {e}")
    cache.clear()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="C2", choices=sorted(WORKLOADS))
    ap.add_argument("--nq", type=int, default=0, help="query count override (C4: 1, 16 or 64)")
    ap.add_argument("--storage", default="f32", choices=["f32", "f16", "bf16"],
                    help="element type of the stored database and the queries")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="default run: skip the extra_configs (C1, C2 fp16/bf16, C3 fp32/bf16, "
                         "C4 nq 1/16/64 fp32 and fp16, C5)")
    ap.add_argument("--kmeans", type=int, default=0, metavar="ITERS",
                    help="time the device k-means loop (mflat_kmeans_train) on C5's points and centroid "
                         "count instead: one JSON line with ms per training iteration")
    ap.add_argument("--ivf", action="store_true",
                    help="time IVF search (mflat_ivf_*) on C2's database and queries instead")
    ap.add_argument("--ivfpq", action="store_true",
                    help="time IVF-PQ search (mflat_ivfpq_*) on C2's database and queries instead")
    ap.add_argument("--rerank", type=int, default=-1, help="--ivfpq: rerank shortlist (default 16 k)")
    ap.add_argument("--nlist", type=int, default=0, help="--ivf: cells (default max(64, sqrt(nb)))")
    ap.add_argument("--nprobe", type=int, default=0, help="--ivf: probed cells (default nlist / 16)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 3 device-to-device copies of MIB MiB (counter calibration)")
    args = ap.parse_args()

    if args.copy_probe:
        import hipmem

        n = args.copy_probe << 20
        src = hipmem.DeviceArray((n,), "uint8")
        dst = hipmem.DeviceArray((n,), "uint8")
        src.fill_bytes(1)
        for _ in range(3):
            hipmem.check(hipmem.hip().hipMemcpy(dst.ptr, src.ptr, n, hipmem.D2D), "hipMemcpy D2D")
        hipmem.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "copies": 3}), flush=True)
        return

    if args.kmeans:
        kmeans_bench(args.kmeans)
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the database would shard by rows with an all-gather merge of per-GPU top-k; "
              "not built). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.ivf:
        ivf_bench(args)
        return
    if args.ivfpq:
        ivfpq_bench(args)
        return

    out = flat_bench(args.config, args.nq, args.storage, args.steps, args.warmup,
                     cpu=not args.no_cpu_baseline, host_api=True)
    if args.config == "C2" and not args.nq and args.storage == "f32" and not args.no_extra:
        out["extra_configs"] = extra_configs(args)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
