# SPDX-License-Identifier: Apache-2.0
"""GPU parity at the exact sizes of BASELINE.json's configurations.

Each configuration is built at its full size and searched whole through the C
ABI (the plan -- split counts, candidate budgets, sample levels, batching -- is
the one the benchmark runs); a fixed strided subset of its queries is compared
with the oracle (the reference CPU path restated, src/FlatIndex.mm:259-290) on
up to 16 host threads. Ids must match except near-ties within 1e-5 relative of
the k-th value, distances within 1e-4 relative (tests/parity.py); every test
prints how many near-tie swaps it saw, which is what explains an id agreement
below 1.0 in a benchmark's CPU-baseline sample.
"""
import time

import numpy as np
import pytest

import datagen
import mflat
import oracle
import parity
from conftest import oracle_threads

pytestmark = pytest.mark.gpu

L2, IP = mflat.MFLAT_METRIC_L2, mflat.MFLAT_METRIC_INNER_PRODUCT


def say(msg):
    print(f"[fullsize] {msg}", flush=True)


def gpu_search(x, q, k, metric, storage=mflat.MFLAT_STORAGE_F32):
    with mflat.FlatIndex(x.shape[1], metric, storage) as idx:
        assert idx.ready()
        idx.add(x)
        gi, gd, ku = idx.search(q, k)
    assert ku == k
    return gi, gd


def compare(tag, gi, gd, x, q, sub, k, metric):
    t0 = time.perf_counter()
    oi, od = oracle.flat_search(x, q[sub], k, metric=metric, threads=oracle_threads())
    t1 = time.perf_counter()
    parity.sorted_lex(gi[sub], gd[sub], 0 if metric == L2 else 1)
    swaps = parity.tolerant(gi[sub], gd[sub], oi, od, x, q[sub], 0 if metric == L2 else 1)
    agree = float(np.mean([len(set(gi[s].tolist()) & set(oi[r].tolist())) / k for r, s in enumerate(sub)]))
    say(f"{tag}: {len(sub)} queries vs oracle ({t1 - t0:.1f} s on {oracle_threads()} threads): "
        f"id agreement {agree:.6f}, near-tie swaps {swaps} (all within the 1e-5 gap)")


def test_c2_full(gpu_ok):
    """C2: 1M x 128 GMM, L2, all 10,000 queries searched, every 5th (2,000) checked."""
    x, q = datagen.gmm()
    say(f"C2 data {x.shape} / {q.shape}")
    gi, gd = gpu_search(x, q, 100, L2)
    compare("C2", gi, gd, x, q, np.arange(0, q.shape[0], 5), 100, L2)


def test_c3_full(gpu_ok):
    """C3: 1M x 768 unit N(0, I), inner product, all 10,000 queries searched,
    every 31st (323) checked."""
    x, q = datagen.unit_normal()
    say(f"C3 data {x.shape} / {q.shape}")
    gi, gd = gpu_search(x, q, 100, IP)
    compare("C3", gi, gd, x, q, np.arange(0, q.shape[0], 31), 100, IP)


def test_c2_full_fp16(gpu_ok):
    """C2 with fp16 storage: the second sample level, the full pass and the
    retry round with the second sample's looser rank (about 90 queries rerun);
    every 20th query (500) checked against the oracle on the rounded inputs."""
    x, q = datagen.gmm()
    gi, gd = gpu_search(x, q, 100, L2, mflat.MFLAT_STORAGE_F16)
    xs, qs, m = oracle.storage_inputs(x, q, L2, mflat.MFLAT_STORAGE_F16)
    del x, q
    compare("C2 fp16", gi, gd, xs, qs, np.arange(0, qs.shape[0], 20), 100, m)


def test_c3_full_bf16(gpu_ok):
    """C3 with bf16 storage: the wide-tile kernel (sample and full passes) and
    the retry window on the 128-query tiled kernel; every 50th query (200)
    checked against the oracle on the rounded inputs."""
    x, q = datagen.unit_normal()
    gi, gd = gpu_search(x, q, 100, IP, mflat.MFLAT_STORAGE_BF16)
    xs, qs, m = oracle.storage_inputs(x, q, IP, mflat.MFLAT_STORAGE_BF16)
    del x, q
    compare("C3 bf16", gi, gd, xs, qs, np.arange(0, qs.shape[0], 50), 100, m)


@pytest.fixture(scope="module")
def c4_data():
    t0 = time.perf_counter()
    x, q = datagen.uniform_pm1()
    say(f"C4 data {x.shape} in {time.perf_counter() - t0:.1f} s")
    return x, q


def test_c4_full_fp32(gpu_ok, c4_data):
    """C4: 10M x 96 uniform [-1, 1], L2, k = 10, batches of 1, 16 and 64 queries
    (each a separate search, as the benchmark runs them), every query checked."""
    x, q = c4_data
    with mflat.FlatIndex(x.shape[1], L2) as idx:
        idx.add(x)
        for nq in (1, 16, 64):
            gi, gd, ku = idx.search(q[:nq], 10)
            assert ku == 10
            compare(f"C4 fp32 nq={nq}", gi, gd, x, q[:nq], np.arange(nq), 10, L2)


def test_c4_full_fp16(gpu_ok, c4_data):
    """C4 with the database stored as fp16 (fp32 accumulation): the oracle runs
    on the identically rounded rows and queries; every query checked."""
    x, q = c4_data
    with mflat.FlatIndex(x.shape[1], L2, mflat.MFLAT_STORAGE_F16) as idx:
        idx.add(x)
        results = {nq: idx.search(q[:nq], 10) for nq in (1, 16, 64)}
    xs, qs, m = oracle.storage_inputs(x, q, L2, mflat.MFLAT_STORAGE_F16)
    for nq, (gi, gd, ku) in results.items():
        assert ku == 10
        compare(f"C4 fp16 nq={nq}", gi, gd, xs, qs[:nq], np.arange(nq), 10, m)


def test_c5_full(gpu_ok):
    """C5: nearest of 65,536 centroids (sampled from the points) for all
    2,000,000 points (the fused k = 1 pass), every 100th point (20,000) checked.
    Points that are themselves centroids match at distance ~0 (the L2 floor)."""
    cents, pts = datagen.kmeans_assign()
    say(f"C5 data points {pts.shape}, centroids {cents.shape}")
    gi, gd = gpu_search(cents, pts, 1, L2)
    compare("C5", gi, gd, cents, pts, np.arange(0, pts.shape[0], 100), 1, L2)
