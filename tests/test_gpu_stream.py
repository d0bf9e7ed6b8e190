# SPDX-License-Identifier: Apache-2.0
"""The streaming top-k scan (batches of <= 16 queries, k <= 32; the library
takes it for single queries by default): every split's exact top-k from
per-wave lists, merged by the select -- no sample, no bound, no retry.
Integer-valued data (exact fp32 sums, ties everywhere) is compared with the
oracle bit for bit; float data within the fp32 tolerances."""
import numpy as np
import pytest

import datagen
import mflat
import oracle
import parity
from conftest import oracle_threads

pytestmark = pytest.mark.gpu

L2, IP, COS = mflat.MFLAT_METRIC_L2, mflat.MFLAT_METRIC_INNER_PRODUCT, mflat.MFLAT_METRIC_COSINE


@pytest.fixture(autouse=True)
def stream_every_small_batch(monkeypatch):
    """The library takes this path for single queries by default; these tests
    run it for every batch of up to 16 (read when an index is created)."""
    monkeypatch.setenv("MFLAT_STREAM_MAXQ", "16")


def run(x, q, k, metric, storage=mflat.MFLAT_STORAGE_F32):
    with mflat.FlatIndex(x.shape[1], metric, storage) as idx:
        idx.add(x)
        gi, gd, ku = idx.search(q, k)
    assert ku == k
    return gi, gd


@pytest.mark.parametrize("nq,k", [(1, 1), (1, 10), (3, 32), (16, 17), (16, 32), (9, 5)])
def test_integer_exact(gpu_ok, nq, k):
    rng = np.random.default_rng(100 + nq * 33 + k)
    x = rng.integers(0, 6, size=(200_000, 24)).astype(np.float32)   # exact ties everywhere
    q = rng.integers(0, 6, size=(nq, 24)).astype(np.float32)
    print(f"[stream] int nq={nq} k={k}", flush=True)
    for metric in (L2, IP):
        gi, gd = run(x, q, k, metric)
        oi, od = oracle.flat_search(x, q, k, metric=metric, threads=oracle_threads())
        parity.exact(gi, gd, oi, od)


@pytest.mark.parametrize("d", [1, 33, 96, 128, 300])
def test_dims(gpu_ok, d):
    """Every kernel variant: buffered blocks (d = 96, 128) and the generic one."""
    rng = np.random.default_rng(7 + d)
    x = rng.integers(-9, 9, size=(50_000, d)).astype(np.float32)
    q = rng.integers(-9, 9, size=(7, d)).astype(np.float32)
    gi, gd = run(x, q, 12, L2)
    oi, od = oracle.flat_search(x, q, 12, threads=oracle_threads())
    parity.exact(gi, gd, oi, od)


def test_float_and_cosine(gpu_ok):
    x, q = datagen.gmm(nb=300_000, nq=16, d=128, seed=61)
    gi, gd = run(x, q, 32, L2)
    oi, od = oracle.flat_search(x, q, 32, threads=oracle_threads())
    parity.tolerant(gi, gd, oi, od, x, q, 0)
    gi, gd = run(x, q, 20, COS)
    oi, od = oracle.flat_search(x, q, 20, metric=COS, threads=oracle_threads())
    parity.tolerant(gi, gd, oi, od, oracle.normalize_rows(x), oracle.normalize_rows(q), 1)


@pytest.mark.parametrize("storage", [mflat.MFLAT_STORAGE_F16, mflat.MFLAT_STORAGE_BF16])
def test_reduced_precision(gpu_ok, storage):
    rng = np.random.default_rng(62)
    x = rng.integers(0, 200, size=(120_000, 96)).astype(np.float32)   # exact in fp16 and bf16
    q = rng.integers(0, 200, size=(16, 96)).astype(np.float32)
    gi, gd = run(x, q, 10, L2, storage)
    oi, od = oracle.flat_search(x, q, 10, threads=oracle_threads())
    parity.exact(gi, gd, oi, od)


def test_fewer_rows_than_k_and_bad_rows(gpu_ok):
    """Padding when the database holds fewer than k rows; rows holding NaN or
    +inf never returned; rows past the end of a split's last tile ignored."""
    rng = np.random.default_rng(63)
    x = rng.integers(0, 5, size=(7, 8)).astype(np.float32)
    q = rng.integers(0, 5, size=(4, 8)).astype(np.float32)
    gi, gd = run(x, q, 10, L2)
    oi, od = oracle.flat_search(x, q, 10)
    parity.exact(gi, gd, oi, od)
    assert np.all(gi[:, 7:] == -1) and np.all(gd[:, 7:] == np.inf)
    x = rng.integers(0, 5, size=(5_000, 8)).astype(np.float32)
    x[[3, 999]] = np.nan
    x[[4, 1000], 2] = np.inf
    gi, gd = run(x, q, 20, L2)
    oi, od = oracle.flat_search(x, q, 20)
    parity.exact(gi, gd, oi, od)
    assert not np.isin(gi, [3, 4, 999, 1000]).any()


def test_rank_follows_row_order(gpu_ok):
    """A database whose distance grows with the row index: the first splits
    hold every result, the others none (each split's list is exact on its own)."""
    rng = np.random.default_rng(64)
    nb = 2_000_000
    x = rng.integers(0, 4, size=(nb, 16)).astype(np.float32)
    x[:, 0] = (np.arange(nb) // 700).astype(np.float32)
    q = rng.integers(0, 4, size=(16, 16)).astype(np.float32)
    q[:, 0] = 0.0
    gi, gd = run(x, q, 32, L2)
    oi, od = oracle.flat_search(x, q, 32, threads=oracle_threads())
    parity.exact(gi, gd, oi, od)


@pytest.mark.parametrize("nq,k", [(1, 32), (3, 20)])
def test_merge_many_close_rows(gpu_ok, nq, k):
    """Every split holds fewer than k rows at distance 0 (one every 500 rows)
    and there are thousands of them: the per-split lists' k-th entries bound
    nothing useful, so the merge takes its radix descent to the exact k-th."""
    rng = np.random.default_rng(65 + nq)
    nb = 2_000_000
    q = rng.integers(0, 4, size=(nq, 16)).astype(np.float32)
    x = rng.integers(0, 4, size=(nb, 16)).astype(np.float32)
    for i in range(nq):
        x[i::500] = q[i]   # distance 0 for query i, one row in 500 (by query)
    print(f"[stream] close rows nq={nq} k={k}", flush=True)
    gi, gd = run(x, q, k, L2)
    oi, od = oracle.flat_search(x, q, k, threads=oracle_threads())
    parity.exact(gi, gd, oi, od)
    assert np.all(gd[:, :k] == 0.0)
