# SPDX-License-Identifier: Apache-2.0
"""The wide-tile fp16/bf16 scan (scan_wide_kernel: 256 rows x 256 queries a
workgroup), which batches of more than 128 queries take when the storage is
fp16 / bf16 and d is beyond scan_resident's LDS (dpad > 256), through the C ABI.

It computes the same keys as the 128-query tiled kernel (scan_filter) -- the
same MFMA sequence per (query, row) pair -- so on float data its results equal
that kernel's bit for bit (MFLAT_WIDE=0, read when an index is created, runs
the tiled kernel instead); on integer-valued data (exact in fp16 / bf16 and in
every fp32 sum) they equal the oracle's. Shapes: 256-query blocks with a
partial last block, a split whose last 256-row step has only one 128-row tile,
dpad = 64 c + 32 (the half chunk), L2 / IP / Cosine, and a distance-sorted
database whose regions overflow (the retry window on the wide tile)."""
import numpy as np
import pytest

import datagen
import mflat
import oracle
import parity
from conftest import oracle_threads

pytestmark = pytest.mark.gpu

L2, IP, COS = mflat.MFLAT_METRIC_L2, mflat.MFLAT_METRIC_INNER_PRODUCT, mflat.MFLAT_METRIC_COSINE
F16, BF16 = mflat.MFLAT_STORAGE_F16, mflat.MFLAT_STORAGE_BF16


def run(x, q, k, metric, storage, monkeypatch, wide):
    monkeypatch.setenv("MFLAT_WIDE", "1" if wide else "0")
    with mflat.FlatIndex(x.shape[1], metric, storage) as idx:
        idx.add(x)
        gi, gd, ku = idx.search(q, k)
    assert ku == k
    return gi, gd


@pytest.mark.parametrize("storage", [F16, BF16])
@pytest.mark.parametrize("nb,nq,k,d,metric", [(60_000, 300, 10, 300, L2), (33_333, 257, 100, 288, IP),
                                               (20_000, 129, 7, 544, L2)])
def test_integer_exact(gpu_ok, monkeypatch, storage, nb, nq, k, d, metric):
    rng = np.random.default_rng(nb + d + nq)
    x = rng.integers(-15, 16, size=(nb, d)).astype(np.float32)
    q = rng.integers(-15, 16, size=(nq, d)).astype(np.float32)
    print(f"[wide] integer storage={storage} nb={nb} nq={nq} k={k} d={d} metric={metric}", flush=True)
    gi, gd = run(x, q, k, metric, storage, monkeypatch, True)
    oi, od = oracle.flat_search(x, q, k, metric=metric, threads=oracle_threads())
    parity.exact(gi, gd, oi, od)


@pytest.mark.parametrize("storage,metric", [(BF16, IP), (F16, L2), (BF16, COS)])
def test_float_equals_tiled_kernel(gpu_ok, monkeypatch, storage, metric):
    """Float data: the wide and the 128-query tiled kernel agree bit for bit;
    both within the fp32 tolerances of the oracle on the rounded inputs."""
    x, q = datagen.gmm(nb=80_000, nq=400, d=320, seed=81)
    print(f"[wide] float storage={storage} metric={metric}", flush=True)
    wi, wd = run(x, q, 50, metric, storage, monkeypatch, True)
    ti, td = run(x, q, 50, metric, storage, monkeypatch, False)
    assert np.array_equal(wi, ti)
    assert np.array_equal(wd, td)
    xs, qs, m = oracle.storage_inputs(x, q, metric, storage)
    oi, od = oracle.flat_search(xs, qs, 50, metric=m, threads=oracle_threads())
    parity.tolerant(wi, wd, oi, od, xs, qs, 0 if metric == L2 else 1)


def test_distance_sorted_retries(gpu_ok, monkeypatch):
    """Row order follows distance: whole splits overflow and the device-built
    retry window reruns on the wide tile (exact integer data, bf16)."""
    rng = np.random.default_rng(83)
    nb, d = 400_000, 288
    x = rng.integers(0, 4, size=(nb, d)).astype(np.float32)
    x[:, 0] = (np.arange(nb) // 300).astype(np.float32)
    q = rng.integers(0, 4, size=(300, d)).astype(np.float32)
    q[:, 0] = 0.0
    print("[wide] distance-sorted retries", flush=True)
    gi, gd = run(x, q, 20, L2, BF16, monkeypatch, True)
    xs, qs, _ = oracle.storage_inputs(x, q, L2, BF16)   # row // 300 above 256 rounds in bf16
    oi, od = oracle.flat_search(xs, qs, 20, threads=oracle_threads())
    parity.exact(gi, gd, oi, od)
