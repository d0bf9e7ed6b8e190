# SPDX-License-Identifier: Apache-2.0
"""The allocation-free entry point (mflat_flat_search_device_noalloc) against
the existing device entry point (mflat_flat_search_device) on the same index,
through the C ABI: two calls in a row, the second with a smaller input (fewer
queries, smaller k), so the second reuses the device's scratch array after the
first. Integer-valued data (exact fp32 sums) must match bit for bit -- and the
oracle; float data within the fp32 tolerances of tests/parity.py. Beyond its
limits (16 queries, k 32, dim 2048) the call returns MFLAT_ERR_BAD_ARG."""
import numpy as np
import pytest

import datagen
import hipmem
import mflat
import oracle
import parity
from conftest import oracle_threads

pytestmark = pytest.mark.gpu

L2, IP, COS = mflat.MFLAT_METRIC_L2, mflat.MFLAT_METRIC_INNER_PRODUCT, mflat.MFLAT_METRIC_COSINE


def dev_search(idx, q, k, noalloc, st):
    qd = hipmem.DeviceArray.from_numpy(q)
    ids = hipmem.DeviceArray((q.shape[0], k), np.int32)
    dist = hipmem.DeviceArray((q.shape[0], k), np.float32)
    fn = idx.search_device_noalloc if noalloc else idx.search_device
    ku = fn(qd, k, ids, dist, stream=st)
    st.synchronize()
    return ids.numpy(), dist.numpy(), ku


@pytest.mark.parametrize("nb,d", [(300_000, 96), (2_000_000, 16)])
def test_noalloc_matches_device_entry_integer(gpu_ok, nb, d):
    """d = 16 runs the most streaming workgroups at once: at 16 queries and
    k = 32 their lists would outgrow the scratch, so the split count is capped."""
    rng = np.random.default_rng(71)
    x = rng.integers(0, 8, size=(nb, d)).astype(np.float32)
    q = rng.integers(0, 8, size=(16, d)).astype(np.float32)
    st = hipmem.Stream()
    try:
        with mflat.FlatIndex(d, L2) as idx:
            idx.add(x)
            for m, k in ((16, 32), (3, 7)):   # the second call smaller than the first
                print(f"[noalloc] integer nb={nb} d={d} m={m} k={k}", flush=True)
                ni, nd, nku = dev_search(idx, q[:m], k, True, st)
                di, dd, dku = dev_search(idx, q[:m], k, False, st)
                assert nku == dku == k
                parity.exact(ni, nd, di, dd)
                oi, od = oracle.flat_search(x, q[:m], k, threads=oracle_threads())
                parity.exact(ni, nd, oi, od)
    finally:
        st.destroy()


@pytest.mark.parametrize("metric,storage", [(L2, mflat.MFLAT_STORAGE_F32), (IP, mflat.MFLAT_STORAGE_F32),
                                            (COS, mflat.MFLAT_STORAGE_F32), (L2, mflat.MFLAT_STORAGE_F16)])
def test_noalloc_matches_device_entry_float(gpu_ok, metric, storage):
    x, q = datagen.gmm(nb=200_000, nq=16, d=128, seed=72)
    st = hipmem.Stream()
    try:
        with mflat.FlatIndex(128, metric, storage) as idx:
            idx.add(x)
            xs, qs = x, q
            if storage != mflat.MFLAT_STORAGE_F32:
                xs, qs, _ = oracle.storage_inputs(x, q, metric, storage)
            if metric == COS:
                xs, qs = oracle.normalize_rows(xs), oracle.normalize_rows(qs)
            for m, k in ((16, 20), (5, 4)):
                print(f"[noalloc] float metric={metric} storage={storage} m={m} k={k}", flush=True)
                ni, nd, nku = dev_search(idx, q[:m], k, True, st)
                di, dd, dku = dev_search(idx, q[:m], k, False, st)
                assert nku == dku == k
                parity.tolerant(ni, nd, di, dd, xs, qs[:m], 0 if metric == L2 else 1)
    finally:
        st.destroy()


def test_noalloc_limits_and_empty_index(gpu_ok):
    lib = mflat.load()
    st = hipmem.Stream()
    try:
        with mflat.FlatIndex(8, L2) as idx:
            q = np.ones((17, 8), np.float32)
            gi, gd, ku = dev_search(idx, q[:4], 5, True, st)   # empty index: padding
            assert ku == 5 and np.all(gi == -1) and np.all(gd == np.inf)
            idx.add(np.arange(80, dtype=np.float32).reshape(10, 8))
            with pytest.raises(mflat.MflatError) as e:
                dev_search(idx, q, 5, True, st)             # 17 queries
            assert e.value.status == mflat.MFLAT_ERR_BAD_ARG
            with pytest.raises(mflat.MflatError) as e:
                dev_search(idx, q[:2], 33, True, st)        # k = 33
            assert e.value.status == mflat.MFLAT_ERR_BAD_ARG
            gi, gd, ku = dev_search(idx, q[:2], 12, True, st)   # fewer rows than k: padding
            oi, od = oracle.flat_search(np.arange(80, dtype=np.float32).reshape(10, 8), q[:2], 12)
            parity.exact(gi, gd, oi, od)
        with mflat.FlatIndex(2049, L2) as idx:
            idx.add(np.zeros((3, 2049), np.float32))
            with pytest.raises(mflat.MflatError) as e:
                dev_search(idx, np.zeros((1, 2049), np.float32), 1, True, st)
            assert e.value.status == mflat.MFLAT_ERR_BAD_ARG
        assert lib.mflat_flat_search_device_noalloc(None, None, 1, 1, None, None, None, None) == \
            mflat.MFLAT_ERR_NULL_ARG
    finally:
        st.destroy()
