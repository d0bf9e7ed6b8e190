# SPDX-License-Identifier: Apache-2.0
"""GPU parity of the IVF-PQ index (mflat_ivfpq_*) against the oracle
restatement of the reference's residual-ADC search and rerank
(oracle.ivfpq_search / pq_rerank: src/IvfPqIndex.mm:383-445, :598-625).

The ADC tables, the coarse term and the exact rerank distances are computed on
the device as the reference's scalar fp32 loops (ascending sums, no fused
multiply-add), so on the GPU's own coarse layer, codebook, codes and probes the
results must match the oracle bit for bit on any data -- ids and distances,
including the scan-order tie rule. The codebook is checked against the library's
k-means on the residual sub-spaces (whose own parity is in
test_gpu_kmeans.py), the codes against its final assignments."""
import numpy as np
import pytest

import datagen
import mflat
import oracle
import parity
from conftest import oracle_threads

pytestmark = pytest.mark.gpu

L2, COS = mflat.MFLAT_METRIC_L2, mflat.MFLAT_METRIC_COSINE


def build(x, nlist, M, metric=L2, rerank=False):
    idx = mflat.IvfPqIndex(x.shape[1], metric, nlist, M, rerank)
    idx.build(x)
    assert idx.ready() and idx.size() == x.shape[0]
    return idx


def oracle_search(idx, q, k, nprobe, metric):
    cent, start, rid, pqc, codes = idx.coarse()
    probed = idx.probe(q, nprobe)
    return oracle.ivfpq_search(cent, start, rid, codes, pqc, q, k, probed, metric, threads=oracle_threads())


def check(idx, q, k, nprobe, metric):
    print(f"[ivfpq] m={q.shape[0]} k={k} nprobe={nprobe} metric={metric} M={idx.m_sub}", flush=True)
    gi, gv, ku = idx.search(q, k, nprobe)
    assert ku == min(k, mflat.load().mflat_max_k())
    oi, ov = oracle_search(idx, q, ku, nprobe, metric)
    parity.exact(gi, gv, oi, ov)
    return gi, gv


@pytest.mark.parametrize("metric", [L2, COS])
@pytest.mark.parametrize("k,nprobe", [(1, 4), (10, 8), (100, 16)])
def test_adc_bit_exact(gpu_ok, metric, k, nprobe):
    x, q = datagen.gmm(nb=50_000, nq=700, d=64, ncenters=128, seed=31)
    with build(x, 64, 8, metric) as idx:
        check(idx, q, k, nprobe, metric)


def test_codebook_is_residual_kmeans(gpu_ok):
    x, _ = datagen.gmm(nb=20_000, nq=1, d=32, ncenters=64, seed=32)
    M = 4
    with build(x, 24, M) as idx:
        cent, start, rid, pqc, codes = idx.coarse()
    assign = np.empty(x.shape[0], np.int64)
    for c in range(24):
        assign[rid[start[c]:start[c + 1]]] = c
    r = (x - cent[assign]).astype(np.float32)
    dsub = 32 // M
    for mm in range(M):
        kc, ka, _, _ = mflat.kmeans_train(np.ascontiguousarray(r[:, mm * dsub:(mm + 1) * dsub]), 256, 12, 0)
        assert np.array_equal(kc, pqc[mm])
        assert np.array_equal(ka[rid], codes[:, mm])


@pytest.mark.parametrize("metric", [L2, COS])
def test_rerank_bit_exact(gpu_ok, metric):
    x, q = datagen.gmm(nb=40_000, nq=500, d=64, ncenters=64, seed=33)
    with build(x, 48, 16, metric, rerank=True) as idx:
        short, _, _ = idx.search(q, 300, 12)
        gi, gv, ku = idx.search(q, 20, 12, rerank=300)
        assert ku == 20
    oi, ov = oracle.pq_rerank(x, q, short, 20, metric)
    parity.exact(gi, gv, oi, ov)


def test_rerank_recall(gpu_ok):
    x, q = datagen.gmm(nb=60_000, nq=400, d=128, ncenters=128, seed=34)
    with build(x, 64, 16, L2, rerank=True) as idx:
        gi, _, _ = idx.search(q, 10, 16, rerank=400)
    fi, _ = oracle.flat_search(x, q, 10, 0, threads=oracle_threads())
    recall = np.mean([len(set(gi[r]) & set(fi[r])) / 10 for r in range(q.shape[0])])
    print(f"[ivfpq] recall@10 with rerank 400: {recall:.4f}", flush=True)
    assert recall >= 0.95


def test_rerank_off_without_stored_rows(gpu_ok):
    x, q = datagen.gmm(nb=10_000, nq=100, d=32, ncenters=32, seed=35)
    with build(x, 16, 4) as idx:
        a = idx.search(q, 10, 4)
        b = idx.search(q, 10, 4, rerank=200)
        parity.exact(a[0], a[1], b[0], b[1])


@pytest.mark.parametrize("d,M", [(12, 3), (24, 6), (96, 32), (64, 64), (16, 1), (16, 2), (128, 128), (40, 20)])
def test_subquantizer_counts(gpu_ok, d, M):
    x, q = datagen.gmm(nb=8_000, nq=200, d=d, ncenters=32, seed=36 + M)
    with build(x, 16, M) as idx:
        check(idx, q, 15, 5, L2)


def test_fewer_rows_than_subcentroids(gpu_ok):
    x, q = datagen.gmm(nb=150, nq=20, d=16, ncenters=8, seed=37)
    with build(x, 4, 4) as idx:
        cent, start, rid, pqc, codes = idx.coarse()
        assert pqc.shape == (4, 256, 4)
        check(idx, q, 10, 2, L2)
        check(idx, q, 200, 4, L2)   # k beyond the union: padding


def test_retries_exact_with_tiny_regions(gpu_ok, monkeypatch):
    x, q = datagen.gmm(nb=30_000, nq=300, d=64, ncenters=64, seed=38)
    with build(x, 32, 8) as idx:
        ref = idx.search(q, 50, 8)
    monkeypatch.setenv("MFLAT_IVF_CAP_B", "3")   # read when the index is created
    with build(x, 32, 8) as idx:
        got = idx.search(q, 50, 8)
        parity.exact(got[0], got[1], ref[0], ref[1])
        check(idx, q, 50, 8, L2)
    monkeypatch.delenv("MFLAT_IVF_CAP_B")


def test_device_entry_point_matches_host(gpu_ok):
    import hipmem

    x, q = datagen.gmm(nb=20_000, nq=256, d=64, ncenters=64, seed=39)
    with build(x, 32, 8, L2, rerank=True) as idx:
        for rr in (0, 100):
            hi, hv, _ = idx.search(q, 10, 6, rerank=rr)
            dq = hipmem.DeviceArray.from_numpy(q)
            di = hipmem.DeviceArray((256, 10), np.int32)
            dv = hipmem.DeviceArray((256, 10), np.float32)
            assert idx.search_device(dq, 10, 6, di, dv, rerank=rr) == 10
            parity.exact(di.numpy(), dv.numpy(), hi, hv)


def test_single_probe_and_all_cells(gpu_ok):
    x, q = datagen.gmm(nb=12_000, nq=150, d=32, ncenters=32, seed=41)
    with build(x, 24, 8) as idx:
        check(idx, q, 20, 1, L2)    # nearest cell only
        check(idx, q, 20, 24, L2)   # every cell
        check(idx, q, 20, 500, L2)  # nprobe clamped to nlist


def test_cosine_zero_rows_and_queries(gpu_ok):
    x, q = datagen.gmm(nb=6_000, nq=100, d=32, ncenters=16, seed=42)
    x[::97] = 0.0   # zero rows stay zero under normalisation
    q[::13] = 0.0
    with build(x, 12, 8, COS, rerank=True) as idx:
        check(idx, q, 15, 4, COS)
        short, _, _ = idx.search(q, 60, 4)
        gi, gv, _ = idx.search(q, 15, 4, rerank=60)
    oi, ov = oracle.pq_rerank(x, q, short, 15, COS)
    parity.exact(gi, gv, oi, ov)


@pytest.mark.parametrize("d,M", [(768, 16), (768, 48), (384, 96)])
def test_large_dims(gpu_ok, d, M):
    """Sub-spaces wider than the lookup-table kernel's 32 columns (768 / 16 = 48)
    take its generic path; d = 768 rows also go through the exact rerank."""
    x, q = datagen.unit_normal(nb=6_000, nq=80, d=d, seed=60 + M)
    with build(x, 12, M, L2, rerank=True) as idx:
        check(idx, q, 10, 3, L2)
        short, _, _ = idx.search(q, 50, 3)
        gi, gv, _ = idx.search(q, 10, 3, rerank=50)
    oi, ov = oracle.pq_rerank(x, q, short, 10, L2)
    parity.exact(gi, gv, oi, ov)
