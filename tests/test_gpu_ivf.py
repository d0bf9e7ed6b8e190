# SPDX-License-Identifier: Apache-2.0
"""GPU parity of the IVF index (mflat_ivf_*) against the oracle restatement of
the reference's two-stage search (oracle.ivf_search: searchCpu over probed
cells, src/IvfIndex.mm:518-560) and its coarse layer.

The fine scan is checked on the GPU's own coarse layer and probes (the
reference's searchCpu takes the probed cells as an argument, probedRows), so a
near-tie between two centroids cannot change which rows are compared; the probe
is checked separately against the oracle's lexicographic nearest-cell order
(probeCellsCpu) with the north-star tolerances, and the coarse layer against
the library's k-means (whose own parity is in test_gpu_kmeans.py) and the CSR
rule. Integer-valued data makes every score exact in fp32, so ids and
distances must match bit for bit, including the scan-order tie rule; float data
uses the tolerances of parity.tolerant (1e-4 relative for fp32 inputs)."""
import os

import numpy as np
import pytest

import datagen
import mflat
import oracle
import parity
from conftest import oracle_threads

pytestmark = pytest.mark.gpu

L2, IP, COS = mflat.MFLAT_METRIC_L2, mflat.MFLAT_METRIC_INNER_PRODUCT, mflat.MFLAT_METRIC_COSINE


def build(x, nlist, metric=L2, storage=mflat.MFLAT_STORAGE_F32):
    idx = mflat.IvfIndex(x.shape[1], metric, nlist, storage)
    idx.build(x)
    assert idx.ready() and idx.size() == x.shape[0]
    return idx


def oracle_on_gpu_layer(idx, x, q, k, nprobe, metric, storage=mflat.MFLAT_STORAGE_F32):
    """searchCpu on the GPU's coarse layer and probes, inputs rounded as stored."""
    _, start, rid = idx.coarse()
    probed = idx.probe(q, nprobe)
    xs, qs = x, q
    if storage != mflat.MFLAT_STORAGE_F32:
        xs, qs, m2 = oracle.storage_inputs(x, q, metric, storage)
        metric = m2
    oi, ov = oracle.ivf_search(xs, start, rid, qs, k, probed, metric, threads=oracle_threads())
    return oi, ov, xs, qs, metric


def check(idx, x, q, k, nprobe, metric, exact=False, storage=mflat.MFLAT_STORAGE_F32):
    print(f"[ivf] n={x.shape[0]} d={x.shape[1]} m={q.shape[0]} k={k} nprobe={nprobe} metric={metric} "
          f"storage={storage}", flush=True)
    gi, gv, ku = idx.search(q, k, nprobe)
    kk = min(k, mflat.load().mflat_max_k())
    assert ku == kk
    oi, ov, xs, qs, om = oracle_on_gpu_layer(idx, x, q, kk, nprobe, metric, storage)
    if exact:
        parity.exact(gi, gv, oi, ov)
    else:
        if om == COS:
            xs, qs, om = oracle.normalize_rows(xs), oracle.normalize_rows(qs), IP
        parity.tolerant(gi, gv, oi, ov, xs, qs, 0 if om == L2 else 1)
    return gi, gv


def int_case(n, nq, d, hi, seed):
    rng = np.random.default_rng(seed)
    x = rng.integers(0, hi, size=(n, d)).astype(np.float32)
    q = rng.integers(0, hi, size=(nq, d)).astype(np.float32)
    return x, q


def test_coarse_layer_is_the_kmeans_and_csr(gpu_ok):
    x, _ = datagen.gmm(nb=30_000, nq=1, d=64, ncenters=64, seed=11)
    with build(x, 48) as idx:
        cent, start, rid = idx.coarse()
        assert idx.nlist() == 48 and cent.shape == (48, 64)
        kc, ka, ks, ko = mflat.kmeans_train(x, 48, 12, 256)
        assert np.array_equal(cent, kc)
        assert np.array_equal(start, ks) and np.array_equal(rid, ko)
        s2, r2 = oracle.ivf_csr(ka, 48)
        assert np.array_equal(start, s2) and np.array_equal(rid, r2)


def test_probe_is_nearest_cells(gpu_ok):
    x, q = datagen.gmm(nb=40_000, nq=700, d=96, ncenters=128, seed=12)
    with build(x, 100) as idx:
        cent, _, _ = idx.coarse()
        for nprobe in (1, 7, 100):
            gp = idx.probe(q, nprobe)
            op = oracle.ivf_probe(cent, q, nprobe)
            d = np.sum((q[:, None, :].astype(np.float64) - cent[None, :, :]) ** 2, axis=2)
            gd = np.take_along_axis(d, gp, 1).astype(np.float32)
            od = np.take_along_axis(d, op, 1).astype(np.float32)
            parity.tolerant(gp, gd, op, od, cent, q, 0)
        assert np.array_equal(idx.probe(q, 10_000), idx.probe(q, 100))   # clamped to nlist


@pytest.mark.parametrize("metric", [L2, IP])
@pytest.mark.parametrize("nprobe", [1, 3, 16])
def test_exact_integer_data(gpu_ok, metric, nprobe):
    """C1-like integer data: exact scores, exact ties, scan-order tie rule."""
    x, q = int_case(20_000, 300, 32, 6, seed=nprobe + 10 * metric)
    with build(x, 40, metric) as idx:
        check(idx, x, q, 25, nprobe, metric, exact=True)


@pytest.mark.parametrize("metric", [L2, IP, COS])
@pytest.mark.parametrize("k,nprobe", [(1, 4), (10, 8), (100, 24)])
def test_gmm_float(gpu_ok, metric, k, nprobe):
    x, q = datagen.gmm(nb=60_000, nq=1_000, d=128, ncenters=256, seed=13)
    if metric == IP:
        x = x / np.linalg.norm(x, axis=1, keepdims=True).astype(np.float32)
    with build(x, 128, metric) as idx:
        check(idx, x, q, k, nprobe, metric)


def test_all_cells_equal_flat_search(gpu_ok):
    x, q = datagen.gmm(nb=20_000, nq=400, d=64, ncenters=64, seed=14)
    with build(x, 32) as idx:
        gi, gv, _ = idx.search(q, 20, 32)
    fi, fv = oracle.flat_search(x, q, 20, 0, threads=oracle_threads())
    parity.tolerant(gi, gv, fi, fv, x, q, 0)


def test_small_batches_and_ragged_shapes(gpu_ok):
    x, q = datagen.gmm(nb=9_000, nq=300, d=40, ncenters=30, seed=15)   # dpad 64, ragged dim
    with build(x, 20) as idx:
        for m in (1, 2, 63, 129, 300):
            check(idx, x, q[:m], 10, 5, L2)


def test_padding_when_probed_cells_are_small(gpu_ok):
    x, q = int_case(300, 20, 8, 5, seed=16)
    with build(x, 64) as idx:
        gi, gv = check(idx, x, q, 200, 2, L2, exact=True)
        assert np.any(gi == -1)
        assert np.all(np.isinf(gv[gi == -1]))


def test_nlist_clamped_and_tiny_index(gpu_ok):
    x, q = int_case(5, 4, 8, 9, seed=17)
    with build(x, 50) as idx:
        assert idx.nlist() == 5
        check(idx, x, q, 3, 5, L2, exact=True)
        check(idx, x, q, 9, 99, L2, exact=True)   # nprobe clamped to nlist


def test_duplicates_tie_in_scan_order(gpu_ok):
    rng = np.random.default_rng(18)
    base = rng.integers(0, 4, size=(50, 16)).astype(np.float32)
    x = np.repeat(base, 40, axis=0)[rng.permutation(2000)]
    with build(x, 25) as idx:
        check(idx, x, base[:30], 64, 6, L2, exact=True)


def test_retries_exact_with_tiny_regions(gpu_ok, monkeypatch):
    """Regions of 4 entries overflow on most queries; the retries must give the
    same answer as the normal plan (exactness never depends on capacities)."""
    x, q = datagen.gmm(nb=30_000, nq=500, d=64, ncenters=64, seed=19)
    with build(x, 64) as idx:
        gi, gv, _ = idx.search(q, 30, 12)
    # the knob is read when an index is created; the build is deterministic,
    # so the second index holds the same cells
    monkeypatch.setenv("MFLAT_IVF_CAP_B", "4")
    with build(x, 64) as idx:
        ri, rv, _ = idx.search(q, 30, 12)
        parity.exact(ri, rv, gi, gv)
        check(idx, x, q, 30, 12, L2)
    xi, qi = int_case(8_000, 200, 16, 4, seed=20)
    monkeypatch.setenv("MFLAT_IVF_CAP_B", "2")
    with build(xi, 16) as idx:
        check(idx, xi, qi, 40, 1, L2, exact=True)
        check(idx, xi, qi, 40, 5, L2, exact=True)
    monkeypatch.delenv("MFLAT_IVF_CAP_B")


def test_many_cells_radix_path(gpu_ok):
    """More than 32,768 cells: the work tables group entries with the radix
    sort and scans of primitives.hip instead of the per-block LDS histograms
    (and k-means groups its points with the same sort). Integer data: exact."""
    xi, qi = int_case(120_000, 300, 16, 6, seed=27)
    with build(xi, 40_000) as idx:
        assert mflat.load().mflat_ivf_nlist(idx.handle) == 40_000
        check(idx, xi, qi, 10, 64, L2, exact=True)
        check(idx, xi, qi, 50, 300, L2, exact=True)


@pytest.mark.parametrize("storage", [mflat.MFLAT_STORAGE_F16, mflat.MFLAT_STORAGE_BF16])
def test_reduced_precision_storage(gpu_ok, storage):
    x, q = datagen.gmm(nb=40_000, nq=600, d=128, ncenters=128, seed=21)
    with build(x, 64, L2, storage) as idx:
        assert mflat.load().mflat_ivf_storage(idx.handle) == storage
        check(idx, x, q, 10, 8, L2, storage=storage)
    xi, qi = int_case(10_000, 200, 64, 8, seed=22)   # exact in fp16 and bf16
    with build(xi, 32, IP, storage) as idx:
        check(idx, xi, qi, 16, 4, IP, exact=True, storage=storage)


def test_device_entry_point_matches_host(gpu_ok):
    import hipmem

    x, q = datagen.gmm(nb=20_000, nq=256, d=128, ncenters=64, seed=23)
    with build(x, 32) as idx:
        hi, hv, _ = idx.search(q, 10, 6)
        dq = hipmem.DeviceArray.from_numpy(q)
        di = hipmem.DeviceArray((256, 10), np.int32)
        dv = hipmem.DeviceArray((256, 10), np.float32)
        assert idx.search_device(dq, 10, 6, di, dv) == 10
        parity.exact(di.numpy(), dv.numpy(), hi, hv)


def test_rebuild_replaces_index(gpu_ok):
    x1, q = int_case(4_000, 50, 16, 7, seed=24)
    x2, _ = int_case(2_500, 1, 16, 7, seed=25)
    with build(x1, 16) as idx:
        idx.build(x2)
        assert idx.size() == 2_500
        check(idx, x2, q, 12, 4, L2, exact=True)


def test_tile_widths_compute_identical_keys(gpu_ok, monkeypatch):
    """Work items of 128 and of 32 queries run the same per-pair MFMA sequence:
    all-wide, all-narrow and mixed tables give bit-identical results (the bound
    pass and the full pass may use different widths for the same row)."""
    x, q = datagen.gmm(nb=50_000, nq=900, d=128, ncenters=128, seed=26)
    with build(x, 96) as idx:
        ref = idx.search(q, 100, 10)
        check(idx, x, q, 100, 10, L2)
    for tiles in ("128", "32"):
        monkeypatch.setenv("MFLAT_IVF_TILES", tiles)   # read when the index is created
        with build(x, 96) as idx:
            got = idx.search(q, 100, 10)
        parity.exact(got[0], got[1], ref[0], ref[1])
    monkeypatch.delenv("MFLAT_IVF_TILES")


# ---- dims beyond scan_resident's 128-query tile: the LDS-tiled kernel --------

def test_large_dim_integer_exact(gpu_ok):
    x, q = int_case(12_000, 150, 256, 16, seed=51)   # fp32 d = 256: a 128-query tile exceeds LDS
    with build(x, 24) as idx:
        check(idx, x, q, 20, 5, L2, exact=True)
    with build(x, 24, IP) as idx:
        check(idx, x, q, 100, 24, IP, exact=True)


@pytest.mark.parametrize("d,metric", [(768, IP), (300, L2), (1120, COS)])
def test_large_dim_float(gpu_ok, d, metric):
    x, q = datagen.unit_normal(nb=8_000, nq=100, d=d, seed=52 + d)
    with build(x, 16, metric) as idx:
        check(idx, x, q, 10, 4, metric)


@pytest.mark.parametrize("storage", [mflat.MFLAT_STORAGE_F16, mflat.MFLAT_STORAGE_BF16])
def test_large_dim_reduced_storage(gpu_ok, storage):
    x, q = datagen.unit_normal(nb=8_000, nq=100, d=512, seed=53)
    with build(x, 16, L2, storage) as idx:
        check(idx, x, q, 10, 4, L2, storage=storage)


@pytest.mark.parametrize("d", [1152, 2048])
def test_very_large_dim(gpu_ok, d):
    x, q = datagen.unit_normal(nb=3_000, nq=130, d=d, seed=54)
    with build(x, 8) as idx:
        check(idx, x, q, 10, 3, L2)


@pytest.mark.parametrize("d,metric", [(256, L2), (768, IP)])
def test_large_dim_tiles_compute_identical_keys(gpu_ok, monkeypatch, d, metric):
    """Above d = 128 the 128-query items run the LDS-tiled kernel and the
    32-query ones scan_resident, and a search mixes them: their keys must be
    bit-identical on float data. All-wide (tiled only), all-narrow (resident
    only) and the default mix must return the same bits."""
    x, q = datagen.unit_normal(nb=8_000, nq=200, d=d, seed=55 + d)
    with build(x, 16, metric) as idx:
        mixed = idx.search(q, 50, 6)
    out = []
    for tiles in ("128", "32"):
        monkeypatch.setenv("MFLAT_IVF_TILES", tiles)   # read when the index is created
        with build(x, 16, metric) as idx:
            out.append(idx.search(q, 50, 6))
    monkeypatch.delenv("MFLAT_IVF_TILES")
    for o in out:
        parity.exact(mixed[0], mixed[1], o[0], o[1])
