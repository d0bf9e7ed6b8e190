# SPDX-License-Identifier: Apache-2.0
"""GPU parity of the reduced-precision storage variants (fp16 / bf16 database
and queries, fp32 accumulation on the fp16 / bf16 matrix cores) through the C
ABI (mflat_flat_create_ex).

The reference has no reduced-precision flat path; the oracle is the reference
CPU algorithm run on identically rounded inputs (oracle.storage_inputs). On
integer-valued data the rounding is exact, so results must match the fp32
oracle bit for bit; on floating-point data the tolerance is the fp32 one
(parity.REL_DIST_FP32 = 1e-4, near-ties 1e-5), tighter than the 1e-2 the
build target allows for fp16 / bf16 inputs, since both sides see the same
rounded values.

Shapes cover both scan kernels (batches <= 64 stream the database, larger ones
use the LDS-tiled kernel), dpad = 64 c + 32 (the tiled kernel's half chunk),
the k = 1 assignment kernel, and the sample / retry levels (nb > 2 R0)."""
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


def run(x, q, k, metric, storage):
    with mflat.FlatIndex(x.shape[1], metric, storage) as idx:
        assert idx.ready()
        assert mflat.load().mflat_flat_storage(idx.handle) == storage
        idx.add(x)
        return idx.search(q, k)


def orc(x, q, k, metric, storage):
    xs, qs, m = oracle.storage_inputs(x, q, metric, storage)
    oi, od = oracle.flat_search(xs, qs, k, metric=m, threads=oracle_threads())
    return oi, od, xs, qs, m


@pytest.mark.parametrize("storage", [F16, BF16])
@pytest.mark.parametrize("nb,nq,k,d", [(20_000, 300, 10, 128), (20_000, 16, 10, 96), (9_000, 130, 100, 96),
                                       (50_000, 257, 1, 128), (5_000, 70, 5, 33)])
def test_integer_exact(gpu_ok, storage, nb, nq, k, d):
    rng = np.random.default_rng(nb + d)
    x = rng.integers(0, 256, size=(nb, d)).astype(np.float32)
    q = rng.integers(0, 256, size=(nq, d)).astype(np.float32)
    print(f"[storage] integer storage={storage} nb={nb} nq={nq} k={k} d={d}", flush=True)
    gi, gd, ku = run(x, q, k, L2, storage)
    assert ku == k
    oi, od = oracle.flat_search(x, q, k, metric=0, threads=oracle_threads())
    parity.exact(gi, gd, oi, od)


@pytest.mark.parametrize("storage", [F16, BF16])
def test_gmm_l2_large_batch(gpu_ok, storage):
    x, q = datagen.gmm(nb=120_000, nq=300, seed=1)
    print(f"[storage] gmm storage={storage}", flush=True)
    gi, gd, _ = run(x, q, 100, L2, storage)
    oi, od, xs, qs, m = orc(x, q, 100, L2, storage)
    parity.sorted_lex(gi, gd, 0)
    parity.tolerant(gi, gd, oi, od, xs, qs, m)


@pytest.mark.parametrize("storage", [F16, BF16])
def test_uniform_small_batch_d96(gpu_ok, storage):
    """Reduced C4 with fp16 / bf16 storage: uniform [-1, 1], d = 96, nq in {1, 16, 64}."""
    x, q = datagen.uniform_pm1(nb=300_000, nq=64, seed=3)
    q = np.concatenate([q, q[:1] * 0.5])     # 65 queries: the tiled kernel at d = 96
    for nq in (1, 16, 64, 65):
        print(f"[storage] uniform storage={storage} nq={nq}", flush=True)
        gi, gd, _ = run(x, q[:nq], 10, L2, storage)
        oi, od, xs, qs, m = orc(x, q[:nq], 10, L2, storage)
        parity.tolerant(gi, gd, oi, od, xs, qs, m)


@pytest.mark.parametrize("storage", [F16, BF16])
def test_ip_and_cosine(gpu_ok, storage):
    x, q = datagen.unit_normal(nb=30_000, nq=200, d=256, seed=2)
    print(f"[storage] ip storage={storage}", flush=True)
    gi, gd, _ = run(x, q, 50, IP, storage)
    oi, od, xs, qs, m = orc(x, q, 50, IP, storage)
    parity.sorted_lex(gi, gd, 1)
    parity.tolerant(gi, gd, oi, od, xs, qs, m)
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((30_000, 100)) * 3).astype(np.float32)
    x[5] = 0.0
    for nq in (9, 70):
        qc = rng.standard_normal((nq, 100)).astype(np.float32)
        print(f"[storage] cosine storage={storage} nq={nq}", flush=True)
        gi, gd, _ = run(x, qc, 20, COS, storage)
        oi, od, xs, qs, m = orc(x, qc, 20, COS, storage)
        parity.tolerant(gi, gd, oi, od, xs, qs, m)


@pytest.mark.parametrize("storage", [F16, BF16])
def test_kmeans_assign_k1(gpu_ok, storage):
    cents, pts = datagen.kmeans_assign(npts=40_000, ncent=4096, seed=4)
    print(f"[storage] k1 storage={storage}", flush=True)
    gi, gd, _ = run(cents, pts, 1, L2, storage)
    oi, od, xs, qs, m = orc(cents, pts, 1, L2, storage)
    parity.tolerant(gi, gd, oi, od, xs, qs, m)

