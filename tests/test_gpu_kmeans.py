# SPDX-License-Identifier: Apache-2.0
"""GPU parity of the device k-means loop (mflat_kmeans_train) against the oracle
restatement of the reference's training loop (oracle.kmeans_train).

Bit-exact cases use points whose every centroid stays a data point or a mean of
identical points (integer coordinates), so assignment distances are exact in
both the GPU's norm identity and the oracle's direct sum, ties resolve to the
lowest centroid in both, and every update is the same sequential double mean.
On general float data the loop is checked through invariants: the returned
assignment is nearest-centroid for the returned centroids (within the fp32
tolerances), the CSR matches it, and every centroid is the mean of the training
points the last iteration assigned to it."""
import numpy as np
import pytest

import datagen
import mflat
import oracle
import parity

pytestmark = pytest.mark.gpu


def exact_case(n_distinct, reps, d, seed):
    rng = np.random.default_rng(seed)
    base = rng.integers(0, 16, size=(n_distinct, d)).astype(np.float32)
    pts = np.repeat(base, reps, axis=0)
    return pts[rng.permutation(pts.shape[0])]


def check_csr(assign, start, order, nlist):
    assert start[0] == 0 and start[-1] == assign.size
    assert np.array_equal(np.diff(start), np.bincount(assign, minlength=nlist))
    assert np.array_equal(order, np.argsort(assign, kind="stable"))


@pytest.mark.parametrize("iters,mpc", [(0, 0), (1, 0), (6, 0), (6, 8)])
def test_exact_loop(gpu_ok, iters, mpc):
    pts = exact_case(40, 50, 24, seed=iters + mpc)     # 2,000 points, 40 locations
    nlist = 32
    print(f"[kmeans] exact iters={iters} mpc={mpc}", flush=True)
    gc, ga, gs, go = mflat.kmeans_train(pts, nlist, iters, mpc)
    oc, oa, os_, oo = oracle.kmeans_train(pts, nlist, iters, mpc)
    assert np.array_equal(gc, oc)
    assert np.array_equal(ga, oa) and np.array_equal(gs, os_) and np.array_equal(go, oo)
    check_csr(ga, gs, go, nlist)


def test_empty_cells_reseeded(gpu_ok):
    """Five distinct locations, 24 cells: most cells empty after the first
    assignment, reseeded from the generator stream every iteration."""
    pts = exact_case(5, 200, 8, seed=3)
    gc, ga, gs, go = mflat.kmeans_train(pts, 24, 4, 0)
    oc, oa, os_, oo = oracle.kmeans_train(pts, 24, 4, 0)
    assert np.array_equal(gc, oc) and np.array_equal(ga, oa) and np.array_equal(go, oo)


def test_nlist_clamped_to_n(gpu_ok):
    pts = exact_case(6, 2, 4, seed=5)
    gc, ga, gs, go = mflat.kmeans_train(pts, 50, 2, 0)
    oc, oa, _, _ = oracle.kmeans_train(pts, 50, 2, 0)
    assert gc.shape[0] == 12 and np.array_equal(gc, oc) and np.array_equal(ga, oa)


def test_float_data_invariants(gpu_ok):
    """GMM points (reduced C5 shape): the final assignment is nearest-centroid for
    the returned centroids, the CSR matches it, runs are deterministic, and the
    centroids follow the oracle loop: bit-identical except in cells where a
    near-tie point went the other way under the GPU's norm-identity distances."""
    cents, pts = datagen.kmeans_assign(npts=40_000, ncent=512, seed=4)
    del cents
    nlist, iters, mpc = 256, 3, 64
    print("[kmeans] float invariants", flush=True)
    gc, ga, gs, go = mflat.kmeans_train(pts, nlist, iters, mpc)
    check_csr(ga, gs, go, nlist)
    oi, od = oracle.argmin_l2(pts, gc)
    gd = np.sum((pts.astype(np.float64) - gc[ga]) ** 2, axis=1).astype(np.float32)
    parity.tolerant(ga[:, None], gd[:, None], oi[:, None], od[:, None], gc, pts, 0)
    gc1, ga1, _, _ = mflat.kmeans_train(pts, nlist, iters, mpc)
    assert np.array_equal(gc1, gc) and np.array_equal(ga1, ga)
    oc, _, _, _ = oracle.kmeans_train(pts, nlist, iters, mpc)
    same = np.all(gc == oc, axis=1)
    print(f"[kmeans] bit-identical centroids {same.mean():.4f}, max diff {np.abs(gc - oc).max():.3g}", flush=True)
    assert same.mean() >= 0.9
    assert np.abs(gc - oc).max() < 0.05
