# SPDX-License-Identifier: Apache-2.0
"""Deterministic synthetic workloads for flat search (the configurations named in
BASELINE.json). Sizes are parameters so tests can draw reduced versions of the
same distributions; the defaults are the full configurations.

All draws use numpy's PCG64 Generator seeded with the configuration's seed, in
float32, in a fixed order, so every process (tests, bench, oracle) sees the same
arrays for the same arguments.
"""
from __future__ import annotations

import numpy as np

L2, IP, COS = 0, 1, 2


def sift_like(nb=100_000, nq=1_000, d=128, seed=0):
    """C1: integer-valued uniform {0..255} entries stored as fp32."""
    rng = np.random.default_rng(seed)
    x = rng.integers(0, 256, size=(nb, d), dtype=np.int32).astype(np.float32)
    q = rng.integers(0, 256, size=(nq, d), dtype=np.int32).astype(np.float32)
    return x, q


def gmm(nb=1_000_000, nq=10_000, d=128, ncenters=1024, sigma=0.3, seed=1):
    """C2 (and the C5 point law): rows = centre[u] + sigma * N(0, I),
    centres ~ N(0, I), u uniform over centres."""
    rng = np.random.default_rng(seed)
    centers = rng.standard_normal((ncenters, d), dtype=np.float32)

    def draw(n):
        out = np.empty((n, d), dtype=np.float32)
        step = 1 << 18
        for s in range(0, n, step):
            e = min(n, s + step)
            u = rng.integers(0, ncenters, size=e - s)
            noise = rng.standard_normal((e - s, d), dtype=np.float32)
            out[s:e] = centers[u] + np.float32(sigma) * noise
        return out

    x = draw(nb)
    q = draw(nq)
    return x, q


def unit_normal(nb=1_000_000, nq=10_000, d=768, seed=2):
    """C3: N(0, I) rows normalised to unit length (inner-product search)."""
    rng = np.random.default_rng(seed)

    def draw(n):
        out = np.empty((n, d), dtype=np.float32)
        step = 1 << 16
        for s in range(0, n, step):
            e = min(n, s + step)
            v = rng.standard_normal((e - s, d), dtype=np.float32)
            nrm = np.sqrt(np.sum(v.astype(np.float64) ** 2, axis=1)).astype(np.float32)
            out[s:e] = v / nrm[:, None]
        return out

    x = draw(nb)
    q = draw(nq)
    return x, q


def uniform_pm1(nb=10_000_000, nq=64, d=96, seed=3):
    """C4: uniform [-1, 1] rows (HBM-bound small-batch search)."""
    rng = np.random.default_rng(seed)
    x = np.empty((nb, d), dtype=np.float32)
    step = 1 << 20
    for s in range(0, nb, step):
        e = min(nb, s + step)
        x[s:e] = rng.uniform(-1.0, 1.0, size=(e - s, d)).astype(np.float32)
    q = rng.uniform(-1.0, 1.0, size=(nq, d)).astype(np.float32)
    return x, q


def kmeans_assign(npts=2_000_000, ncent=65_536, d=128, ncenters=4096, sigma=0.5, seed=4):
    """C5: points from a GMM; centroids = distinct points sampled without
    replacement. Returns (centroids as the database, points as the queries)."""
    pts, _ = gmm(nb=npts, nq=0, d=d, ncenters=ncenters, sigma=sigma, seed=seed)
    rng = np.random.default_rng(seed + 1000)
    pick = rng.choice(npts, size=ncent, replace=False)
    pick.sort()
    cents = np.ascontiguousarray(pts[pick])
    return cents, pts


CONFIGS = {
    "C1": dict(gen=sift_like, metric=L2, k=10),
    "C2": dict(gen=gmm, metric=L2, k=100),
    "C3": dict(gen=unit_normal, metric=IP, k=100),
    "C4": dict(gen=uniform_pm1, metric=L2, k=10),
    "C5": dict(gen=kmeans_assign, metric=L2, k=1),
}
