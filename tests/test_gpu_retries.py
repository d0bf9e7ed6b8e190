# SPDX-License-Identifier: Apache-2.0
"""Retries of the flat search: device-built work lists, the exact second round
and the host's fallback windows, on integer-valued data (every fp32 sum exact,
so results are compared with the oracle bit for bit).

A database whose row order follows distance puts every row under a query's
first bound into one or two database splits: their regions overflow, the k-th
best of what they stored admits still more rows than a region holds, and only
the second round's count-sized region ends it. Knobs read when an index is
created (MFLAT_RETRY_WINDOW, MFLAT_RETRY_POOL) shrink the device-built window
and the second round's pool, so the host's fallback windows and pool drain run
too; results never depend on them.
"""
import numpy as np
import pytest

import mflat
import oracle
import parity
from conftest import oracle_threads

pytestmark = pytest.mark.gpu

L2 = mflat.MFLAT_METRIC_L2


def sorted_db(nb, d, seed, block):
    """Rows whose first coordinate is row // block (so distance from a query at
    the origin grows with the row index, in steps) and whose other coordinates
    are 0..3: squared distances stay below 2^24, exact in fp32, with many ties."""
    rng = np.random.default_rng(seed)
    x = rng.integers(0, 4, size=(nb, d)).astype(np.float32)
    x[:, 0] = (np.arange(nb) // block).astype(np.float32)
    return x


def queries(n, d, seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 4, size=(n, d)).astype(np.float32)
    q[:, 0] = 0.0
    return q


def check(x, q, k, env, monkeypatch):
    for name in ("MFLAT_RETRY_WINDOW", "MFLAT_RETRY_POOL"):
        monkeypatch.delenv(name, raising=False)
    for name, v in env.items():
        monkeypatch.setenv(name, str(v))   # read when the index is created
    print(f"[retries] nb={x.shape[0]} d={x.shape[1]} nq={q.shape[0]} k={k} env={env}", flush=True)
    with mflat.FlatIndex(x.shape[1], L2) as idx:
        idx.add(x)
        gi, gd, ku = idx.search(q, k)
    assert ku == k
    oi, od = oracle.flat_search(x, q, k, threads=oracle_threads())
    parity.exact(gi, gd, oi, od)


def test_distance_sorted_10m_small_batches(gpu_ok, monkeypatch):
    """10M x 16, rank following row order; batches of 1 and 16 queries, k = 10
    and 40 (a single query at k <= 32 takes the streaming top-k scan; the rest
    the sample, full pass and retries of the streaming kernel family)."""
    x = sorted_db(10_000_000, 16, seed=31, block=2500)
    for nq in (1, 16):
        for k in (10, 40):
            check(x, queries(nq, 16, seed=32 + nq), k, {}, monkeypatch)


def test_distance_sorted_large_batch(gpu_ok, monkeypatch):
    """2M x 16, rank following row order, 300 queries (the 128-query kernels):
    most queries fail the full pass. Default plan, then a 16-query window (the
    host runs the other windows) and a 64-entry pool (the retry pass drains
    through the host's pool fallback)."""
    x = sorted_db(2_000_000, 16, seed=33, block=500)
    q = queries(300, 16, seed=34)
    check(x, q, 10, {}, monkeypatch)
    check(x, q, 10, {"MFLAT_RETRY_WINDOW": 16}, monkeypatch)
    check(x, q, 50, {"MFLAT_RETRY_WINDOW": 16, "MFLAT_RETRY_POOL": 64}, monkeypatch)


def test_small_batch_pool_fallback(gpu_ok, monkeypatch):
    """The streaming (<= 64 queries) family through the same fallbacks."""
    x = sorted_db(3_000_000, 16, seed=35, block=800)
    q = queries(40, 16, seed=36)
    check(x, q, 20, {"MFLAT_RETRY_WINDOW": 8, "MFLAT_RETRY_POOL": 32}, monkeypatch)
