# SPDX-License-Identifier: Apache-2.0
"""Pins the IVF oracle (oracle.ivf_*: the reference's CoarseQuantizer CSR and
probe, src/CoarseQuantizer.mm:134-143,190-197, and IvfIndex's searchCpu,
src/IvfIndex.mm:518-560) with checks that do not restate its loop:

  * all cells probed: the result is the exact flat search (orc_cpu_search, a
    separate restatement) whenever distances are distinct;
  * brute force over the union of the probed cells, ranked by (distance, scan
    position) with Python-level sorting, on integer data full of exact ties --
    a tie order by id instead of scan order, a dropped cell, a probe-order slip
    or a wrong reordered id fails it;
  * nprobe = 1 is the top-k of the nearest cell alone; padding beyond the union;
  * the CSR against numpy's stable argsort; the probe against a brute-force
    lexicographic sort of (sqL2, cell).
"""
import numpy as np
import pytest

import oracle


def int_data(n, d, hi, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, hi, size=(n, d)).astype(np.float32)


def random_csr(n, nlist, seed):
    rng = np.random.default_rng(seed)
    assign = rng.integers(0, nlist, size=n)
    return (assign,) + oracle.ivf_csr(assign, nlist)


def test_csr_matches_stable_argsort():
    assign, start, rid = random_csr(5000, 37, seed=1)
    assert start[0] == 0 and start[-1] == 5000
    assert np.array_equal(np.diff(start), np.bincount(assign, minlength=37))
    assert np.array_equal(rid, np.argsort(assign, kind="stable"))


def sql2_seq(a, b):
    """float32 sequential (a - b)^2 sum, the reference's sqL2 order."""
    acc = np.float32(0.0)
    for x, y in zip(a, b):
        e = np.float32(x) - np.float32(y)
        acc = np.float32(acc + np.float32(e * e))
    return acc


def test_probe_is_lexicographic_nearest_cells():
    cent = int_data(40, 6, 4, seed=2)          # many exactly tied centroid distances
    q = int_data(25, 6, 4, seed=3)
    got = oracle.ivf_probe(cent, q, 7)
    for r in range(q.shape[0]):
        order = sorted(range(cent.shape[0]), key=lambda c: (float(sql2_seq(q[r], cent[c])), c))
        assert list(got[r]) == order[:7]


def brute_union(db, start, rid, q, k, probed, metric):
    """Top-k over the probed cells by (score, scan position); python sort."""
    ids = np.full((q.shape[0], k), -1, np.int32)
    vals = np.full((q.shape[0], k), np.inf if metric == 0 else -np.inf, np.float32)
    for r in range(q.shape[0]):
        cand = []
        pos = 0
        for c in probed[r]:
            for slot in range(start[c], start[c + 1]):
                row = rid[slot]
                if metric == 0:
                    key = float(np.sum((db[row].astype(np.float64) - q[r]) ** 2))
                else:
                    key = -float(db[row].astype(np.float64) @ q[r])
                cand.append((key, pos, row))
                pos += 1
        cand.sort()
        for i, (key, _, row) in enumerate(cand[:k]):
            ids[r, i] = row
            vals[r, i] = key if metric == 0 else -key
    return ids, vals


@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("nprobe", [1, 3, 8])
def test_against_brute_force_with_ties(metric, nprobe):
    # integer data: every score is exact in fp32, and ties are plentiful
    db = int_data(600, 8, 3, seed=10 + nprobe)
    q = int_data(40, 8, 3, seed=20 + nprobe)
    assign, start, rid = random_csr(db.shape[0], 12, seed=nprobe)
    rng = np.random.default_rng(nprobe)
    probed = np.stack([rng.permutation(12)[:nprobe] for _ in range(q.shape[0])]).astype(np.int32)
    oi, ov = oracle.ivf_search(db, start, rid, q, 15, probed, metric)
    bi, bv = brute_union(db, start, rid, q, 15, probed, metric)
    assert np.array_equal(oi, bi)
    assert np.array_equal(ov, bv)


def test_all_cells_is_flat_search():
    rng = np.random.default_rng(5)
    db = rng.standard_normal((3000, 24)).astype(np.float32)
    q = rng.standard_normal((30, 24)).astype(np.float32)
    cent = db[:20].copy()
    assign, _ = oracle.argmin_l2(db, cent)
    start, rid = oracle.ivf_csr(assign, 20)
    for metric in (0, 1, 2):
        probed = oracle.ivf_probe(cent, q, 20, metric)
        assert sorted(probed[0].tolist()) == list(range(20))
        oi, ov = oracle.ivf_search(db, start, rid, q, 12, probed, metric)
        fi, fv = oracle.flat_search(db, q, 12, metric)
        assert np.array_equal(oi, fi), metric
        assert np.array_equal(ov, fv), metric


def test_nprobe1_is_nearest_cell_alone_and_pads():
    db = int_data(400, 5, 50, seed=7)
    cent = db[[0, 100, 200, 300]].copy()
    assign, _ = oracle.argmin_l2(db, cent)
    start, rid = oracle.ivf_csr(assign, 4)
    q = int_data(10, 5, 50, seed=8)
    probed = oracle.ivf_probe(cent, q, 1)
    k = 500   # more than any cell holds
    oi, ov = oracle.ivf_search(db, start, rid, q, k, probed, 0)
    for r in range(q.shape[0]):
        c = probed[r, 0]
        members = rid[start[c]:start[c + 1]]
        fi, fv = oracle.flat_search(db[members], q[r:r + 1], k, 0)
        n = members.size
        assert np.array_equal(oi[r, :n], members[fi[0, :n]])
        assert np.array_equal(ov[r, :n], fv[0, :n])
        assert np.all(oi[r, n:] == -1) and np.all(np.isinf(ov[r, n:]))


def test_cosine_is_ip_on_normalised_inputs():
    rng = np.random.default_rng(9)
    db = rng.standard_normal((800, 16)).astype(np.float32) * 3
    q = rng.standard_normal((12, 16)).astype(np.float32)
    assign = rng.integers(0, 6, size=800)
    start, rid = oracle.ivf_csr(assign, 6)
    probed = np.tile(np.arange(6, dtype=np.int32)[::-1], (12, 1))
    ci, cv = oracle.ivf_search(db, start, rid, q, 9, probed, 2)
    ii, iv = oracle.ivf_search(oracle.normalize_rows(db), start, rid, oracle.normalize_rows(q), 9, probed, 1)
    assert np.array_equal(ci, ii) and np.array_equal(cv, iv)
