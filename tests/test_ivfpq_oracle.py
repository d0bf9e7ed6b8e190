# SPDX-License-Identifier: Apache-2.0
"""Pins the IVF-PQ oracle (oracle.ivfpq_search / pq_rerank / pq_train: the
reference's residual-ADC searchCpu, src/IvfPqIndex.mm:383-445, its rerank
:598-625, and its per-sub-space k-means training, src/PqTrainer.h:37-66) with
checks that do not restate its loops:

  * on integer-valued centroids, sub-centroids and queries every product and
    sum is exact in fp32, so the ADC distance must equal ||q - x_hat||^2 of
    the reconstruction x_hat = c + concat_m(p_m[code_m]) computed in integers --
    a dropped term, a wrong sign, a swapped table index or an off-by-one
    sub-space fails it;
  * the ranking against a Python sort of (distance, scan position) over the
    probed cells (scan order: cells in probe order, rows in cell order), with
    duplicate codes making exact ties;
  * the rerank against an exact float64 brute force over the shortlist;
  * the trained codes are each sub-vector's nearest sub-centroid (lowest index
    on ties), and fewer rows than 256 cells wrap the seeds.
"""
import numpy as np
import pytest

import oracle


def int_pq_case(seed, n=700, d=12, M=4, nlist=5, nq=30):
    rng = np.random.default_rng(seed)
    cent = rng.integers(-3, 4, size=(nlist, d)).astype(np.float32)
    pqc = rng.integers(-2, 3, size=(M, 256, d // M)).astype(np.float32)
    codes = rng.integers(0, 256, size=(n, M)).astype(np.uint8)
    codes[n // 2:n // 2 + 40] = codes[n // 2]   # duplicates -> exact ties
    assign = rng.integers(0, nlist, size=n)
    start, rid = oracle.ivf_csr(assign, nlist)
    codes_cell = codes[rid]
    q = rng.integers(-4, 5, size=(nq, d)).astype(np.float32)
    return cent, pqc, codes, assign, start, rid, codes_cell, q


def reconstruct(cent, pqc, codes, assign):
    M = pqc.shape[0]
    parts = [pqc[mm][codes[:, mm].astype(np.int64)] for mm in range(M)]
    return cent[assign].astype(np.int64) + np.concatenate(parts, axis=1).astype(np.int64)


@pytest.mark.parametrize("nprobe", [1, 2, 5])
def test_adc_is_exact_reconstruction_distance_on_integers(nprobe):
    cent, pqc, codes, assign, start, rid, codes_cell, q = int_pq_case(nprobe)
    rng = np.random.default_rng(100 + nprobe)
    probed = np.stack([rng.permutation(cent.shape[0])[:nprobe] for _ in range(q.shape[0])]).astype(np.int32)
    k = 25
    oi, ov = oracle.ivfpq_search(cent, start, rid, codes_cell, pqc, q, k, probed)
    xhat = reconstruct(cent, pqc, codes, assign)
    for r in range(q.shape[0]):
        cand = []
        pos = 0
        for c in probed[r]:
            for slot in range(start[c], start[c + 1]):
                row = rid[slot]
                cand.append((int(np.sum((xhat[row] - q[r].astype(np.int64)) ** 2)), pos, row))
                pos += 1
        cand.sort()
        want_i = [row for _, _, row in cand[:k]] + [-1] * max(0, k - len(cand))
        want_v = [float(dist) for dist, _, _ in cand[:k]] + [np.inf] * max(0, k - len(cand))
        assert list(oi[r]) == want_i, r
        assert np.array_equal(ov[r], np.array(want_v, np.float32)), r


def test_cosine_search_normalises_queries():
    cent, pqc, codes, assign, start, rid, codes_cell, q = int_pq_case(7)
    probed = np.tile(np.arange(cent.shape[0], dtype=np.int32), (q.shape[0], 1))
    a = oracle.ivfpq_search(cent, start, rid, codes_cell, pqc, q, 10, probed, metric=2)
    b = oracle.ivfpq_search(cent, start, rid, codes_cell, pqc, oracle.normalize_rows(q), 10, probed, metric=0)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_rerank_against_brute_force():
    rng = np.random.default_rng(3)
    full = rng.integers(0, 5, size=(400, 8)).astype(np.float32)
    q = rng.integers(0, 5, size=(20, 8)).astype(np.float32)
    short = np.stack([rng.permutation(400)[:60] for _ in range(20)]).astype(np.int32)
    short[3, 50:] = -1                                   # padding at the end of a shortlist
    for metric in (0, 2):
        ids, vals = oracle.pq_rerank(full, q, short, 12, metric)
        fn = oracle.normalize_rows(full) if metric == 2 else full
        qn = oracle.normalize_rows(q) if metric == 2 else q
        for r in range(20):
            cand = []
            for i, row in enumerate(short[r]):
                if row < 0:
                    continue
                if metric == 0:
                    key = float(np.sum((fn[row].astype(np.float64) - qn[r]) ** 2))
                else:
                    key = -float(fn[row].astype(np.float64) @ qn[r])
                cand.append((key, i, row))
            cand.sort()
            want = [row for _, _, row in cand[:12]]
            if metric == 0:   # integer data: exact values and ties
                assert list(ids[r]) == want, r
            else:             # normalised data: the float64 order, up to float32 near-ties
                got = set(ids[r].tolist())
                assert len(got & set(want)) >= 11, r


def test_trained_codes_are_nearest_subcentroids():
    rng = np.random.default_rng(4)
    r = rng.standard_normal((900, 8)).astype(np.float32)
    pqc, codes = oracle.pq_train(r, M=2, iters=3)
    for mm in range(2):
        sub = r[:, mm * 4:(mm + 1) * 4].astype(np.float64)
        d = np.sum((sub[:, None, :] - pqc[mm][None].astype(np.float64)) ** 2, axis=2)
        chosen = d[np.arange(900), codes[:, mm]]
        assert np.all(chosen <= d.min(axis=1) * (1 + 1e-6) + 1e-9)   # nearest, up to fp32 near-ties
    # one sub-space's codebook and codes are that sub-space's k-means
    c0, a0, _, _ = oracle.kmeans_train(np.ascontiguousarray(r[:, :4]), 256, 3, 0, wrap=True)
    assert np.array_equal(c0, pqc[0]) and np.array_equal(a0, codes[:, 0])


def test_fewer_rows_than_cells_wrap_the_seeds():
    r = np.arange(40 * 4, dtype=np.float32).reshape(40, 4)
    cent, assign, start, order = oracle.kmeans_train(r, 256, 0, 0, wrap=True)
    assert cent.shape == (256, 4)
    rng = oracle.MT19937Stream(12345)
    perm = oracle.seed_permutation(40, rng)
    assert np.array_equal(cent, r[perm[np.arange(256) % 40]])
    assert np.all(assign < 40)   # duplicate seeds beyond the first never win (strict <)
