# SPDX-License-Identifier: Apache-2.0
"""Writes the committed fixtures in this directory. Run in a container where the
reference tree exists and `make -C oracle ref` has built oracle/_ref:

    python tests/golden/make_golden.py

distance_primitives.npz  inputs and outputs of the reference's own
                         src/Distance.h dot / sqL2 / rowSqNorms / normalizeRows,
                         computed by that code (oracle/_ref).
flat_small.npz           small flat searches (ties, padding, NaN and +-inf rows,
                         every metric) whose
                         expected results are derived from the reference's
                         primitives: every (query, row) score by ref_score
                         (src/Distance.h:67-69), winners in the order strict '>'
                         insertion yields (score descending, id ascending;
                         src/FlatIndex.mm:259-290), values by ref_score_to_value,
                         padding ids -1 / ref_empty_value; Cosine rows and queries
                         normalised by ref_normalize_rows (src/FlatIndex.mm:241,313).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle  # noqa: E402


def primitives(r):
    rng = np.random.default_rng(2024)
    d = 77
    a = rng.uniform(-4, 4, size=(64, d)).astype(np.float32)
    b = rng.uniform(-4, 4, size=(64, d)).astype(np.float32)
    v = rng.standard_normal((32, 130)).astype(np.float32) * 5
    v[4] = 0.0
    dot = np.array([r.ref_dot(a[i].ctypes.data, b[i].ctypes.data, d) for i in range(64)], np.float32)
    sq = np.array([r.ref_sql2(a[i].ctypes.data, b[i].ctypes.data, d) for i in range(64)], np.float32)
    norms = np.empty(32, np.float32)
    r.ref_row_sq_norms(v.ctypes.data, 32, 130, norms.ctypes.data)
    nv = v.copy()
    r.ref_normalize_rows(nv.ctypes.data, 32, 130)
    np.savez(os.path.join(HERE, "distance_primitives.npz"), a=a, b=b, v=v, dot=dot, sql2=sq,
             norms=norms, normalized=nv)


def ref_search(r, x, q, k, metric):
    x = np.ascontiguousarray(x, np.float32)
    q = np.ascontiguousarray(q, np.float32)
    if metric == 2:
        x = x.copy(); q = q.copy()
        r.ref_normalize_rows(x.ctypes.data, x.shape[0], x.shape[1])
        r.ref_normalize_rows(q.ctypes.data, q.shape[0], q.shape[1])
    sm = 0 if metric == 0 else 1
    nb, d = x.shape
    ids = np.full((q.shape[0], k), -1, np.int32)
    vals = np.full((q.shape[0], k), r.ref_empty_value(metric), np.float32)
    for i in range(q.shape[0]):
        s = np.array([r.ref_score(sm, q[i].ctypes.data, x[j].ctypes.data, d) for j in range(nb)], np.float32)
        ok = s > -np.inf           # a -inf / NaN score is never inserted
        cand = np.nonzero(ok)[0]
        order = cand[np.lexsort((cand, -s[cand]))][:k]
        ids[i, :len(order)] = order
        vals[i, :len(order)] = [r.ref_score_to_value(sm, float(s[j])) for j in order]
    return ids, vals


def flat_cases():
    rng = np.random.default_rng(99)
    base = rng.integers(0, 3, size=(6, 5)).astype(np.float32)
    cases = {
        "ties_l2": (np.vstack([base] * 5), base[:4] + 0, 7, 0),
        "ties_ip": (np.vstack([base] * 5), base[:4] + 0, 9, 1),
        "pad_l2": (rng.uniform(-1, 1, (6, 9)).astype(np.float32), rng.uniform(-1, 1, (3, 9)).astype(np.float32), 10, 0),
        "pad_cos": (rng.uniform(-1, 1, (4, 9)).astype(np.float32), rng.uniform(-1, 1, (3, 9)).astype(np.float32), 6, 2),
        "float_l2": (rng.standard_normal((300, 33)).astype(np.float32), rng.standard_normal((12, 33)).astype(np.float32), 20, 0),
        "float_ip": (rng.standard_normal((300, 33)).astype(np.float32), rng.standard_normal((12, 33)).astype(np.float32), 20, 1),
        "float_cos": (rng.standard_normal((300, 33)).astype(np.float32) * 7, rng.standard_normal((12, 33)).astype(np.float32), 20, 2),
        "int_l2": (rng.integers(0, 256, (400, 64)).astype(np.float32), rng.integers(0, 256, (10, 64)).astype(np.float32), 15, 0),
    }
    nanx = rng.standard_normal((40, 6)).astype(np.float32)
    nanx[3, 1] = np.nan
    cases["nan_row_l2"] = (nanx, rng.standard_normal((3, 6)).astype(np.float32), 40, 0)
    # rows holding +inf / -inf: an L2 score of -inf is never inserted; an inner
    # product of +inf is the best score there is (value +inf), one of -inf is
    # never inserted. Queries have no zero coordinate (no inf * 0 = NaN).
    infx = rng.standard_normal((50, 8)).astype(np.float32)
    infx[7, 2] = np.inf
    infx[19, 5] = -np.inf
    infq = rng.standard_normal((4, 8)).astype(np.float32)
    cases["inf_rows_l2"] = (infx, infq, 50, 0)
    cases["inf_rows_ip"] = (infx, infq, 50, 1)
    return cases


def main():
    r = oracle.ref_lib()
    if r is None:
        raise SystemExit("oracle/_ref/libref_distance.so missing: run `make -C oracle ref`")
    primitives(r)
    out = {}
    for name, (x, q, k, metric) in flat_cases().items():
        ids, vals = ref_search(r, x, q, k, metric)
        out[name + "__x"] = x
        out[name + "__q"] = q
        out[name + "__k"] = np.int64(k)
        out[name + "__metric"] = np.int64(metric)
        out[name + "__ids"] = ids
        out[name + "__vals"] = vals
    np.savez(os.path.join(HERE, "flat_small.npz"), **out)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
