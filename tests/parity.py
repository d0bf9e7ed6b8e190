# SPDX-License-Identifier: Apache-2.0
"""Parity comparison between the HIP path and the oracle.

Integer / exactly representable inputs: bit-exact ids and distances.
Floating-point inputs (tolerances stated by the build target):
  * per query, the id SET equals the oracle's, except ids whose distance lies
    within a relative gap of REL_TIE = 1e-5 of the oracle's k-th value
    (near-ties at the cut);
  * distances compared position-wise on the sorted lists within REL_DIST
    (1e-4 for fp32 inputs) relative, plus, for L2, an absolute floor of
    2^-20 * (||q||^2 + ||x||^2) that covers the cancellation of the
    ||q||^2 + ||x||^2 - 2 q.x identity (e.g. exact self-matches at 0).
"""
import numpy as np

REL_TIE = 1e-5
REL_DIST_FP32 = 1e-4


def exact(gi, gd, oi, od):
    assert gi.shape == oi.shape, (gi.shape, oi.shape)
    bad = np.nonzero(np.any(gi != oi, axis=1) | np.any(gd != od, axis=1))[0]
    assert bad.size == 0, f"{bad.size} queries differ; first {bad[:5]}: gpu {gi[bad[0]][:8]} {gd[bad[0]][:8]} " \
                          f"oracle {oi[bad[0]][:8]} {od[bad[0]][:8]}"


def true_values(db, q, ids, metric):
    """float64 metric values of (q, db[id]) pairs; -1 ids -> nan."""
    out = np.full(ids.shape, np.nan)
    for r in range(ids.shape[0]):
        v = ids[r]
        ok = v >= 0
        x = db[v[ok]].astype(np.float64)
        qq = q[r].astype(np.float64)
        if metric == 0:
            out[r, ok] = np.sum((x - qq) ** 2, axis=1)
        else:
            out[r, ok] = x @ qq
    return out


def tolerant(gi, gd, oi, od, db, q, metric, rel_dist=REL_DIST_FP32, rel_tie=REL_TIE):
    """metric: 0 L2 (smaller nearer), else similarity (larger nearer); db/q are the
    vectors the scores were computed on (normalised ones for cosine)."""
    assert gi.shape == oi.shape
    m, k = oi.shape
    qn = np.sum(q.astype(np.float64) ** 2, axis=1)
    xn = np.sum(db.astype(np.float64) ** 2, axis=1)
    tg = true_values(db, q, gi, metric)
    to = true_values(db, q, oi, metric)
    nbad = 0
    msgs = []
    for r in range(m):
        kth = od[r, k - 1]
        floor = 2.0 ** -20 * (qn[r] + (xn.max() if xn.size else 0.0)) if metric == 0 else 1e-6
        gap = rel_tie * abs(kth) + floor
        sg, so = set(gi[r].tolist()), set(oi[r].tolist())
        ok = True
        for i in sg - so:
            j = list(gi[r]).index(i)
            if i < 0 or not abs(tg[r, j] - kth) <= gap:
                ok = False
        for i in so - sg:
            j = list(oi[r]).index(i)
            if i < 0 or not abs(to[r, j] - kth) <= gap:
                ok = False
        fl = floor if metric == 0 else 1e-6
        dd = np.abs(gd[r].astype(np.float64) - od[r].astype(np.float64))
        fin = np.isfinite(od[r])
        if not np.array_equal(np.isfinite(gd[r]), fin):
            ok = False
        elif np.any(dd[fin] > rel_dist * np.abs(od[r][fin]) + fl):
            ok = False
        if not ok:
            nbad += 1
            if len(msgs) < 3:
                msgs.append(f"q{r}: gpu {gi[r][:6]} {gd[r][:6]} / oracle {oi[r][:6]} {od[r][:6]}")
    assert nbad == 0, f"{nbad}/{m} queries out of tolerance: " + " | ".join(msgs)


def sorted_lex(ids, vals, metric):
    """Rows ordered nearest-first with ties by ascending id (-1 padding last)."""
    for r in range(ids.shape[0]):
        n = int(np.sum(ids[r] >= 0))
        assert np.all(ids[r, n:] == -1)
        key = vals[r, :n] if metric == 0 else -vals[r, :n]
        for i in range(n - 1):
            assert key[i] < key[i + 1] or (key[i] == key[i + 1] and ids[r, i] < ids[r, i + 1]), (r, i)
