# SPDX-License-Identifier: Apache-2.0
"""Parity comparison between the HIP path and the oracle.

Integer / exactly representable inputs: bit-exact ids and distances.
Floating-point inputs (tolerances stated by the build target):
  * per query, the id SET equals the oracle's, except ids whose distance lies
    within a relative gap of REL_TIE = 1e-5 of the oracle's k-th value
    (near-ties at the cut);
  * distances compared position-wise on the sorted lists within REL_DIST
    (1e-4 for fp32 inputs) relative, plus, for L2, an absolute floor of
    2^-20 * (||q||^2 + ||x||^2), x the pair's own row (the larger norm of the
    two rows compared at a position), that covers the cancellation of the
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


def tolerant(gi, gd, oi, od, db, q, metric, rel_dist=REL_DIST_FP32, rel_tie=REL_TIE):
    """metric: 0 L2 (smaller nearer), else similarity (larger nearer); db/q are the
    vectors the scores were computed on (normalised ones for cosine).

    Returns the number of near-tie swaps: ids one side returned and the other did
    not, each within the near-tie gap of the oracle's k-th value. Only the rows
    the two results name are read from db (float64 per query), so a 10M-row
    database is never copied whole."""
    assert gi.shape == oi.shape
    m, k = oi.shape
    nbad = 0
    swaps = 0
    msgs = []
    for r in range(m):
        qq = q[r].astype(np.float64)
        qn = float(qq @ qq)
        named = np.union1d(gi[r][gi[r] >= 0], oi[r][oi[r] >= 0])
        xs = db[named].astype(np.float64)
        xn = dict(zip(named.tolist(), np.sum(xs * xs, axis=1).tolist()))
        tv = np.sum((xs - qq) ** 2, axis=1) if metric == 0 else xs @ qq
        true = dict(zip(named.tolist(), tv.tolist()))

        def floor(*ids):
            # L2: the identity ||q||^2 + ||x||^2 - 2 q.x cancels to within a few
            # ulps of the pair's own norms (exact self-matches come out near 0)
            if metric != 0:
                return 1e-6
            return 2.0 ** -20 * (qn + max([xn.get(i, 0.0) for i in ids if i >= 0] or [0.0]))

        kth = float(od[r, k - 1])
        sg, so = set(gi[r].tolist()), set(oi[r].tolist())
        ok = True
        for i in (sg - so) | (so - sg):
            if i < 0 or not abs(true[i] - kth) <= rel_tie * abs(kth) + floor(i):
                ok = False
        swaps += len(sg - so)
        fin = np.isfinite(od[r])
        if not np.array_equal(np.isfinite(gd[r]), fin):
            ok = False
        else:
            for j in np.nonzero(fin)[0]:
                g, o = float(gd[r, j]), float(od[r, j])
                if abs(g - o) > rel_dist * abs(o) + floor(int(gi[r, j]), int(oi[r, j])):
                    ok = False
                    break
        if not ok:
            nbad += 1
            if len(msgs) < 3:
                msgs.append(f"q{r}: gpu {gi[r][:6]} {gd[r][:6]} / oracle {oi[r][:6]} {od[r][:6]}")
    assert nbad == 0, f"{nbad}/{m} queries out of tolerance: " + " | ".join(msgs)
    return swaps


def sorted_lex(ids, vals, metric):
    """Rows ordered nearest-first with ties by ascending id (-1 padding last)."""
    for r in range(ids.shape[0]):
        n = int(np.sum(ids[r] >= 0))
        assert np.all(ids[r, n:] == -1)
        key = vals[r, :n] if metric == 0 else -vals[r, :n]
        for i in range(n - 1):
            assert key[i] < key[i + 1] or (key[i] == key[i + 1] and ids[r, i] < ids[r, i + 1]), (r, i)
