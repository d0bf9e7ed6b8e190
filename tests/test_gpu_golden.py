# SPDX-License-Identifier: Apache-2.0
"""The committed golden searches (tests/golden/flat_small.npz, expected results
derived from the reference's own src/Distance.h primitives by
tests/golden/make_golden.py) run through the HIP path via mflat_flat_search.

Integer-valued cases (every fp32 sum exact, ties everywhere) must match bit for
bit, ids and values; float cases within the fp32 tolerances of tests/parity.py
(the GPU computes L2 through the norm identity, the reference's CPU path by a
direct sum). A row holding NaN is never returned; rows holding +-inf follow the
reference's strict '>' rule (an L2 score of -inf and an inner product of -inf
are never inserted, an inner product of +inf ranks first with value +inf);
padding is id -1 with +inf (L2) / -inf (IP, Cosine)."""
import os

import numpy as np
import pytest

import mflat
import oracle
import parity

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "flat_small.npz")
EXACT = {"ties_l2", "ties_ip", "int_l2"}


def _cases():
    z = np.load(GOLDEN)
    return sorted({f.split("__")[0] for f in z.files})


@pytest.mark.parametrize("name", _cases())
def test_golden_case_through_hip(gpu_ok, name):
    z = np.load(GOLDEN)
    x, q = z[name + "__x"], z[name + "__q"]
    k, metric = int(z[name + "__k"]), int(z[name + "__metric"])
    ids, vals = z[name + "__ids"], z[name + "__vals"]
    print(f"[golden] {name}: nb={x.shape[0]} d={x.shape[1]} m={q.shape[0]} k={k} metric={metric}", flush=True)
    with mflat.FlatIndex(x.shape[1], metric) as idx:
        assert idx.ready()
        idx.add(x)
        gi, gd, ku = idx.search(q, k)
    assert ku == k
    parity.sorted_lex(gi, gd, 0 if metric == 0 else 1)
    # padding positions and kinds agree with the reference's
    assert np.array_equal(gi == -1, ids == -1), (gi, ids)
    pad = ids == -1
    assert np.all(gd[pad] == (np.inf if metric == 0 else -np.inf))
    if name in EXACT:
        parity.exact(gi, gd, ids, vals)
        return
    bad = [r for r in range(x.shape[0]) if not np.all(np.isfinite(x[r]))]
    if bad and metric == 0:
        assert not np.isin(gi, bad).any(), "a row holding NaN or inf was returned for L2"
    if name == "inf_rows_ip":
        # +inf dots lead each list: compared exactly (value +inf, same ids, same
        # order); the finite remainder of each query within tolerance
        top = vals == np.inf
        assert np.array_equal(gi[top], ids[top]) and np.array_equal(gd[top], vals[top])
        xs = np.where(np.isfinite(x), x, 0.0).astype(np.float32)
        for r in range(q.shape[0]):
            n = int(top[r].sum())
            parity.tolerant(gi[r:r + 1, n:], gd[r:r + 1, n:], ids[r:r + 1, n:], vals[r:r + 1, n:], xs,
                            q[r:r + 1], 1)
        return
    if metric == 2:
        xs, qs, m = oracle.normalize_rows(x), oracle.normalize_rows(q), 1
    else:
        xs, qs, m = x, q, metric
    if name == "nan_row_l2":
        # the row holding NaN never ranks; compare against the finite rows
        assert not np.isin(gi, bad).any()
    xs = np.where(np.isfinite(xs), xs, 0.0).astype(np.float32)   # rows named are finite
    parity.tolerant(gi, gd, ids, vals, xs, qs, 0 if m == 0 else 1)
