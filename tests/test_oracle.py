# SPDX-License-Identifier: Apache-2.0
"""Pins the CPU oracle before it is trusted as the parity checker.

The reference holds no golden vectors or known-answer tests for this path, so
the oracle is pinned by:
  * the reference's own primitives (src/Distance.h, compiled where it lies into
    oracle/_ref by `make -C oracle ref`), bit for bit, live when built and via
    the committed fixture tests/golden/distance_primitives.npz otherwise;
  * closed forms (orthonormal bases, integer data whose fp32 sums are exact,
    exact self-matches, duplicated rows);
  * brute force: an independent lexicographic full sort and numpy float64;
  * invariants (sortedness, prefix property, padding, cosine == IP on unit rows,
    k = 1 == argmin).
Each check is chosen so a plausible slip (reversed tie order, '>=' instead of
'>', a dropped term, a wrong sign, float instead of double norms) fails it.
"""
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def rnd(shape, seed, lo=-3.0, hi=3.0):
    return np.random.default_rng(seed).uniform(lo, hi, size=shape).astype(np.float32)


def test_primitives_vs_reference_fixture():
    g = np.load(os.path.join(GOLDEN, "distance_primitives.npz"))
    a, b, v = g["a"], g["b"], g["v"]
    o = oracle.lib()
    d = a.shape[1]
    dots = np.array([o.orc_dot(a[i].ctypes.data, b[i].ctypes.data, d) for i in range(a.shape[0])], np.float32)
    sq = np.array([o.orc_sql2(a[i].ctypes.data, b[i].ctypes.data, d) for i in range(a.shape[0])], np.float32)
    assert np.array_equal(dots.view(np.uint32), g["dot"].view(np.uint32))
    assert np.array_equal(sq.view(np.uint32), g["sql2"].view(np.uint32))
    assert np.array_equal(oracle.row_sq_norms(v).view(np.uint32), g["norms"].view(np.uint32))
    assert np.array_equal(oracle.normalize_rows(v).view(np.uint32), g["normalized"].view(np.uint32))


@pytest.mark.skipif(oracle.ref_lib() is None, reason="oracle/_ref not built (reference tree absent)")
def test_primitives_vs_reference_live():
    r = oracle.ref_lib()
    o = oracle.lib()
    for d in (1, 3, 96, 128, 767):
        a = rnd((50, d), d)
        b = rnd((50, d), d + 1)
        for i in range(50):
            pa, pb = a[i].ctypes.data, b[i].ctypes.data
            assert np.float32(o.orc_dot(pa, pb, d)) == np.float32(r.ref_dot(pa, pb, d))
            assert np.float32(o.orc_sql2(pa, pb, d)) == np.float32(r.ref_sql2(pa, pb, d))
            assert np.float32(r.ref_score(0, pa, pb, d)) == -np.float32(o.orc_sql2(pa, pb, d))
            assert np.float32(r.ref_score(1, pa, pb, d)) == np.float32(o.orc_dot(pa, pb, d))
        ref_n = np.empty(50, np.float32)
        r.ref_row_sq_norms(a.ctypes.data, 50, d, ref_n.ctypes.data)
        assert np.array_equal(ref_n, oracle.row_sq_norms(a))
        an = a.copy()
        an[3] = 0.0
        ref_v = an.copy()
        r.ref_normalize_rows(ref_v.ctypes.data, 50, d)
        assert np.array_equal(ref_v.view(np.uint32), oracle.normalize_rows(an).view(np.uint32))
    assert r.ref_empty_value(0) == np.inf and r.ref_empty_value(1) == -np.inf
    assert r.ref_score_to_value(0, -2.5) == 2.5 and r.ref_score_to_value(2, 1.5) == 1.5


def test_norms_are_double_accumulated():
    # A float accumulation of these squares loses the small terms; double keeps them.
    v = np.array([[4096.0] + [1.0] * 127], np.float32)
    got = oracle.row_sq_norms(v)[0]
    assert got == np.float32(4096.0 ** 2 + 127)
    assert got != np.float32(4096.0 ** 2)   # what a float accumulation returns


def test_integer_data_matches_float64_brute_force():
    rng = np.random.default_rng(0)
    x = rng.integers(0, 256, size=(3000, 64)).astype(np.float32)
    q = rng.integers(0, 256, size=(40, 64)).astype(np.float32)
    ids, vals = oracle.flat_search(x, q, 25, metric=0)
    d = ((q[:, None, :].astype(np.float64) - x[None, :, :]) ** 2).sum(-1)
    for r in range(40):
        order = np.lexsort((np.arange(3000), d[r]))[:25]
        assert np.array_equal(ids[r], order)
        assert np.array_equal(vals[r], d[r, order].astype(np.float32))


def test_matches_independent_lexicographic_sort():
    x = rnd((2000, 48), 1)
    q = rnd((30, 48), 2)
    a_ids, a_vals = oracle.flat_search(x, q, 40, metric=0)
    b_ids, b_vals = oracle.brute_lex(x, q, 40)
    assert np.array_equal(a_ids, b_ids) and np.array_equal(a_vals, b_vals)


def test_ties_keep_lowest_id_first():
    base = np.array([[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0]], np.float32)
    x = np.concatenate([base, base, base, base])   # ids i, i+3, i+6, i+9 identical
    q = np.array([[1, 0, 0, 0]], np.float32)
    ids, vals = oracle.flat_search(x, q, 6, metric=0)
    assert ids[0].tolist() == [0, 3, 6, 9, 1, 2]
    assert vals[0].tolist() == [0, 0, 0, 0, 2, 2]
    # the k-th slot among equals goes to the lowest id (strict '>' insertion)
    ids, _ = oracle.flat_search(x, q, 2, metric=0)
    assert ids[0].tolist() == [0, 3]
    ids, vals = oracle.flat_search(x, q, 5, metric=1)
    assert ids[0].tolist() == [0, 3, 6, 9, 1] and vals[0].tolist() == [1, 1, 1, 1, 0]


def test_orthonormal_basis_inner_product():
    d = 32
    x = np.eye(d, dtype=np.float32)
    q = rnd((10, d), 5)
    ids, vals = oracle.flat_search(x, q, 8, metric=1)
    for r in range(10):
        order = np.lexsort((np.arange(d), -q[r]))[:8]
        assert np.array_equal(ids[r], order)
        assert np.array_equal(vals[r], q[r, order])


def test_self_match_is_zero_and_first():
    x = rnd((500, 20), 6)
    ids, vals = oracle.flat_search(x, x[:50], 3, metric=0)
    assert np.array_equal(ids[:, 0], np.arange(50)) and np.all(vals[:, 0] == 0)


def test_padding_when_db_smaller_than_k():
    x = rnd((5, 8), 7)
    q = rnd((2, 8), 8)
    for metric, empty in ((0, np.inf), (1, -np.inf), (2, -np.inf)):
        ids, vals = oracle.flat_search(x, q, 9, metric=metric)
        assert np.all(ids[:, 5:] == -1) and np.all(vals[:, 5:] == empty)
        assert sorted(ids[0, :5].tolist()) == [0, 1, 2, 3, 4]
    ids, vals = oracle.flat_search(np.zeros((0, 8), np.float32), q, 4, metric=0)
    assert np.all(ids == -1) and np.all(vals == np.inf)


def test_sorted_and_prefix_property():
    x = rnd((4000, 16), 9)
    q = rnd((20, 16), 10)
    i10, v10 = oracle.flat_search(x, q, 10, metric=0)
    i50, v50 = oracle.flat_search(x, q, 50, metric=0)
    assert np.array_equal(i50[:, :10], i10) and np.array_equal(v50[:, :10], v10)
    assert np.all(np.diff(v50, axis=1) >= 0)
    j10, w10 = oracle.flat_search(x, q, 10, metric=1)
    assert np.all(np.diff(w10, axis=1) <= 0)


def test_cosine_equals_ip_on_normalised_rows():
    x = rnd((1000, 24), 11)
    q = rnd((15, 24), 12)
    ci, cv = oracle.flat_search(x, q, 12, metric=2)
    ii, iv = oracle.flat_search(oracle.normalize_rows(x), oracle.normalize_rows(q), 12, metric=1)
    assert np.array_equal(ci, ii) and np.array_equal(cv, iv)
    n = oracle.normalize_rows(np.vstack([x[:3], np.zeros((1, 24), np.float32)]))
    assert np.all(n[3] == 0)
    assert np.allclose(np.sum(n[:3].astype(np.float64) ** 2, axis=1), 1.0, atol=1e-6)


def test_k1_equals_argmin():
    x = rnd((3000, 12), 13)
    q = rnd((100, 12), 14)
    i1, v1 = oracle.flat_search(x, q, 1, metric=0)
    ai, ad = oracle.argmin_l2(q, x)
    assert np.array_equal(i1[:, 0], ai) and np.array_equal(v1[:, 0], ad)


def test_nan_rows_never_inserted():
    x = rnd((50, 8), 15)
    x[7, 2] = np.nan
    q = x[7:8].copy()
    q[0, 2] = 0.0
    ids, _ = oracle.flat_search(x, q, 50, metric=0)
    assert 7 not in ids[0].tolist() and ids[0, -1] == -1


def test_threaded_equals_serial():
    x = rnd((3000, 32), 16)
    q = rnd((64, 32), 17)
    a = oracle.flat_search(x, q, 20, metric=0, threads=1)
    b = oracle.flat_search(x, q, 20, metric=0, threads=8)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_golden_flat_fixture():
    """Regression fixture: oracle results on small fixed inputs (ties, padding,
    every metric), generated by tests/golden/make_golden.py."""
    g = np.load(os.path.join(GOLDEN, "flat_small.npz"))
    for name in sorted({k.split("__")[0] for k in g.files}):
        x, q = g[name + "__x"], g[name + "__q"]
        metric, k = int(g[name + "__metric"]), int(g[name + "__k"])
        ids, vals = oracle.flat_search(x, q, k, metric=metric)
        assert np.array_equal(ids, g[name + "__ids"]), name
        assert np.array_equal(vals.view(np.uint32), g[name + "__vals"].view(np.uint32)), name


# ---- reduced-precision rounding (oracle inputs for fp16 / bf16 storage) -------

def test_round_bf16_matches_torch_and_closed_forms():
    """bf16 rounding against torch's CPU conversion (round to nearest even) on
    random values across magnitudes and on the cases a slip would break: exact
    ties to even, overflow to inf, subnormals, signed zero, inf and NaN."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(21)
    x = (rng.standard_normal(200_000) * np.exp(rng.uniform(-60, 60, 200_000))).astype(np.float32)
    special = np.array([0.0, -0.0, 1.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -8 + 2.0 ** -20,
                        3.3895314e38, 3.4e38, -3.4e38, np.inf, -np.inf, 1e-40, -1e-45, 2.0 ** -126],
                       dtype=np.float32)
    for v in (x, special):
        a = oracle.round_bf16(v)
        b = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    r = oracle.round_bf16(special)
    assert r[3] == 1.0                      # tie -> even (mantissa 0)
    assert r[4] == 1.0 + 2.0 ** -6          # tie -> even (rounds up)
    assert r[5] == 1.0 + 2.0 ** -7          # above the tie -> up
    assert np.isinf(r[7]) and r[7] > 0 and np.isinf(r[8]) and r[8] < 0
    assert np.signbit(r[1]) and r[1] == 0.0
    n = oracle.round_bf16(np.array([np.nan, -np.nan], np.float32))
    assert np.all(n.view(np.uint32) == 0x7FC00000)


def test_round_f16_closed_forms():
    v = np.array([1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 65504.0, 65519.0, 65520.0, 2.0 ** -24,
                  2.0 ** -25, 255.0, -0.0], dtype=np.float32)
    r = oracle.round_f16(v)
    assert r[0] == 1.0 and r[1] == 1.0 + 2.0 ** -9       # ties to even
    assert r[2] == 65504.0 and r[3] == 65504.0 and np.isinf(r[4])
    assert r[5] == 2.0 ** -24 and r[6] == 0.0            # smallest subnormal; tie -> 0
    assert r[7] == 255.0 and np.signbit(r[8])


def test_storage_inputs_integer_data_is_identity():
    """Integers 0..255 are exact in fp16 and bf16, so the storage oracle on C1-like
    data is the fp32 oracle itself (the GPU's bit-exact reduced-precision tests
    rest on this)."""
    rng = np.random.default_rng(5)
    x = rng.integers(0, 256, size=(500, 24)).astype(np.float32)
    q = rng.integers(0, 256, size=(9, 24)).astype(np.float32)
    for st in (oracle.STORAGE_F16, oracle.STORAGE_BF16):
        xs, qs, m = oracle.storage_inputs(x, q, 0, st)
        assert m == 0 and np.array_equal(xs, x) and np.array_equal(qs, q)
    xs, qs, m = oracle.storage_inputs(x, q, 2, oracle.STORAGE_BF16)
    assert m == 1 and np.array_equal(xs, oracle.round_bf16(oracle.normalize_rows(x)))


# ---- k-means oracle ------------------------------------------------------------

def test_mt19937_stream_known_answers():
    """The C++ standard fixes the 10000th output of a default-seeded mt19937
    (seed 5489) at 4123659995 ([rand.predef]); its first output is 3499211612."""
    r = oracle.MT19937Stream(5489)
    v = [r() for _ in range(10000)]
    assert v[0] == 3499211612 and v[-1] == 4123659995


def test_bounded_draw_rejects_the_biased_tail():
    """bounded(r) redraws u >= 2^32 - 2^32 mod r: with r = 3 the largest u
    (2^32 - 1) is rejected, the next draw 5 gives 5 mod 3."""
    seq = iter([2 ** 32 - 1, 5, 7])
    assert oracle.bounded(lambda: next(seq), 3) == 2
    seq = iter([2 ** 32 - 2, 1])
    assert oracle.bounded(lambda: next(seq), 3) == (2 ** 32 - 2) % 3
    r = oracle.MT19937Stream(1)
    draws = np.array([oracle.bounded(r, 7) for _ in range(70_000)])
    counts = np.bincount(draws, minlength=7)
    assert counts.size == 7 and np.all(np.abs(counts - 10_000) < 500)
    p = oracle.seed_permutation(1000, oracle.MT19937Stream(12345))
    assert np.array_equal(np.sort(p), np.arange(1000)) and not np.array_equal(p, np.arange(1000))


def test_kmeans_update_is_sequential_double_mean():
    rng = np.random.default_rng(8)
    pts = (rng.standard_normal((5000, 12)) * 100).astype(np.float32)
    a = rng.integers(0, 30, 5000).astype(np.int32)
    a[a == 7] = 8                                  # cell 7 empty -> reseeded from row 123
    reseed = np.full(30, -1, np.int32)
    reseed[7] = 123
    got = oracle.kmeans_update(pts, a, 30, np.zeros((30, 12), np.float32), reseed)
    for c in range(30):
        if c == 7:
            assert np.array_equal(got[c], pts[123])
            continue
        rows = pts[a == c].astype(np.float64)
        seq = np.cumsum(rows, axis=0)[-1]          # sequential, ascending index
        assert np.array_equal(got[c], (seq / rows.shape[0]).astype(np.float32))
    ints = rng.integers(-50, 50, size=(400, 5)).astype(np.float32)
    ai = (np.arange(400) % 4).astype(np.int32)
    m = oracle.kmeans_update(ints, ai, 4, np.zeros((4, 5), np.float32), np.full(4, -1, np.int32))
    for c in range(4):
        assert np.array_equal(m[c], (ints[ai == c].astype(np.float64).sum(0) / 100).astype(np.float32))
