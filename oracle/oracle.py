# SPDX-License-Identifier: Apache-2.0
"""TEST INFRASTRUCTURE ONLY: ctypes access to the CPU oracle (flat_oracle.c,
built into oracle/_build/liboracle.so) and, where it was built, to the
reference's own Distance.h primitives (oracle/_ref/libref_distance.so).

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use this
module, as the checker or as the timed CPU baseline -- never as the product.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int64, c_void_p

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(_HERE, "_build", "liboracle.so")
REF_SO = os.path.join(_HERE, "_ref", "libref_distance.so")

_o = None
_r = None


def lib():
    global _o
    if _o is None:
        if not os.path.exists(ORACLE_SO):
            raise FileNotFoundError(f"{ORACLE_SO} not built: run `make -C oracle`")
        o = ctypes.CDLL(ORACLE_SO)
        o.orc_dot.restype = c_float
        o.orc_dot.argtypes = [c_void_p, c_void_p, c_int]
        o.orc_sql2.restype = c_float
        o.orc_sql2.argtypes = [c_void_p, c_void_p, c_int]
        o.orc_row_sq_norms.restype = None
        o.orc_row_sq_norms.argtypes = [c_void_p, c_int64, c_int, c_void_p]
        o.orc_normalize_rows.restype = None
        o.orc_normalize_rows.argtypes = [c_void_p, c_int64, c_int]
        for name in ("orc_cpu_search", "orc_flat_search"):
            f = getattr(o, name)
            f.restype = c_int
            f.argtypes = [c_void_p, c_int64, c_int, c_int, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_int]
        o.orc_argmin_l2.restype = None
        o.orc_argmin_l2.argtypes = [c_void_p, c_int64, c_void_p, c_int64, c_int, c_void_p, c_void_p]
        o.orc_kmeans_update.restype = None
        o.orc_kmeans_update.argtypes = [c_void_p, c_int64, c_int, c_void_p, c_int, c_void_p, c_void_p]
        o.orc_ivf_search.restype = c_int
        o.orc_ivf_search.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_int64, c_void_p,
                                     c_int, c_int, c_void_p, c_void_p, c_int]
        o.orc_ivfpq_search.restype = c_int
        o.orc_ivfpq_search.argtypes = [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                       c_void_p, c_int64, c_void_p, c_int, c_int, c_void_p, c_void_p, c_int]
        o.orc_pq_rerank.restype = c_int
        o.orc_pq_rerank.argtypes = [c_void_p, c_int, c_int, c_void_p, c_int64, c_void_p, c_int, c_int, c_void_p,
                                    c_void_p]
        o.orc_brute_lex.restype = c_int
        o.orc_brute_lex.argtypes = [c_void_p, c_int64, c_int, c_void_p, c_int64, c_int, c_void_p, c_void_p]
        _o = o
    return _o


def ref_lib():
    """The reference's own primitives, or None when oracle/_ref was not built."""
    global _r
    if _r is None and os.path.exists(REF_SO):
        r = ctypes.CDLL(REF_SO)
        r.ref_dot.restype = c_float
        r.ref_dot.argtypes = [c_void_p, c_void_p, c_int]
        r.ref_sql2.restype = c_float
        r.ref_sql2.argtypes = [c_void_p, c_void_p, c_int]
        r.ref_row_sq_norms.restype = None
        r.ref_row_sq_norms.argtypes = [c_void_p, c_int, c_int, c_void_p]
        r.ref_normalize_rows.restype = None
        r.ref_normalize_rows.argtypes = [c_void_p, c_int, c_int]
        r.ref_score.restype = c_float
        r.ref_score.argtypes = [c_int, c_void_p, c_void_p, c_int]
        r.ref_score_to_value.restype = c_float
        r.ref_score_to_value.argtypes = [c_int, c_float]
        r.ref_empty_value.restype = c_float
        r.ref_empty_value.argtypes = [c_int]
        r.ref_l2_score_from_dot.restype = c_float
        r.ref_l2_score_from_dot.argtypes = [c_float, c_float, c_float]
        _r = r
    return _r


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def flat_search(db, q, k, metric=0, threads=1):
    """FlatIndex add+search semantics of the reference CPU path (unclamped k).
    Returns (ids int32 [m, k], values float32 [m, k])."""
    db = _f32(db)
    q = _f32(q)
    d = db.shape[1] if db.ndim == 2 and db.size else q.shape[1]
    nb = db.shape[0] if db.size else 0
    m = q.shape[0]
    ids = np.empty((m, k), dtype=np.int32)
    vals = np.empty((m, k), dtype=np.float32)
    rc = lib().orc_flat_search(db.ctypes.data, nb, d, metric, q.ctypes.data, m, k,
                               ids.ctypes.data, vals.ctypes.data, threads)
    if rc != 0:
        raise RuntimeError(f"orc_flat_search rc={rc}")
    return ids, vals


def row_sq_norms(v):
    v = _f32(v)
    out = np.empty(v.shape[0], dtype=np.float32)
    lib().orc_row_sq_norms(v.ctypes.data, v.shape[0], v.shape[1], out.ctypes.data)
    return out


def normalize_rows(v):
    v = _f32(v).copy()
    lib().orc_normalize_rows(v.ctypes.data, v.shape[0], v.shape[1])
    return v


def argmin_l2(pts, cents):
    pts = _f32(pts)
    cents = _f32(cents)
    ids = np.empty(pts.shape[0], dtype=np.int32)
    d = np.empty(pts.shape[0], dtype=np.float32)
    lib().orc_argmin_l2(pts.ctypes.data, pts.shape[0], cents.ctypes.data, cents.shape[0],
                        pts.shape[1], ids.ctypes.data, d.ctypes.data)
    return ids, d


def brute_lex(db, q, k):
    db = _f32(db)
    q = _f32(q)
    ids = np.empty((q.shape[0], k), dtype=np.int32)
    vals = np.empty((q.shape[0], k), dtype=np.float32)
    lib().orc_brute_lex(db.ctypes.data, db.shape[0], db.shape[1], q.ctypes.data, q.shape[0], k,
                        ids.ctypes.data, vals.ctypes.data)
    return ids, vals


# ---- reduced-precision storage (fp16 / bf16) --------------------------------
# The reference stores fp32 only; the library's fp16 / bf16 storage variants are
# checked against this oracle run on identically rounded inputs: the fp32
# values rounded to nearest even (after the Cosine normalisation, in fp32),
# then searched exactly in fp32.

STORAGE_F32, STORAGE_F16, STORAGE_BF16 = 0, 1, 2


def round_f16(x):
    """fp32 -> IEEE binary16 (numpy's round-to-nearest-even cast) -> fp32."""
    with np.errstate(over="ignore"):
        return _f32(x).astype(np.float16).astype(np.float32)


def round_bf16(x):
    """fp32 -> bfloat16, round to nearest even on the upper 16 bits of the
    pattern; NaN -> the quiet NaN 0x7fc0 -> fp32."""
    x = _f32(x)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    r[np.isnan(x)] = 0x7FC0
    return (r << 16).astype(np.uint32).view(np.float32).reshape(x.shape)


def round_storage(x, storage):
    if storage == STORAGE_F32:
        return _f32(x)
    if storage == STORAGE_F16:
        return round_f16(x)
    if storage == STORAGE_BF16:
        return round_bf16(x)
    raise ValueError(storage)


def storage_inputs(db, q, metric, storage):
    """(db', q', metric') such that flat_search(db', q', k, metric') is the
    exact answer for an index of this storage type: Cosine rows and queries are
    normalised (reference rule) before rounding and then compared by dot."""
    if metric == 2:
        return (round_storage(normalize_rows(db), storage), round_storage(normalize_rows(q), storage), 1)
    return round_storage(db, storage), round_storage(q, storage), metric


# ---- k-means training (the device k-means loop's checker) --------------------
# Restates the loop of the reference's CoarseQuantizer::train over
# detail::kmeansGpu (src/CoarseQuantizer.mm:104-159, src/Internal.h:234-382)
# with the scalar update of src/CoarseQuantizer.mm:44-66, and the library's
# documented seeding shuffle (the reference's std::shuffle draws are specific to
# its standard library).

class MT19937Stream:
    """Raw 32-bit outputs of std::mt19937(seed): numpy's legacy RandomState with
    an integer seed is the same generator (pinned against the standard's known
    answer in tests/test_oracle.py)."""

    def __init__(self, seed):
        self._rs = np.random.RandomState(seed)
        self._buf = np.empty(0, np.uint32)
        self._pos = 0

    def __call__(self):
        if self._pos == self._buf.size:
            self._buf = np.frombuffer(self._rs.bytes(4 * 4096), dtype="<u4")
            self._pos = 0
        v = int(self._buf[self._pos])
        self._pos += 1
        return v


def bounded(rng, r):
    """Uniform in [0, r): redraw while u >= 2^32 - 2^32 mod r, then u mod r."""
    lim = (1 << 32) - ((1 << 32) % r)
    while True:
        u = rng()
        if u < lim:
            return u % r


def seed_permutation(n, rng):
    """Fisher-Yates from the top with bounded() draws."""
    perm = list(range(n))
    for i in range(n - 1, 0, -1):
        j = bounded(rng, i + 1)
        perm[i], perm[j] = perm[j], perm[i]
    return np.array(perm, dtype=np.int64)


def kmeans_update(pts, assign, nlist, cent, reseed):
    pts = _f32(pts)
    assign = np.ascontiguousarray(assign, np.int32)
    reseed = np.ascontiguousarray(reseed, np.int32)
    out = _f32(cent).copy()
    lib().orc_kmeans_update(pts.ctypes.data, pts.shape[0], pts.shape[1], assign.ctypes.data, nlist,
                            reseed.ctypes.data, out.ctypes.data)
    return out


def kmeans_train(points, nlist, iters, max_points_per_centroid=256, wrap=False):
    """Returns (centroids, assign, cell_start, order) as the library's
    mflat_kmeans_train defines them. wrap: nlist stays as given above n, seed c
    being point perm[c mod n] (the PQ sub-quantizers' 256 cells,
    src/Internal.h:241-248)."""
    points = _f32(points)
    n, d = points.shape
    nlist = nlist if wrap else min(nlist, n)
    rng = MT19937Stream(12345)
    perm = seed_permutation(n, rng)
    cent = points[perm[np.arange(nlist) % n]].copy()
    train_n = n
    if max_points_per_centroid > 0 and max_points_per_centroid * nlist < n:
        train_n = max_points_per_centroid * nlist
    train = points[perm[:train_n]].copy() if train_n < n else points
    for _ in range(iters):
        a, _ = argmin_l2(train, cent)
        counts = np.bincount(a, minlength=nlist)
        reseed = np.array([rng() % train_n if counts[c] == 0 else -1 for c in range(nlist)], np.int32)
        cent = kmeans_update(train, a, nlist, cent, reseed)
    a, _ = argmin_l2(points, cent)
    counts = np.bincount(a, minlength=nlist)
    start = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    order = np.argsort(a, kind="stable").astype(np.int32)
    return cent, a.astype(np.int32), start, order


# ---- IVF (the inverted-file index's checker) ----------------------------------
# Restates the reference's IvfIndex build and two-stage search: the coarse layer
# of CoarseQuantizer::train (src/CoarseQuantizer.mm:104-159), its CSR
# (:134-143), the CPU probe (probeCellsCpu, :190-197) and searchCpu
# (src/IvfIndex.mm:518-560) over the probed cells.

IVF_TRAIN_ITERS = 12            # src/IvfIndex.mm:493
IVF_POINTS_PER_CENTROID = 256   # src/CoarseQuantizer.mm:116-117


def ivf_csr(assign, nlist):
    """Cell histogram -> prefix sum -> stable slot permutation
    (src/CoarseQuantizer.mm:134-143): (cell_start [nlist + 1], reordered_ids [n])."""
    assign = np.asarray(assign, np.int64)
    start = np.zeros(nlist + 1, np.int64)
    for a in assign:
        start[a + 1] += 1
    start = np.cumsum(start)
    cursor = start[:-1].copy()
    rid = np.empty(assign.size, np.int32)
    for i, a in enumerate(assign):
        rid[cursor[a]] = i
        cursor[a] += 1
    return start.astype(np.int32), rid


def ivf_build(db, nlist, metric=0):
    """(centroids, cell_start, reordered_ids) of IvfIndex::build on the
    library's k-means (kmeans_train above): Cosine rows are normalised first."""
    db = normalize_rows(db) if metric == 2 else _f32(db)
    cent, assign, _, _ = kmeans_train(db, nlist, IVF_TRAIN_ITERS, IVF_POINTS_PER_CENTROID)
    start, rid = ivf_csr(assign, cent.shape[0])
    return cent, start, rid


def ivf_probe(cent, q, nprobe, metric=0):
    """probeCellsCpu: the nprobe cells of smallest (sqL2(q, centroid), cell),
    nearest first (src/CoarseQuantizer.mm:190-197) -- cpuSearch over the
    centroids under L2 keeps the same order (strict '>' keeps the lower cell on
    ties). Cosine queries are normalised first (src/IvfIndex.mm:773-780)."""
    q = normalize_rows(q) if metric == 2 else _f32(q)
    nprobe = max(1, min(int(nprobe), cent.shape[0]))
    ids, _ = flat_search(cent, q, nprobe, 0)
    return ids


def ivf_payload(db, rid, metric=0):
    """The rows in cell order (the reference's reorderedDb), Cosine-normalised."""
    db = normalize_rows(db) if metric == 2 else _f32(db)
    return np.ascontiguousarray(db[np.asarray(rid, np.int64)]) if db.size else db


def ivf_search(db, cell_start, rid, q, k, probed, metric=0, threads=1, payload=None):
    """searchCpu over the given probed cells: (ids [m, k], values [m, k]).
    db: the caller's rows (row-major, original order); Cosine rows and
    queries are normalised and ranked by the dot product. payload: a
    precomputed ivf_payload(db, rid, metric) (db is then unused)."""
    q = _f32(q)
    rid = np.ascontiguousarray(rid, np.int32)
    rdb = ivf_payload(db, rid, metric) if payload is None else payload
    if metric == 2:
        q = normalize_rows(q)
        metric = 1
    start = np.ascontiguousarray(cell_start, np.int32)
    probed = np.ascontiguousarray(probed, np.int32)
    m, d = q.shape
    ids = np.empty((m, k), np.int32)
    vals = np.empty((m, k), np.float32)
    rc = lib().orc_ivf_search(rdb.ctypes.data, rid.ctypes.data, start.ctypes.data, d, metric, q.ctypes.data, m,
                              probed.ctypes.data, probed.shape[1], k, ids.ctypes.data, vals.ctypes.data, threads)
    if rc != 0:
        raise RuntimeError(f"orc_ivf_search rc={rc}")
    return ids, vals


# ---- IVF-PQ (the compressed index's checker) ----------------------------------
# Restates IvfPqIndex's build (src/IvfPqIndex.mm:286-340: coarse cells as IVF,
# residual PQ with 256-cell k-means per sub-space over all rows, codes = the
# final assignments) and its CPU search (:383-445) and rerank (:598-625).

PQ_KSUB = 256


def pq_train(residuals, M, iters=IVF_TRAIN_ITERS):
    """(pqc [M, 256, dsub], codes [n, M] uint8 in row order): k-means of each
    sub-space (every row trains; seeds wrap when n < 256)."""
    r = _f32(residuals)
    n, d = r.shape
    dsub = d // M
    pqc = np.empty((M, PQ_KSUB, dsub), np.float32)
    codes = np.empty((n, M), np.uint8)
    for mm in range(M):
        sub = np.ascontiguousarray(r[:, mm * dsub:(mm + 1) * dsub])
        c, a, _, _ = kmeans_train(sub, PQ_KSUB, iters, 0, wrap=True)
        pqc[mm] = c
        codes[:, mm] = a
    return pqc, codes


def ivfpq_search(cent, cell_start, rid, codes_cell, pqc, q, k, probed, metric=0, threads=1):
    """searchCpu of the residual IVF-PQ index over given probed cells: ids and
    ADC distances [m, k]. codes_cell: n x M codes in cell order."""
    q = normalize_rows(q) if metric == 2 else _f32(q)
    cent = _f32(cent)
    pqc = _f32(pqc)
    M = pqc.shape[0]
    codes_cell = np.ascontiguousarray(codes_cell, np.uint8)
    start = np.ascontiguousarray(cell_start, np.int32)
    rid = np.ascontiguousarray(rid, np.int32)
    probed = np.ascontiguousarray(probed, np.int32)
    m, d = q.shape
    ids = np.empty((m, k), np.int32)
    vals = np.empty((m, k), np.float32)
    rc = lib().orc_ivfpq_search(cent.ctypes.data, cent.shape[0], start.ctypes.data, rid.ctypes.data,
                                codes_cell.ctypes.data, pqc.ctypes.data, M, d, q.ctypes.data, m, probed.ctypes.data,
                                probed.shape[1], k, ids.ctypes.data, vals.ctypes.data, threads)
    if rc != 0:
        raise RuntimeError(f"orc_ivfpq_search rc={rc}")
    return ids, vals


def pq_rerank(full, q, short_ids, k, metric=0):
    """Exact rerank of a shortlist (metric 0 L2, 2 Cosine: rows and queries
    normalised, ranked by dot)."""
    full = normalize_rows(full) if metric == 2 else _f32(full)
    q = normalize_rows(q) if metric == 2 else _f32(q)
    short_ids = np.ascontiguousarray(short_ids, np.int32)
    m, d = q.shape
    ids = np.empty((m, k), np.int32)
    vals = np.empty((m, k), np.float32)
    rc = lib().orc_pq_rerank(full.ctypes.data, d, 0 if metric == 0 else 1, q.ctypes.data, m, short_ids.ctypes.data,
                             short_ids.shape[1], k, ids.ctypes.data, vals.ctypes.data)
    if rc != 0:
        raise RuntimeError(f"orc_pq_rerank rc={rc}")
    return ids, vals
