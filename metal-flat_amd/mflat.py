# SPDX-License-Identifier: Apache-2.0
"""ctypes binding of libmflat.so (the C ABI declared in include/mflat.h).

This is the binding a Python caller of the reference's C ABI
(c/include/mflat.h) would write: opaque handle, status codes, caller-owned
output arrays. It loads the in-tree build at metal-flat_amd/lib/libmflat.so and
raises if it is missing -- there is no other implementation behind it.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_longlong, c_void_p

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libmflat.so")

MFLAT_METRIC_L2 = 0
MFLAT_METRIC_INNER_PRODUCT = 1
MFLAT_METRIC_COSINE = 2

MFLAT_STORAGE_F32 = 0
MFLAT_STORAGE_F16 = 1
MFLAT_STORAGE_BF16 = 2
STORAGE_NAMES = {"f32": MFLAT_STORAGE_F32, "f16": MFLAT_STORAGE_F16, "bf16": MFLAT_STORAGE_BF16}

MFLAT_OK = 0
MFLAT_ERR_NULL_ARG = 1
MFLAT_ERR_BAD_ARG = 2
MFLAT_ERR_ALLOC = 3
MFLAT_ERR_NOT_READY = 4
MFLAT_ERR_INTERNAL = 5

MFLAT_LOG_INFO, MFLAT_LOG_WARN, MFLAT_LOG_ERROR, MFLAT_LOG_OFF = 0, 1, 2, 3

LOG_HANDLER_T = ctypes.CFUNCTYPE(None, c_int, c_char_p, c_void_p)

# Every symbol include/mflat.h declares, with its ctypes signature.
SIGNATURES = {
    "mflat_version": (c_char_p, []),
    "mflat_status_str": (c_char_p, [c_int]),
    "mflat_max_k": (c_int, []),
    "mflat_set_log_handler": (None, [LOG_HANDLER_T, c_void_p]),
    "mflat_set_log_level": (None, [c_int]),
    "mflat_log_level": (c_int, []),
    "mflat_flat_create": (c_void_p, [c_int, c_int, POINTER(c_int)]),
    "mflat_flat_create_ex": (c_void_p, [c_int, c_int, c_int, POINTER(c_int)]),
    "mflat_flat_storage": (c_int, [c_void_p]),
    "mflat_flat_free": (None, [c_void_p]),
    "mflat_flat_ready": (c_int, [c_void_p]),
    "mflat_flat_size": (c_int, [c_void_p]),
    "mflat_flat_dim": (c_int, [c_void_p]),
    "mflat_flat_add": (c_int, [c_void_p, c_void_p, c_int]),
    "mflat_flat_reset": (c_int, [c_void_p]),
    "mflat_flat_search": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, POINTER(c_int)]),
    "mflat_flat_search_i64": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, POINTER(c_int)]),
    "mflat_flat_search_device": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p,
                                         POINTER(c_int), c_void_p]),
    "mflat_flat_search_device_noalloc": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p,
                                                 POINTER(c_int), c_void_p]),
    "mflat_flat_add_device": (c_int, [c_void_p, c_void_p, c_int, c_void_p]),
    "mflat_kmeans_train": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                                   c_void_p, c_void_p, POINTER(c_int)]),
    "mflat_ivf_create": (c_void_p, [c_int, c_int, c_int, POINTER(c_int)]),
    "mflat_ivf_create_ex": (c_void_p, [c_int, c_int, c_int, c_int, POINTER(c_int)]),
    "mflat_ivf_free": (None, [c_void_p]),
    "mflat_ivf_ready": (c_int, [c_void_p]),
    "mflat_ivf_size": (c_int, [c_void_p]),
    "mflat_ivf_dim": (c_int, [c_void_p]),
    "mflat_ivf_nlist": (c_int, [c_void_p]),
    "mflat_ivf_storage": (c_int, [c_void_p]),
    "mflat_ivf_build": (c_int, [c_void_p, c_void_p, c_int]),
    "mflat_ivf_search": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, POINTER(c_int)]),
    "mflat_ivf_search_device": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p,
                                        POINTER(c_int), c_void_p]),
    "mflat_ivf_probe": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "mflat_ivf_coarse": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p]),
    "mflat_ivfpq_create": (c_void_p, [c_int, c_int, c_int, c_int, POINTER(c_int)]),
    "mflat_ivfpq_free": (None, [c_void_p]),
    "mflat_ivfpq_set_rerank": (None, [c_void_p, c_int]),
    "mflat_ivfpq_ready": (c_int, [c_void_p]),
    "mflat_ivfpq_size": (c_int, [c_void_p]),
    "mflat_ivfpq_dim": (c_int, [c_void_p]),
    "mflat_ivfpq_nlist": (c_int, [c_void_p]),
    "mflat_ivfpq_subquantizers": (c_int, [c_void_p]),
    "mflat_ivfpq_build": (c_int, [c_void_p, c_void_p, c_int]),
    "mflat_ivfpq_search": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                                   POINTER(c_int)]),
    "mflat_ivfpq_search_device": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                                          POINTER(c_int), c_void_p]),
    "mflat_ivfpq_probe": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "mflat_ivfpq_coarse": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "mflat_profile_enable": (None, [c_int]),
    "mflat_profile_reset": (None, []),
    "mflat_profile_read": (c_int, [c_char_p, POINTER(c_double), POINTER(c_longlong)]),
}

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libmflat.so once; raises FileNotFoundError if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} not built: run `make -C metal-flat_amd` "
                                "(or __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class MflatError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        msg = load().mflat_status_str(status).decode()
        super().__init__(f"{what}: status {status} ({msg})")


def _check(status: int, what: str) -> None:
    if status != MFLAT_OK:
        raise MflatError(status, what)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class FlatIndex:
    """Python view of one mflat_flat_index_t (reference FlatIndex.h:37-77)."""

    def __init__(self, dim: int, metric: int = MFLAT_METRIC_L2, storage: int = MFLAT_STORAGE_F32):
        """storage: MFLAT_STORAGE_F32 (the reference's mflat_flat_create) or a
        reduced-precision type (mflat_flat_create_ex)."""
        lib = load()
        st = c_int(-1)
        if storage == MFLAT_STORAGE_F32:
            self._h = lib.mflat_flat_create(int(dim), int(metric), ctypes.byref(st))
        else:
            self._h = lib.mflat_flat_create_ex(int(dim), int(metric), int(storage), ctypes.byref(st))
        if not self._h:
            raise MflatError(st.value, "mflat_flat_create")
        self.dim = int(dim)
        self.metric = int(metric)
        self.storage = int(storage)

    def close(self) -> None:
        if getattr(self, "_h", None):
            load().mflat_flat_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self):
        return self._h

    def ready(self) -> bool:
        return load().mflat_flat_ready(self._h) == 1

    def size(self) -> int:
        return load().mflat_flat_size(self._h)

    def add(self, vectors) -> None:
        v = _f32(vectors).reshape(-1, self.dim)
        _check(load().mflat_flat_add(self._h, v.ctypes.data, v.shape[0]), "mflat_flat_add")

    def reset(self) -> None:
        _check(load().mflat_flat_reset(self._h), "mflat_flat_reset")

    def search(self, queries, k: int):
        """Returns (ids int32 [m, k_used], distances float32 [m, k_used], k_used)."""
        q = _f32(queries).reshape(-1, self.dim)
        m = q.shape[0]
        kk = max(1, min(int(k), load().mflat_max_k()))
        ids = np.full((max(m, 1), kk), -7, dtype=np.int32)
        dist = np.full((max(m, 1), kk), np.nan, dtype=np.float32)
        used = c_int(-1)
        _check(load().mflat_flat_search(self._h, q.ctypes.data, m, int(k), ids.ctypes.data,
                                         dist.ctypes.data, ctypes.byref(used)), "mflat_flat_search")
        ku = used.value
        if m > 0 and ku == kk:   # every column produced: the buffers are the result
            return ids, dist, ku
        flat_i = ids.reshape(-1)[: m * ku].reshape(m, ku)
        flat_d = dist.reshape(-1)[: m * ku].reshape(m, ku)
        return flat_i.copy(), flat_d.copy(), ku

    def search_i64(self, queries, k: int):
        """mflat_flat_search_i64: as search, ids int64."""
        q = _f32(queries).reshape(-1, self.dim)
        m = q.shape[0]
        kk = max(1, min(int(k), load().mflat_max_k()))
        ids = np.full((max(m, 1), kk), -7, dtype=np.int64)
        dist = np.full((max(m, 1), kk), np.nan, dtype=np.float32)
        used = c_int(-1)
        _check(load().mflat_flat_search_i64(self._h, q.ctypes.data, m, int(k), ids.ctypes.data,
                                             dist.ctypes.data, ctypes.byref(used)), "mflat_flat_search_i64")
        ku = used.value
        return (ids.reshape(-1)[: m * ku].reshape(m, ku).copy(),
                dist.reshape(-1)[: m * ku].reshape(m, ku).copy(), ku)

    # ---- device-pointer entry points ----
    # x / q / outputs: any object with .data_ptr() and .shape holding contiguous
    # device memory of the index's GPU (hipmem.DeviceArray, or a torch tensor
    # when torch shares the process -- see hipmem's note on runtimes).
    def add_device(self, x, stream=None) -> None:
        _check(load().mflat_flat_add_device(self._h, x.data_ptr(), x.shape[0],
                                            _stream_ptr(stream)), "mflat_flat_add_device")

    def search_device(self, q, k: int, out_ids, out_dist, stream=None) -> int:
        used = c_int(-1)
        _check(load().mflat_flat_search_device(
            self._h, q.data_ptr(), q.shape[0], int(k),
            out_ids.data_ptr() if out_ids is not None else None,
            out_dist.data_ptr() if out_dist is not None else None,
            ctypes.byref(used), _stream_ptr(stream)), "mflat_flat_search_device")
        return used.value

    def search_device_noalloc(self, q, k: int, out_ids, out_dist, stream=None) -> int:
        """mflat_flat_search_device_noalloc: stream-ordered (synchronise the
        stream before reading the outputs); m <= 16, k <= 32, dim <= 992 (fp32)
        or 2016 (fp16 / bf16)."""
        used = c_int(-1)
        _check(load().mflat_flat_search_device_noalloc(
            self._h, q.data_ptr(), q.shape[0], int(k),
            out_ids.data_ptr() if out_ids is not None else None,
            out_dist.data_ptr() if out_dist is not None else None,
            ctypes.byref(used), _stream_ptr(stream)), "mflat_flat_search_device_noalloc")
        return used.value


class IvfIndex:
    """Python view of one mflat_ivf_index_t (reference IvfIndex.h:29-62)."""

    def __init__(self, dim: int, metric: int = MFLAT_METRIC_L2, nlist: int = 64,
                 storage: int = MFLAT_STORAGE_F32):
        lib = load()
        st = c_int(-1)
        if storage == MFLAT_STORAGE_F32:
            self._h = lib.mflat_ivf_create(int(dim), int(metric), int(nlist), ctypes.byref(st))
        else:
            self._h = lib.mflat_ivf_create_ex(int(dim), int(metric), int(nlist), int(storage), ctypes.byref(st))
        if not self._h:
            raise MflatError(st.value, "mflat_ivf_create")
        self.dim = int(dim)
        self.metric = int(metric)
        self.storage = int(storage)

    def close(self) -> None:
        if getattr(self, "_h", None):
            load().mflat_ivf_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self):
        return self._h

    def ready(self) -> bool:
        return load().mflat_ivf_ready(self._h) == 1

    def size(self) -> int:
        return load().mflat_ivf_size(self._h)

    def nlist(self) -> int:
        return load().mflat_ivf_nlist(self._h)

    def build(self, vectors) -> None:
        v = _f32(vectors).reshape(-1, self.dim)
        _check(load().mflat_ivf_build(self._h, v.ctypes.data, v.shape[0]), "mflat_ivf_build")

    def search(self, queries, k: int, nprobe: int):
        """Returns (ids int32 [m, k_used], distances float32 [m, k_used], k_used)."""
        q = _f32(queries).reshape(-1, self.dim)
        m = q.shape[0]
        kk = max(1, min(int(k), load().mflat_max_k()))
        ids = np.full((max(m, 1), kk), -7, dtype=np.int32)
        dist = np.full((max(m, 1), kk), np.nan, dtype=np.float32)
        used = c_int(-1)
        _check(load().mflat_ivf_search(self._h, q.ctypes.data, m, int(k), int(nprobe), ids.ctypes.data,
                                        dist.ctypes.data, ctypes.byref(used)), "mflat_ivf_search")
        ku = used.value
        return (ids.reshape(-1)[: m * ku].reshape(m, ku).copy(),
                dist.reshape(-1)[: m * ku].reshape(m, ku).copy(), ku)

    def search_device(self, q, k: int, nprobe: int, out_ids, out_dist, stream=None) -> int:
        used = c_int(-1)
        _check(load().mflat_ivf_search_device(
            self._h, q.data_ptr(), q.shape[0], int(k), int(nprobe),
            out_ids.data_ptr() if out_ids is not None else None,
            out_dist.data_ptr() if out_dist is not None else None,
            ctypes.byref(used), _stream_ptr(stream)), "mflat_ivf_search_device")
        return used.value

    def probe(self, queries, nprobe: int) -> np.ndarray:
        """The m x nprobe nearest cells (nprobe clamped to [1, nlist]), nearest first."""
        q = _f32(queries).reshape(-1, self.dim)
        m = q.shape[0]
        npb = max(1, min(int(nprobe), self.nlist()))
        cells = np.full((max(m, 1), npb), -7, dtype=np.int32)
        _check(load().mflat_ivf_probe(self._h, q.ctypes.data, m, int(nprobe), cells.ctypes.data), "mflat_ivf_probe")
        return cells[:m].copy()

    def coarse(self):
        """(centroids [nlist, dim] float32, cell_start [nlist + 1] int32,
        reordered_ids [size] int32) of a built index."""
        nl, n = self.nlist(), self.size()
        cent = np.empty((nl, self.dim), np.float32)
        start = np.empty(nl + 1, np.int32)
        rid = np.empty(max(n, 1), np.int32)
        _check(load().mflat_ivf_coarse(self._h, cent.ctypes.data, start.ctypes.data, rid.ctypes.data),
               "mflat_ivf_coarse")
        return cent, start, rid[:n]


class IvfPqIndex:
    """Python view of one mflat_ivfpq_index_t (reference IvfPqIndex.h:37-99)."""

    def __init__(self, dim: int, metric: int = MFLAT_METRIC_L2, nlist: int = 64, m_sub: int = 8,
                 rerank: bool = False):
        lib = load()
        st = c_int(-1)
        self._h = lib.mflat_ivfpq_create(int(dim), int(metric), int(nlist), int(m_sub), ctypes.byref(st))
        if not self._h:
            raise MflatError(st.value, "mflat_ivfpq_create")
        if rerank:
            lib.mflat_ivfpq_set_rerank(self._h, 1)
        self.dim = int(dim)
        self.metric = int(metric)
        self.m_sub = int(m_sub)

    def close(self) -> None:
        if getattr(self, "_h", None):
            load().mflat_ivfpq_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self):
        return self._h

    def ready(self) -> bool:
        return load().mflat_ivfpq_ready(self._h) == 1

    def size(self) -> int:
        return load().mflat_ivfpq_size(self._h)

    def nlist(self) -> int:
        return load().mflat_ivfpq_nlist(self._h)

    def build(self, vectors) -> None:
        v = _f32(vectors).reshape(-1, self.dim)
        _check(load().mflat_ivfpq_build(self._h, v.ctypes.data, v.shape[0]), "mflat_ivfpq_build")

    def search(self, queries, k: int, nprobe: int, rerank: int = 0):
        """Returns (ids int32 [m, k_used], distances float32 [m, k_used], k_used)."""
        q = _f32(queries).reshape(-1, self.dim)
        m = q.shape[0]
        kk = max(1, min(int(k), load().mflat_max_k()))
        ids = np.full((max(m, 1), kk), -7, dtype=np.int32)
        dist = np.full((max(m, 1), kk), np.nan, dtype=np.float32)
        used = c_int(-1)
        _check(load().mflat_ivfpq_search(self._h, q.ctypes.data, m, int(k), int(nprobe), int(rerank),
                                          ids.ctypes.data, dist.ctypes.data, ctypes.byref(used)),
               "mflat_ivfpq_search")
        ku = used.value
        return (ids.reshape(-1)[: m * ku].reshape(m, ku).copy(),
                dist.reshape(-1)[: m * ku].reshape(m, ku).copy(), ku)

    def search_device(self, q, k: int, nprobe: int, out_ids, out_dist, rerank: int = 0, stream=None) -> int:
        used = c_int(-1)
        _check(load().mflat_ivfpq_search_device(
            self._h, q.data_ptr(), q.shape[0], int(k), int(nprobe), int(rerank),
            out_ids.data_ptr() if out_ids is not None else None,
            out_dist.data_ptr() if out_dist is not None else None,
            ctypes.byref(used), _stream_ptr(stream)), "mflat_ivfpq_search_device")
        return used.value

    def probe(self, queries, nprobe: int) -> np.ndarray:
        q = _f32(queries).reshape(-1, self.dim)
        m = q.shape[0]
        npb = max(1, min(int(nprobe), self.nlist()))
        cells = np.full((max(m, 1), npb), -7, dtype=np.int32)
        _check(load().mflat_ivfpq_probe(self._h, q.ctypes.data, m, int(nprobe), cells.ctypes.data),
               "mflat_ivfpq_probe")
        return cells[:m].copy()

    def coarse(self):
        """(centroids [nlist, dim], cell_start [nlist + 1], reordered_ids [n],
        pq_centroids [m_sub, 256, dim / m_sub], codes [n, m_sub] in cell order)."""
        nl, n, M = self.nlist(), self.size(), self.m_sub
        cent = np.empty((nl, self.dim), np.float32)
        start = np.empty(nl + 1, np.int32)
        rid = np.empty(max(n, 1), np.int32)
        pqc = np.empty((M, 256, self.dim // M), np.float32)
        codes = np.empty((max(n, 1), M), np.uint8)
        _check(load().mflat_ivfpq_coarse(self._h, cent.ctypes.data, start.ctypes.data, rid.ctypes.data,
                                         pqc.ctypes.data, codes.ctypes.data), "mflat_ivfpq_coarse")
        return cent, start, rid[:n], pqc, codes[:n]


def kmeans_train(points, nlist: int, iters: int, max_points_per_centroid: int = 256):
    """mflat_kmeans_train: returns (centroids [nlist_used, dim] float32,
    assign [n] int32, cell_start [nlist_used + 1] int32, order [n] int32)."""
    x = _f32(points)
    n, d = x.shape
    nl = min(int(nlist), n)
    cent = np.empty((max(int(nlist), 1), d), np.float32)
    assign = np.empty(n, np.int32)
    start = np.empty(max(int(nlist), 1) + 1, np.int32)
    order = np.empty(n, np.int32)
    used = c_int(-1)
    _check(load().mflat_kmeans_train(x.ctypes.data, n, d, int(nlist), int(iters), int(max_points_per_centroid),
                                     cent.ctypes.data, assign.ctypes.data, start.ctypes.data, order.ctypes.data,
                                     ctypes.byref(used)), "mflat_kmeans_train")
    assert used.value == nl
    return cent[:nl].copy(), assign, start[: nl + 1].copy(), order


def _stream_ptr(stream):
    if stream is None:
        return None
    return ctypes.c_void_p(int(getattr(stream, "cuda_stream", stream)))


def profile_enable(on: bool) -> None:
    load().mflat_profile_enable(1 if on else 0)


def profile_reset() -> None:
    load().mflat_profile_reset()


def profile_read(name: str):
    ms, n = c_double(0.0), c_longlong(0)
    rc = load().mflat_profile_read(name.encode(), ctypes.byref(ms), ctypes.byref(n))
    if rc != 0:
        raise KeyError(name)
    return ms.value, n.value
