# SPDX-License-Identifier: Apache-2.0
"""C ABI semantics that need no GPU (reference c/mflat.cpp:32-129 and
c/include/mflat.h:31-90): the library loads, exports every symbol the header
declares, and validates arguments exactly like the reference shell."""
import ctypes
import os
import re

import numpy as np
import pytest

import mflat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mflat.h")


def header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"MFLAT_API[^;(]*?\b(mflat_\w+)\s*\(", text)))


def test_loads_and_exports_every_declared_symbol():
    lib = mflat.load()
    syms = header_symbols()
    assert len(syms) >= 19, syms
    for s in syms:
        assert hasattr(lib, s), s
    assert set(syms) == set(mflat.SIGNATURES), set(syms) ^ set(mflat.SIGNATURES)


def test_dynamic_symbols_are_the_c_abi_only():
    """Like the reference's C library (hidden visibility, CMakeLists.txt:44-47),
    libmflat.so's dynamic symbol table holds the C ABI and nothing else: no
    kernel host stubs, no C++ internals."""
    import shutil
    import subprocess

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--defined-only", mflat.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    names = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    extra = sorted(n for n in names if not n.startswith("mflat_"))
    assert not extra, extra[:10]
    assert set(header_symbols()) <= names


def test_version_status_maxk():
    lib = mflat.load()
    assert lib.mflat_version() == b"0.1.0"
    assert lib.mflat_max_k() == 1024
    expect = {0: b"ok", 1: b"null argument", 2: b"bad argument", 3: b"allocation failed",
              4: b"index not ready", 5: b"internal error"}
    for k, v in expect.items():
        assert lib.mflat_status_str(k) == v
    assert lib.mflat_status_str(99) == b"unknown"


def test_create_arguments():
    lib = mflat.load()
    st = ctypes.c_int(-1)
    assert not lib.mflat_flat_create(0, 0, ctypes.byref(st)) and st.value == mflat.MFLAT_ERR_BAD_ARG
    assert not lib.mflat_flat_create(-3, 0, None)
    h = lib.mflat_flat_create(7, 42, ctypes.byref(st))   # unknown metric maps to L2
    assert h and st.value == 0
    assert lib.mflat_flat_dim(h) == 7 and lib.mflat_flat_size(h) == 0
    lib.mflat_flat_free(h)
    lib.mflat_flat_free(None)   # NULL is a no-op


def test_create_ex_storage_arguments():
    """Additive reduced-precision constructor: same checks as create, plus the
    storage type, which must be one of the three defined values."""
    lib = mflat.load()
    st = ctypes.c_int(-1)
    for bad in (-1, 3, 7):
        assert not lib.mflat_flat_create_ex(8, 0, bad, ctypes.byref(st)) and st.value == mflat.MFLAT_ERR_BAD_ARG
    assert not lib.mflat_flat_create_ex(0, 0, mflat.MFLAT_STORAGE_F16, ctypes.byref(st))
    assert st.value == mflat.MFLAT_ERR_BAD_ARG
    for storage in (mflat.MFLAT_STORAGE_F32, mflat.MFLAT_STORAGE_F16, mflat.MFLAT_STORAGE_BF16):
        h = lib.mflat_flat_create_ex(5, 1, storage, ctypes.byref(st))
        assert h and st.value == 0 and lib.mflat_flat_storage(h) == storage and lib.mflat_flat_dim(h) == 5
        lib.mflat_flat_free(h)
    h = lib.mflat_flat_create(5, 0, None)
    assert lib.mflat_flat_storage(h) == mflat.MFLAT_STORAGE_F32
    lib.mflat_flat_free(h)
    assert lib.mflat_flat_storage(None) == mflat.MFLAT_STORAGE_F32


def test_null_handles_and_arguments():
    lib = mflat.load()
    x = np.zeros((2, 4), np.float32)
    used = ctypes.c_int(-1)
    assert lib.mflat_flat_add(None, x.ctypes.data, 2) == mflat.MFLAT_ERR_NULL_ARG
    assert lib.mflat_flat_reset(None) == mflat.MFLAT_ERR_NULL_ARG
    assert lib.mflat_flat_search(None, x.ctypes.data, 1, 1, None, None, None) == mflat.MFLAT_ERR_NULL_ARG
    assert lib.mflat_flat_ready(None) == 0 and lib.mflat_flat_size(None) == 0 and lib.mflat_flat_dim(None) == 0
    h = lib.mflat_flat_create(4, 0, None)
    try:
        assert lib.mflat_flat_add(h, None, 2) == mflat.MFLAT_ERR_NULL_ARG
        assert lib.mflat_flat_add(h, x.ctypes.data, -1) == mflat.MFLAT_ERR_BAD_ARG
        assert lib.mflat_flat_add(h, x.ctypes.data, 0) == mflat.MFLAT_OK
        assert lib.mflat_flat_search(h, None, 1, 1, None, None, None) == mflat.MFLAT_ERR_NULL_ARG
        assert lib.mflat_flat_search(h, x.ctypes.data, -1, 1, None, None, None) == mflat.MFLAT_ERR_BAD_ARG
        assert lib.mflat_flat_search(h, x.ctypes.data, 1, 0, None, None, None) == mflat.MFLAT_ERR_BAD_ARG
        # m == 0: OK with k_used = 0 (reference c/mflat.cpp:44), before any device use
        assert lib.mflat_flat_search(h, x.ctypes.data, 0, 5, None, None, ctypes.byref(used)) == 0
        assert used.value == 0
        for fn in (lib.mflat_flat_search, lib.mflat_flat_search_i64):   # same checks on the int64-id entry
            assert fn(None, x.ctypes.data, 1, 1, None, None, None) == mflat.MFLAT_ERR_NULL_ARG
            assert fn(h, None, 1, 1, None, None, None) == mflat.MFLAT_ERR_NULL_ARG
            assert fn(h, x.ctypes.data, -1, 1, None, None, None) == mflat.MFLAT_ERR_BAD_ARG
            assert fn(h, x.ctypes.data, 1, 0, None, None, None) == mflat.MFLAT_ERR_BAD_ARG
            used.value = -1
            assert fn(h, x.ctypes.data, 0, 5, None, None, ctypes.byref(used)) == 0 and used.value == 0
        assert lib.mflat_flat_search_device(h, None, 1, 1, None, None, None, None) == mflat.MFLAT_ERR_NULL_ARG
        assert lib.mflat_flat_search_device(h, x.ctypes.data, 1, 0, None, None, None, None) == mflat.MFLAT_ERR_BAD_ARG
        assert lib.mflat_flat_add_device(h, x.ctypes.data, -2, None) == mflat.MFLAT_ERR_BAD_ARG
    finally:
        lib.mflat_flat_free(h)


def test_log_level_roundtrip_and_handler():
    lib = mflat.load()
    got = []

    @mflat.LOG_HANDLER_T
    def handler(level, msg, user):
        got.append((level, msg.decode(), user))

    old = lib.mflat_log_level()
    try:
        # out-of-range thresholds clamp to [INFO, OFF]
        lib.mflat_set_log_level(7)
        assert lib.mflat_log_level() == mflat.MFLAT_LOG_OFF
        lib.mflat_set_log_level(-3)
        assert lib.mflat_log_level() == mflat.MFLAT_LOG_INFO
        lib.mflat_set_log_level(mflat.MFLAT_LOG_WARN)
        assert lib.mflat_log_level() == mflat.MFLAT_LOG_WARN
        lib.mflat_set_log_handler(handler, ctypes.c_void_p(0x5EED))
        idx = mflat.FlatIndex(8)
        if idx.ready():
            pytest.skip("a GPU is present; the no-device message is not emitted")
        # no device: search fails loudly with NOT_READY and an error message
        idx.add(np.ones((3, 8), np.float32))
        assert idx.size() == 3
        with pytest.raises(mflat.MflatError) as e:
            idx.search(np.ones((1, 8), np.float32), 2)
        assert e.value.status == mflat.MFLAT_ERR_NOT_READY
        assert any(lv == mflat.MFLAT_LOG_ERROR and "HIP device" in m for lv, m, _ in got), got
        assert all(u == 0x5EED for _, _, u in got), got   # the registered user value, unchanged
        n = len(got)
        lib.mflat_set_log_level(mflat.MFLAT_LOG_OFF)
        with pytest.raises(mflat.MflatError):
            idx.search(np.ones((1, 8), np.float32), 2)
        assert len(got) == n            # Off silences everything
        idx.close()
    finally:
        lib.mflat_set_log_handler(ctypes.cast(None, mflat.LOG_HANDLER_T), None)
        lib.mflat_set_log_level(old)


def test_no_device_is_not_ready():
    idx = mflat.FlatIndex(16, mflat.MFLAT_METRIC_COSINE)
    if idx.ready():
        pytest.skip("a GPU is present")
    assert idx.ready() is False
    idx.add(np.ones((10, 16), np.float32))
    idx.reset()
    assert idx.size() == 0
    idx.close()


def test_profile_names():
    mflat.profile_reset()
    for name in ("scan_filter", "scan_sample", "scan_retry", "select", "argmin", "norms", "prep", "ivf_scan",
                 "ivf_bound"):
        ms, n = mflat.profile_read(name)
        assert ms == 0.0 and n == 0
    with pytest.raises(KeyError):
        mflat.profile_read("nope")


def test_kmeans_arguments():
    lib = mflat.load()
    x = np.zeros((10, 4), np.float32)
    c = np.zeros((3, 4), np.float32)
    used = ctypes.c_int(-1)
    f = lib.mflat_kmeans_train
    assert f(None, 10, 4, 3, 1, 0, c.ctypes.data, None, None, None, None) == mflat.MFLAT_ERR_NULL_ARG
    assert f(x.ctypes.data, 10, 4, 3, 1, 0, None, None, None, None, None) == mflat.MFLAT_ERR_NULL_ARG
    for n, d, nl, it, mpc in ((0, 4, 3, 1, 0), (10, 0, 3, 1, 0), (10, 4, 0, 1, 0), (10, 4, 3, -1, 0),
                              (10, 4, 3, 1, -5)):
        assert f(x.ctypes.data, n, d, nl, it, mpc, c.ctypes.data, None, None, None,
                 ctypes.byref(used)) == mflat.MFLAT_ERR_BAD_ARG
    rc = f(x.ctypes.data, 10, 4, 3, 1, 0, c.ctypes.data, None, None, None, ctypes.byref(used))
    idx = mflat.FlatIndex(4)
    if not idx.ready():
        assert rc == mflat.MFLAT_ERR_NOT_READY
    idx.close()


def test_ivf_arguments():
    """reference c/mflat.cpp:131-159: create / build / search checks, in that order."""
    lib = mflat.load()
    st = ctypes.c_int(-1)
    assert not lib.mflat_ivf_create(0, 0, 4, ctypes.byref(st)) and st.value == mflat.MFLAT_ERR_BAD_ARG
    assert not lib.mflat_ivf_create(8, 0, 0, ctypes.byref(st)) and st.value == mflat.MFLAT_ERR_BAD_ARG
    assert not lib.mflat_ivf_create_ex(8, 0, 4, 9, ctypes.byref(st)) and st.value == mflat.MFLAT_ERR_BAD_ARG
    lib.mflat_ivf_free(None)
    for f in (lib.mflat_ivf_ready, lib.mflat_ivf_size, lib.mflat_ivf_dim, lib.mflat_ivf_nlist):
        assert f(None) == 0
    h = lib.mflat_ivf_create(8, 42, 5, ctypes.byref(st))   # unknown metric maps to L2
    assert h and st.value == mflat.MFLAT_OK
    assert lib.mflat_ivf_ready(h) == 0 and lib.mflat_ivf_size(h) == 0
    assert lib.mflat_ivf_dim(h) == 8 and lib.mflat_ivf_nlist(h) == 5
    assert lib.mflat_ivf_storage(h) == mflat.MFLAT_STORAGE_F32
    x = np.zeros((3, 8), np.float32)
    used = ctypes.c_int(-1)
    assert lib.mflat_ivf_build(None, x.ctypes.data, 3) == mflat.MFLAT_ERR_NULL_ARG
    assert lib.mflat_ivf_build(h, None, 3) == mflat.MFLAT_ERR_NULL_ARG
    assert lib.mflat_ivf_build(h, x.ctypes.data, 0) == mflat.MFLAT_ERR_BAD_ARG
    s = lib.mflat_ivf_search
    assert s(None, x.ctypes.data, 1, 1, 1, None, None, None) == mflat.MFLAT_ERR_NULL_ARG
    assert s(h, None, 1, 1, 1, None, None, None) == mflat.MFLAT_ERR_NULL_ARG
    for m, k, npb in ((-1, 1, 1), (1, 0, 1), (1, 1, 0)):
        assert s(h, x.ctypes.data, m, k, npb, None, None, None) == mflat.MFLAT_ERR_BAD_ARG
    # not built: NOT_READY (even for m == 0, as the reference checks ready first)
    assert s(h, x.ctypes.data, 0, 1, 1, None, None, ctypes.byref(used)) == mflat.MFLAT_ERR_NOT_READY
    assert lib.mflat_ivf_probe(h, x.ctypes.data, 1, 1, x.ctypes.data) == mflat.MFLAT_ERR_NOT_READY
    assert lib.mflat_ivf_coarse(h, None, None, None) == mflat.MFLAT_ERR_NOT_READY
    assert lib.mflat_ivf_coarse(None, None, None, None) == mflat.MFLAT_ERR_NULL_ARG
    probe = mflat.FlatIndex(4)
    if not probe.ready():
        # no device: build fails loudly, nothing falls back to the CPU
        assert lib.mflat_ivf_build(h, x.ctypes.data, 3) == mflat.MFLAT_ERR_NOT_READY
        assert lib.mflat_ivf_ready(h) == 0
    probe.close()
    lib.mflat_ivf_free(h)
    hx = lib.mflat_ivf_create_ex(8, 1, 3, mflat.MFLAT_STORAGE_BF16, ctypes.byref(st))
    assert hx and lib.mflat_ivf_storage(hx) == mflat.MFLAT_STORAGE_BF16
    lib.mflat_ivf_free(hx)


def test_ivfpq_arguments():
    """reference c/mflat.cpp:161-198: create / build / search checks."""
    lib = mflat.load()
    st = ctypes.c_int(-1)
    for dim, metric, nl, m in ((0, 0, 4, 2), (8, 0, 0, 2), (8, 0, 4, 0), (8, 0, 4, 3),
                               (8, mflat.MFLAT_METRIC_INNER_PRODUCT, 4, 2), (256, 0, 4, 256)):
        assert not lib.mflat_ivfpq_create(dim, metric, nl, m, ctypes.byref(st)), (dim, metric, nl, m)
        assert st.value == mflat.MFLAT_ERR_BAD_ARG
    lib.mflat_ivfpq_free(None)
    lib.mflat_ivfpq_set_rerank(None, 1)
    for f in (lib.mflat_ivfpq_ready, lib.mflat_ivfpq_size, lib.mflat_ivfpq_dim, lib.mflat_ivfpq_nlist,
              lib.mflat_ivfpq_subquantizers):
        assert f(None) == 0
    h = lib.mflat_ivfpq_create(8, mflat.MFLAT_METRIC_COSINE, 6, 4, ctypes.byref(st))
    assert h and st.value == mflat.MFLAT_OK
    assert lib.mflat_ivfpq_ready(h) == 0 and lib.mflat_ivfpq_dim(h) == 8
    assert lib.mflat_ivfpq_nlist(h) == 6 and lib.mflat_ivfpq_subquantizers(h) == 4
    lib.mflat_ivfpq_set_rerank(h, 1)
    x = np.zeros((3, 8), np.float32)
    assert lib.mflat_ivfpq_build(None, x.ctypes.data, 3) == mflat.MFLAT_ERR_NULL_ARG
    assert lib.mflat_ivfpq_build(h, x.ctypes.data, 0) == mflat.MFLAT_ERR_BAD_ARG
    s = lib.mflat_ivfpq_search
    assert s(h, None, 1, 1, 1, 0, None, None, None) == mflat.MFLAT_ERR_NULL_ARG
    for m, k, npb, rr in ((-1, 1, 1, 0), (1, 0, 1, 0), (1, 1, 0, 0), (1, 1, 1, -1)):
        assert s(h, x.ctypes.data, m, k, npb, rr, None, None, None) == mflat.MFLAT_ERR_BAD_ARG
    assert s(h, x.ctypes.data, 1, 1, 1, 0, None, None, None) == mflat.MFLAT_ERR_NOT_READY
    assert lib.mflat_ivfpq_coarse(h, None, None, None, None, None) == mflat.MFLAT_ERR_NOT_READY
    probe = mflat.FlatIndex(4)
    if not probe.ready():
        assert lib.mflat_ivfpq_build(h, x.ctypes.data, 3) == mflat.MFLAT_ERR_NOT_READY
    probe.close()
    lib.mflat_ivfpq_free(h)
