// SPDX-License-Identifier: Apache-2.0
// mflat_abi.cpp -- the C ABI (include/mflat.h) over the engine.
//
// Behaviour of the reference's c/mflat.cpp:32-129: an opaque handle wrapping
// the engine plus a std::mutex that serialises add / reset / search per handle;
// every entry point is a try/catch that maps exceptions to status codes;
// results are copied into caller-owned buffers with row stride k_used.
#include <algorithm>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "../../include/mflat.h"
#include "flat_index.hpp"
#include "ivf_index.hpp"
#include "kmeans.hpp"
#include "log.hpp"

using mflat_amd::FlatIndex;
using mflat_amd::Metric;

namespace mflat_amd {
void prof_enable(int on);
void prof_reset();
int prof_read(const char* name, double* ms, long long* n);
}  // namespace mflat_amd

namespace {

// reference c/mflat.cpp:32-38: unknown values map to L2
Metric conv(mflat_metric_t m) {
    switch (m) {
        case MFLAT_METRIC_INNER_PRODUCT: return Metric::InnerProduct;
        case MFLAT_METRIC_COSINE: return Metric::Cosine;
        default: return Metric::L2;
    }
}

template <class F>
mflat_status_t guarded(F&& f) {
    try {
        return f();
    } catch (const std::bad_alloc&) {
        return MFLAT_ERR_ALLOC;
    } catch (const mflat_amd::NotReady& e) {
        MFLAT_LOG_ERROR("%s", e.what());
        return MFLAT_ERR_NOT_READY;
    } catch (const mflat_amd::BadArg& e) {
        MFLAT_LOG_ERROR("%s", e.what());
        return MFLAT_ERR_BAD_ARG;
    } catch (const std::exception& e) {
        MFLAT_LOG_ERROR("%s", e.what());
        return MFLAT_ERR_INTERNAL;
    } catch (...) {
        return MFLAT_ERR_INTERNAL;
    }
}

}  // namespace

struct mflat_flat_index {
    FlatIndex idx;
    std::mutex mu;
    mflat_flat_index(int d, Metric m, mflat_amd::Storage st) : idx(d, m, st) {}
};

struct mflat_ivf_index {
    mflat_amd::IvfIndex idx;
    std::mutex mu;
    mflat_ivf_index(int d, Metric m, int nl, mflat_amd::Storage st) : idx(d, m, nl, st) {}
};

struct mflat_ivfpq_index {
    mflat_amd::IvfIndex idx;
    std::mutex mu;
    mflat_ivfpq_index(int d, Metric m, int nl, int sub) : idx(d, m, nl, mflat_amd::kF32, sub) {}
};

extern "C" {

MFLAT_API const char* mflat_version(void) { return "0.1.0"; }
MFLAT_API int mflat_max_k(void) { return MFLAT_MAX_K; }

MFLAT_API const char* mflat_status_str(mflat_status_t s) {
    switch (s) {
        case MFLAT_OK: return "ok";
        case MFLAT_ERR_NULL_ARG: return "null argument";
        case MFLAT_ERR_BAD_ARG: return "bad argument";
        case MFLAT_ERR_ALLOC: return "allocation failed";
        case MFLAT_ERR_NOT_READY: return "index not ready";
        case MFLAT_ERR_INTERNAL: return "internal error";
    }
    return "unknown";
}

// the engine's router holds the caller's handler and user value as given
MFLAT_API void mflat_set_log_handler(mflat_log_handler_t h, void* user) { mflat_amd::logRoute(h, user); }
MFLAT_API void mflat_set_log_level(mflat_log_level_t l) { mflat_amd::logSetThreshold(l); }
MFLAT_API mflat_log_level_t mflat_log_level(void) { return mflat_amd::logThreshold(); }

MFLAT_API mflat_flat_index_t* mflat_flat_create_ex(int dim, mflat_metric_t metric, mflat_storage_t storage,
                                                   mflat_status_t* st) {
    if (dim <= 0 || (storage != MFLAT_STORAGE_F32 && storage != MFLAT_STORAGE_F16 &&
                     storage != MFLAT_STORAGE_BF16)) {
        if (st) *st = MFLAT_ERR_BAD_ARG;
        return nullptr;
    }
    try {
        auto* h = new mflat_flat_index(dim, conv(metric), static_cast<mflat_amd::Storage>(storage));
        if (st) *st = MFLAT_OK;
        return h;
    } catch (const std::bad_alloc&) {
        if (st) *st = MFLAT_ERR_ALLOC;
        return nullptr;
    } catch (...) {
        if (st) *st = MFLAT_ERR_INTERNAL;
        return nullptr;
    }
}

MFLAT_API mflat_flat_index_t* mflat_flat_create(int dim, mflat_metric_t metric, mflat_status_t* st) {
    return mflat_flat_create_ex(dim, metric, MFLAT_STORAGE_F32, st);
}

MFLAT_API mflat_storage_t mflat_flat_storage(const mflat_flat_index_t* h) {
    return h ? static_cast<mflat_storage_t>(h->idx.storage()) : MFLAT_STORAGE_F32;
}

MFLAT_API void mflat_flat_free(mflat_flat_index_t* h) { delete h; }
MFLAT_API int mflat_flat_ready(const mflat_flat_index_t* h) { return (h && h->idx.ready()) ? 1 : 0; }
MFLAT_API int mflat_flat_size(const mflat_flat_index_t* h) { return h ? h->idx.size() : 0; }
MFLAT_API int mflat_flat_dim(const mflat_flat_index_t* h) { return h ? h->idx.dim() : 0; }

MFLAT_API mflat_status_t mflat_flat_add(mflat_flat_index_t* h, const float* v, int n) {
    if (!h || !v) return MFLAT_ERR_NULL_ARG;
    if (n < 0) return MFLAT_ERR_BAD_ARG;
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        h->idx.add(v, n);
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_flat_reset(mflat_flat_index_t* h) {
    if (!h) return MFLAT_ERR_NULL_ARG;
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        h->idx.reset();
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_flat_search(mflat_flat_index_t* h, const float* q, int m, int k,
                                           int32_t* oi, float* od, int* ok) {
    if (!h || !q) return MFLAT_ERR_NULL_ARG;
    if (m < 0 || k < 1) return MFLAT_ERR_BAD_ARG;
    if (m == 0) {   // reference c/mflat.cpp:44: empty result, k_used = 0
        if (ok) *ok = 0;
        return MFLAT_OK;
    }
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        const int used = h->idx.search(q, m, k, oi, od);
        if (ok) *ok = used;
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_flat_search_i64(mflat_flat_index_t* h, const float* q, int m, int k,
                                               int64_t* oi, float* od, int* ok) {
    if (!h || !q) return MFLAT_ERR_NULL_ARG;
    if (m < 0 || k < 1) return MFLAT_ERR_BAD_ARG;
    if (m == 0) {
        if (ok) *ok = 0;
        return MFLAT_OK;
    }
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        std::vector<int32_t> ids32;
        if (oi) ids32.resize((size_t)m * std::min(std::max(k, 1), MFLAT_MAX_K));
        const int used = h->idx.search(q, m, k, oi ? ids32.data() : nullptr, od);
        if (oi)
            for (size_t i = 0; i < (size_t)m * used; ++i) oi[i] = ids32[i];
        if (ok) *ok = used;
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_flat_search_device(mflat_flat_index_t* h, const float* q, int m, int k,
                                                  int32_t* oi, float* od, int* ok, void* stream) {
    if (!h || !q) return MFLAT_ERR_NULL_ARG;
    if (m < 0 || k < 1) return MFLAT_ERR_BAD_ARG;
    if (m == 0) {
        if (ok) *ok = 0;
        return MFLAT_OK;
    }
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        const int used = h->idx.searchDevice(q, m, k, oi, od, static_cast<hipStream_t>(stream));
        if (ok) *ok = used;
        return MFLAT_OK;
    });
}

// No counterpart in the reference: the allocation-free variant of
// mflat_flat_search_device (the engine's searchDeviceNoAlloc).
MFLAT_API mflat_status_t mflat_flat_search_device_noalloc(mflat_flat_index_t* h, const float* q, int m, int k,
                                                          int32_t* oi, float* od, int* ok, void* stream) {
    if (!h || !q) return MFLAT_ERR_NULL_ARG;
    if (m < 0 || k < 1) return MFLAT_ERR_BAD_ARG;
    if (m == 0) {
        if (ok) *ok = 0;
        return MFLAT_OK;
    }
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        const int used = h->idx.searchDeviceNoAlloc(q, m, k, oi, od, static_cast<hipStream_t>(stream));
        if (ok) *ok = used;
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_flat_add_device(mflat_flat_index_t* h, const float* v, int n, void* stream) {
    if (!h || !v) return MFLAT_ERR_NULL_ARG;
    if (n < 0) return MFLAT_ERR_BAD_ARG;
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        if (n > 0 && !h->idx.ready())
            throw mflat_amd::NotReady("no usable HIP device: device-pointer add needs a gfx950 GPU");
        h->idx.addDevice(v, n, static_cast<hipStream_t>(stream));
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_kmeans_train(const float* pts, int n, int dim, int nlist, int iters, int mpc,
                                            float* oc, int32_t* oa, int32_t* ocs, int32_t* oo, int* onl) {
    if (!pts || !oc) return MFLAT_ERR_NULL_ARG;
    if (n < 1 || dim < 1 || nlist < 1 || iters < 0 || mpc < 0) return MFLAT_ERR_BAD_ARG;
    return guarded([&] {
        const int used = mflat_amd::kmeansTrain(pts, n, dim, nlist, iters, mpc, oc, oa, ocs, oo);
        if (onl) *onl = used;
        return MFLAT_OK;
    });
}

MFLAT_API mflat_ivf_index_t* mflat_ivf_create_ex(int dim, mflat_metric_t metric, int nlist, mflat_storage_t storage,
                                                 mflat_status_t* st) {
    if (dim <= 0 || nlist <= 0 || (storage != MFLAT_STORAGE_F32 && storage != MFLAT_STORAGE_F16 &&
                                   storage != MFLAT_STORAGE_BF16)) {
        if (st) *st = MFLAT_ERR_BAD_ARG;
        return nullptr;
    }
    try {
        auto* h = new mflat_ivf_index(dim, conv(metric), nlist, static_cast<mflat_amd::Storage>(storage));
        if (st) *st = MFLAT_OK;
        return h;
    } catch (const std::bad_alloc&) {
        if (st) *st = MFLAT_ERR_ALLOC;
        return nullptr;
    } catch (...) {
        if (st) *st = MFLAT_ERR_INTERNAL;
        return nullptr;
    }
}

MFLAT_API mflat_ivf_index_t* mflat_ivf_create(int dim, mflat_metric_t metric, int nlist, mflat_status_t* st) {
    return mflat_ivf_create_ex(dim, metric, nlist, MFLAT_STORAGE_F32, st);
}

MFLAT_API void mflat_ivf_free(mflat_ivf_index_t* h) { delete h; }
MFLAT_API int mflat_ivf_ready(const mflat_ivf_index_t* h) { return (h && h->idx.ready()) ? 1 : 0; }
MFLAT_API int mflat_ivf_size(const mflat_ivf_index_t* h) { return h ? h->idx.size() : 0; }
MFLAT_API int mflat_ivf_dim(const mflat_ivf_index_t* h) { return h ? h->idx.dim() : 0; }
MFLAT_API int mflat_ivf_nlist(const mflat_ivf_index_t* h) { return h ? h->idx.nlist() : 0; }
MFLAT_API mflat_storage_t mflat_ivf_storage(const mflat_ivf_index_t* h) {
    return h ? static_cast<mflat_storage_t>(h->idx.storage()) : MFLAT_STORAGE_F32;
}

MFLAT_API mflat_status_t mflat_ivf_build(mflat_ivf_index_t* h, const float* v, int n) {
    if (!h || !v) return MFLAT_ERR_NULL_ARG;
    if (n <= 0) return MFLAT_ERR_BAD_ARG;
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        h->idx.build(v, n);
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_ivf_search(mflat_ivf_index_t* h, const float* q, int m, int k, int nprobe,
                                          int32_t* oi, float* od, int* ok) {
    if (!h || !q) return MFLAT_ERR_NULL_ARG;
    if (m < 0 || k < 1 || nprobe < 1) return MFLAT_ERR_BAD_ARG;
    if (!h->idx.ready()) return MFLAT_ERR_NOT_READY;
    if (m == 0) {
        if (ok) *ok = 0;
        return MFLAT_OK;
    }
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        const int used = h->idx.search(q, m, k, nprobe, oi, od);
        if (ok) *ok = used;
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_ivf_search_device(mflat_ivf_index_t* h, const float* q, int m, int k, int nprobe,
                                                 int32_t* oi, float* od, int* ok, void* stream) {
    if (!h || !q) return MFLAT_ERR_NULL_ARG;
    if (m < 0 || k < 1 || nprobe < 1) return MFLAT_ERR_BAD_ARG;
    if (!h->idx.ready()) return MFLAT_ERR_NOT_READY;
    if (m == 0) {
        if (ok) *ok = 0;
        return MFLAT_OK;
    }
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        const int used = h->idx.searchDevice(q, m, k, nprobe, oi, od, static_cast<hipStream_t>(stream));
        if (ok) *ok = used;
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_ivf_probe(mflat_ivf_index_t* h, const float* q, int m, int nprobe, int32_t* cells) {
    if (!h || !q || !cells) return MFLAT_ERR_NULL_ARG;
    if (m < 0 || nprobe < 1) return MFLAT_ERR_BAD_ARG;
    if (!h->idx.ready()) return MFLAT_ERR_NOT_READY;
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        h->idx.probe(q, m, nprobe, cells);
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_ivf_coarse(const mflat_ivf_index_t* h, float* oc, int32_t* ocs, int32_t* orid) {
    if (!h) return MFLAT_ERR_NULL_ARG;
    if (!h->idx.ready()) return MFLAT_ERR_NOT_READY;
    auto* hh = const_cast<mflat_ivf_index_t*>(h);
    return guarded([&] {
        std::lock_guard<std::mutex> lk(hh->mu);
        const auto& c = h->idx.centroids();
        const auto& cs = h->idx.cellStart();
        const auto& r = h->idx.reorderedIds();
        if (oc) std::memcpy(oc, c.data(), c.size() * sizeof(float));
        if (ocs) std::memcpy(ocs, cs.data(), cs.size() * sizeof(int32_t));
        if (orid) std::memcpy(orid, r.data(), r.size() * sizeof(int32_t));
        return MFLAT_OK;
    });
}

MFLAT_API mflat_ivfpq_index_t* mflat_ivfpq_create(int dim, mflat_metric_t metric, int nlist, int m_sub,
                                                 mflat_status_t* st) {
    // reference c/mflat.cpp:162-167 (IP unsupported); m_sub above 128 is this
    // build's own limit (one query's lookup table in LDS)
    if (dim <= 0 || nlist <= 0 || m_sub <= 0 || dim % m_sub != 0 || m_sub > 128 ||
        metric == MFLAT_METRIC_INNER_PRODUCT) {
        if (st) *st = MFLAT_ERR_BAD_ARG;
        return nullptr;
    }
    try {
        auto* h = new mflat_ivfpq_index(dim, conv(metric), nlist, m_sub);
        if (st) *st = MFLAT_OK;
        return h;
    } catch (const std::bad_alloc&) {
        if (st) *st = MFLAT_ERR_ALLOC;
        return nullptr;
    } catch (...) {
        if (st) *st = MFLAT_ERR_INTERNAL;
        return nullptr;
    }
}

MFLAT_API void mflat_ivfpq_free(mflat_ivfpq_index_t* h) { delete h; }
MFLAT_API void mflat_ivfpq_set_rerank(mflat_ivfpq_index_t* h, int enable) {
    if (!h) return;
    std::lock_guard<std::mutex> lk(h->mu);
    h->idx.setRerank(enable != 0);
}
MFLAT_API int mflat_ivfpq_ready(const mflat_ivfpq_index_t* h) { return (h && h->idx.ready()) ? 1 : 0; }
MFLAT_API int mflat_ivfpq_size(const mflat_ivfpq_index_t* h) { return h ? h->idx.size() : 0; }
MFLAT_API int mflat_ivfpq_dim(const mflat_ivfpq_index_t* h) { return h ? h->idx.dim() : 0; }
MFLAT_API int mflat_ivfpq_nlist(const mflat_ivfpq_index_t* h) { return h ? h->idx.nlist() : 0; }
MFLAT_API int mflat_ivfpq_subquantizers(const mflat_ivfpq_index_t* h) { return h ? h->idx.subquantizers() : 0; }

MFLAT_API mflat_status_t mflat_ivfpq_build(mflat_ivfpq_index_t* h, const float* v, int n) {
    if (!h || !v) return MFLAT_ERR_NULL_ARG;
    if (n <= 0) return MFLAT_ERR_BAD_ARG;
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        h->idx.build(v, n);
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_ivfpq_search(mflat_ivfpq_index_t* h, const float* q, int m, int k, int nprobe,
                                            int rerank, int32_t* oi, float* od, int* ok) {
    if (!h || !q) return MFLAT_ERR_NULL_ARG;
    if (m < 0 || k < 1 || nprobe < 1 || rerank < 0) return MFLAT_ERR_BAD_ARG;
    if (!h->idx.ready()) return MFLAT_ERR_NOT_READY;
    if (m == 0) {
        if (ok) *ok = 0;
        return MFLAT_OK;
    }
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        const int used = h->idx.search(q, m, k, nprobe, oi, od, rerank);
        if (ok) *ok = used;
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_ivfpq_search_device(mflat_ivfpq_index_t* h, const float* q, int m, int k, int nprobe,
                                                   int rerank, int32_t* oi, float* od, int* ok, void* stream) {
    if (!h || !q) return MFLAT_ERR_NULL_ARG;
    if (m < 0 || k < 1 || nprobe < 1 || rerank < 0) return MFLAT_ERR_BAD_ARG;
    if (!h->idx.ready()) return MFLAT_ERR_NOT_READY;
    if (m == 0) {
        if (ok) *ok = 0;
        return MFLAT_OK;
    }
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        const int used = h->idx.searchDevice(q, m, k, nprobe, oi, od, static_cast<hipStream_t>(stream), rerank);
        if (ok) *ok = used;
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_ivfpq_probe(mflat_ivfpq_index_t* h, const float* q, int m, int nprobe,
                                           int32_t* cells) {
    if (!h || !q || !cells) return MFLAT_ERR_NULL_ARG;
    if (m < 0 || nprobe < 1) return MFLAT_ERR_BAD_ARG;
    if (!h->idx.ready()) return MFLAT_ERR_NOT_READY;
    return guarded([&] {
        std::lock_guard<std::mutex> lk(h->mu);
        h->idx.probe(q, m, nprobe, cells);
        return MFLAT_OK;
    });
}

MFLAT_API mflat_status_t mflat_ivfpq_coarse(const mflat_ivfpq_index_t* h, float* oc, int32_t* ocs, int32_t* orid,
                                            float* opqc, uint8_t* ocodes) {
    if (!h) return MFLAT_ERR_NULL_ARG;
    if (!h->idx.ready()) return MFLAT_ERR_NOT_READY;
    auto* hh = const_cast<mflat_ivfpq_index_t*>(h);
    return guarded([&] {
        std::lock_guard<std::mutex> lk(hh->mu);
        const auto& c = h->idx.centroids();
        const auto& cs = h->idx.cellStart();
        const auto& r = h->idx.reorderedIds();
        const auto& pqc = h->idx.pqCentroids();
        if (oc) std::memcpy(oc, c.data(), c.size() * sizeof(float));
        if (ocs) std::memcpy(ocs, cs.data(), cs.size() * sizeof(int32_t));
        if (orid) std::memcpy(orid, r.data(), r.size() * sizeof(int32_t));
        if (opqc) std::memcpy(opqc, pqc.data(), pqc.size() * sizeof(float));
        if (ocodes) {
            const std::vector<uint8_t> codes = h->idx.codes();
            std::memcpy(ocodes, codes.data(), codes.size());
        }
        return MFLAT_OK;
    });
}

MFLAT_API void mflat_profile_enable(int on) { mflat_amd::prof_enable(on); }
MFLAT_API void mflat_profile_reset(void) { mflat_amd::prof_reset(); }
MFLAT_API int mflat_profile_read(const char* name, double* total_ms, long long* launches) {
    return mflat_amd::prof_read(name, total_ms, launches);
}

}  // extern "C"
