/* SPDX-License-Identifier: Apache-2.0 */
/* mflat.h -- C ABI of the MI355X-native exact flat-search library (libmflat.so).
 *
 * Drop-in for the flat-search part of metal-flat's C ABI
 * (reference: c/include/mflat.h:31-90, implementation c/mflat.cpp:32-129).
 * Same opaque handle, same status codes, same caller-owned output buffers,
 * same row-major nearest-first results with -1 id padding.
 *
 * Buffer contract for mflat_flat_search: out_ids and out_distances are
 * caller-allocated, each holding at least m * k elements (either may be NULL).
 * *out_k_used (nullable) receives the number of columns actually written;
 * the row stride of both outputs is k_used (reference c/mflat.cpp:42-50).
 *
 * Divergences from the reference, all deliberate:
 *  - MFLAT_MAX_K is 1024 (reference 64, include/metalflat/FlatIndex.h:43);
 *    k above it is clamped with a one-time warning per index, as in the
 *    reference (src/FlatIndex.mm:298-304).
 *  - There is no CPU fallback. Without a usable HIP device an index can be
 *    created and filled (mflat_flat_ready() == 0) but mflat_flat_search
 *    returns MFLAT_ERR_NOT_READY (reference: exact CPU path,
 *    src/FlatIndex.mm:317-321).
 *  - The IVF entry points (reference c/include/mflat.h:92-105) are here,
 *    with the same argument checks and result layout; IVF search serves
 *    k <= MFLAT_MAX_K and nprobe <= MFLAT_MAX_K on the device (the reference
 *    serves k > 64 on its CPU path, src/IvfIndex.mm:762-764); any dim.
 *  - The IVF-PQ entry points (reference c/include/mflat.h:107-129) are here with
 *    the reference C ABI's behaviour: residual PQ, no OPQ (the reference's C
 *    ABI reaches neither of its setResidual / setOpq switches); k up to
 *    MFLAT_MAX_K (reference 64), rerank shortlists up to MFLAT_MAX_K rows, and
 *    m_sub <= 128.
 *  - Additive entry points (reduced-precision storage, device-pointer
 *    search/add, kernel timing) follow the flat block; they have no
 *    counterpart in the reference.
 */
#ifndef MFLAT_H
#define MFLAT_H

#include <stdint.h>

#define MFLAT_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

#define MFLAT_VERSION_MAJOR 0
#define MFLAT_VERSION_MINOR 1
#define MFLAT_VERSION_PATCH 0
#define MFLAT_MAX_K 1024        /* largest k one search returns (reference: 64) */

/* value-stable; reference c/include/mflat.h:36-40 */
typedef enum {
    MFLAT_METRIC_L2            = 0,   /* squared Euclidean, smaller = nearer */
    MFLAT_METRIC_INNER_PRODUCT = 1,   /* dot product, larger = nearer        */
    MFLAT_METRIC_COSINE        = 2    /* dot of L2-normalised vectors        */
} mflat_metric_t;

/* value-stable; reference c/include/mflat.h:42-49 */
typedef enum {
    MFLAT_OK            = 0,
    MFLAT_ERR_NULL_ARG  = 1,    /* a required pointer was NULL                     */
    MFLAT_ERR_BAD_ARG   = 2,    /* dim/n/m/k out of range                          */
    MFLAT_ERR_ALLOC     = 3,    /* host or device allocation failed                */
    MFLAT_ERR_NOT_READY = 4,    /* no usable HIP device for this index             */
    MFLAT_ERR_INTERNAL  = 5     /* unexpected exception or HIP runtime error       */
} mflat_status_t;

/* reference c/include/mflat.h:51-53, c/mflat.cpp:72-73,86-96 */
MFLAT_API const char* mflat_version(void);               /* "0.1.0"             */
MFLAT_API const char* mflat_status_str(mflat_status_t);  /* static; do not free */
MFLAT_API int         mflat_max_k(void);                 /* MFLAT_MAX_K         */

/* ---------------- Logging (reference c/include/mflat.h:55-74) ------------- */
typedef enum {
    MFLAT_LOG_INFO  = 0,
    MFLAT_LOG_WARN  = 1,
    MFLAT_LOG_ERROR = 2,
    MFLAT_LOG_OFF   = 3          /* threshold only; never delivered to a handler */
} mflat_log_level_t;

/* msg: NUL-terminated, no "[mflat]" prefix, no newline; user round-trips. */
typedef void (*mflat_log_handler_t)(mflat_log_level_t level, const char* msg, void* user);

/* handler == NULL restores the built-in stderr sink (reference c/mflat.cpp:75-79). */
MFLAT_API void              mflat_set_log_handler(mflat_log_handler_t handler, void* user);
MFLAT_API void              mflat_set_log_level(mflat_log_level_t threshold);
MFLAT_API mflat_log_level_t mflat_log_level(void);

/* ---------------- FlatIndex (exact) -------------------------------------- */
typedef struct mflat_flat_index mflat_flat_index_t;      /* opaque */

/* reference c/mflat.cpp:99-104: dim <= 0 -> NULL + MFLAT_ERR_BAD_ARG;
   an unknown metric value maps to L2 (c/mflat.cpp:32-38). */
MFLAT_API mflat_flat_index_t*
mflat_flat_create(int dim, mflat_metric_t metric, mflat_status_t* out_status);
/* reference c/mflat.cpp:105; NULL is a no-op */
MFLAT_API void mflat_flat_free(mflat_flat_index_t*);

/* reference c/mflat.cpp:106-108: 1 = HIP device usable, 0 = none */
MFLAT_API int mflat_flat_ready(const mflat_flat_index_t*);
MFLAT_API int mflat_flat_size (const mflat_flat_index_t*);
MFLAT_API int mflat_flat_dim  (const mflat_flat_index_t*);

/* reference c/mflat.cpp:110-116: append n row-major vectors (n*dim floats,
   host memory, borrowed for the call). NULL -> NULL_ARG, n < 0 -> BAD_ARG,
   n == 0 -> OK. Cosine rows are stored L2-normalised. */
MFLAT_API mflat_status_t mflat_flat_add(mflat_flat_index_t*, const float* vectors, int n);
/* reference c/mflat.cpp:117-121 */
MFLAT_API mflat_status_t mflat_flat_reset(mflat_flat_index_t*);
/* reference c/mflat.cpp:122-129: m < 0 or k < 1 -> BAD_ARG; m == 0 -> OK with
   *out_k_used = 0. queries: m*dim floats in host memory. */
MFLAT_API mflat_status_t mflat_flat_search(mflat_flat_index_t*, const float* queries,
        int m, int k, int32_t* out_ids, float* out_distances, int* out_k_used);

/* ---------------- IvfIndex (approximate) ---------------------------------- */
/* reference c/include/mflat.h:92-105, c/mflat.cpp:131-159, src/IvfIndex.mm.
   build() trains nlist k-means cells (12 iterations, at most 256 training
   points per centroid; nlist clamped to n) and files every row under its
   nearest centroid; search() takes each query's nprobe nearest centroids
   (nprobe clamped to [1, nlist]) and returns the exact top-k over the rows of
   those cells: ids are the caller's row indices, values as for the flat
   index, ties in scan order (cells nearest first, rows in ascending id within
   a cell), -1 / +-inf padding when the probed cells hold fewer than k rows. */
typedef struct mflat_ivf_index mflat_ivf_index_t;      /* opaque */

/* reference c/mflat.cpp:132-137: dim <= 0 or nlist <= 0 -> NULL + BAD_ARG */
MFLAT_API mflat_ivf_index_t*
mflat_ivf_create(int dim, mflat_metric_t metric, int nlist, mflat_status_t* out_status);
MFLAT_API void mflat_ivf_free(mflat_ivf_index_t*);      /* NULL is a no-op */

MFLAT_API int mflat_ivf_ready(const mflat_ivf_index_t*);  /* 1 after build() */
MFLAT_API int mflat_ivf_size (const mflat_ivf_index_t*);
MFLAT_API int mflat_ivf_dim  (const mflat_ivf_index_t*);
MFLAT_API int mflat_ivf_nlist(const mflat_ivf_index_t*);  /* requested, then trained */

/* reference c/mflat.cpp:144-150: NULL -> NULL_ARG, n <= 0 -> BAD_ARG; rows
   are host memory, borrowed for the call; a rebuild replaces the index.
   No usable device -> MFLAT_ERR_NOT_READY (no CPU fallback). */
MFLAT_API mflat_status_t mflat_ivf_build(mflat_ivf_index_t*, const float* vectors, int n);
/* reference c/mflat.cpp:151-159: NULL -> NULL_ARG; m < 0, k < 1 or
   nprobe < 1 -> BAD_ARG; not built -> NOT_READY; m == 0 -> OK, k_used 0.
   Outputs hold m * k elements with row stride k_used. */
MFLAT_API mflat_status_t mflat_ivf_search(mflat_ivf_index_t*, const float* queries,
        int m, int k, int nprobe, int32_t* out_ids, float* out_distances, int* out_k_used);

/* ---------------- IvfPqIndex (compressed) ---------------------------------- */
/* reference c/include/mflat.h:107-129, c/mflat.cpp:161-198, src/IvfPqIndex.mm.
   build() trains the coarse cells as mflat_ivf_build, then product-quantizes
   every row's residual to its cell centroid: m_sub sub-vectors of dim / m_sub
   columns, each replaced by the byte id of its nearest of 256 sub-centroids
   (k-means per sub-space, 12 iterations over all rows). search() ranks the
   rows of each query's nprobe nearest cells by the asymmetric distance
   ||q - c||^2 + sum_m (||p_m||^2 - 2 q_m . p_m + 2 c_m . p_m) (p_m the row's
   sub-centroids), ties in scan order, and reports that value (an
   approximate squared distance, for L2 and Cosine alike). With rerank > k on
   an index built after mflat_ivfpq_set_rerank(h, 1), the top-rerank of that
   ranking is re-ranked by exact distance (values: squared L2, or the dot for
   Cosine), ties in shortlist order. Metric must be L2 or Cosine. */
typedef struct mflat_ivfpq_index mflat_ivfpq_index_t;  /* opaque */

/* reference c/mflat.cpp:162-170: dim, nlist, m_sub <= 0, dim % m_sub != 0 or
   INNER_PRODUCT -> NULL + BAD_ARG (also m_sub > 128 here) */
MFLAT_API mflat_ivfpq_index_t*
mflat_ivfpq_create(int dim, mflat_metric_t metric, int nlist, int m_sub, mflat_status_t* out_status);
MFLAT_API void mflat_ivfpq_free(mflat_ivfpq_index_t*);
/* keep the full rows for exact reranking; takes effect at the next build */
MFLAT_API void mflat_ivfpq_set_rerank(mflat_ivfpq_index_t*, int enable);

MFLAT_API int mflat_ivfpq_ready(const mflat_ivfpq_index_t*);  /* 1 after build() */
MFLAT_API int mflat_ivfpq_size (const mflat_ivfpq_index_t*);
MFLAT_API int mflat_ivfpq_dim  (const mflat_ivfpq_index_t*);
MFLAT_API int mflat_ivfpq_nlist(const mflat_ivfpq_index_t*);
MFLAT_API int mflat_ivfpq_subquantizers(const mflat_ivfpq_index_t*);  /* bytes per code */

/* reference c/mflat.cpp:182-188 */
MFLAT_API mflat_status_t mflat_ivfpq_build(mflat_ivfpq_index_t*, const float* vectors, int n);
/* reference c/mflat.cpp:189-198: rerank < 0 -> BAD_ARG besides the IVF checks;
   rerank 0 or 1 (or <= k) = off. */
MFLAT_API mflat_status_t mflat_ivfpq_search(mflat_ivfpq_index_t*, const float* queries,
        int m, int k, int nprobe, int rerank,
        int32_t* out_ids, float* out_distances, int* out_k_used);

/* ---------------- Additive: reduced-precision storage --------------------- */
/* No counterpart in the reference (its FlatIndex stores fp32 only,
   src/FlatIndex.mm:236-245). The index holds its database, and each search
   its queries, in the chosen element type: the caller's fp32 values are
   rounded to nearest even (after the Cosine normalisation, in fp32), dots
   accumulate in fp32 on the fp16/bf16 matrix cores, norms are double sums of
   the rounded values. Results are those of exact fp32 search on the rounded
   inputs (up to fp32 accumulation order); values beyond the type's range
   become +-inf and such rows or queries are never returned. Half the HBM of
   fp32. Every other entry point behaves as for an fp32 index. */
typedef enum {
    MFLAT_STORAGE_F32  = 0,
    MFLAT_STORAGE_F16  = 1,   /* IEEE binary16 */
    MFLAT_STORAGE_BF16 = 2    /* bfloat16 */
} mflat_storage_t;

/* As mflat_flat_create; an unknown storage value -> NULL + MFLAT_ERR_BAD_ARG. */
MFLAT_API mflat_flat_index_t*
mflat_flat_create_ex(int dim, mflat_metric_t metric, mflat_storage_t storage, mflat_status_t* out_status);
/* storage type of the index (MFLAT_STORAGE_F32 for NULL) */
MFLAT_API mflat_storage_t mflat_flat_storage(const mflat_flat_index_t*);

/* ---------------- Additive: 64-bit ids ----------------------------------- */
/* No counterpart in the reference (its ids are int32, c/include/mflat.h:84-90).
   Same arguments, checks, status codes and results as mflat_flat_search, with
   the ids widened to int64 (-1 padding stays -1), for callers whose id type is
   64-bit. */
MFLAT_API mflat_status_t mflat_flat_search_i64(mflat_flat_index_t*, const float* queries,
        int m, int k, int64_t* out_ids, float* out_distances, int* out_k_used);

/* ---------------- Additive: k-means (IVF coarse-quantizer training) ------ */
/* No C counterpart in the reference: its k-means is internal to IVF training
   (CoarseQuantizer::train over detail::kmeansGpu, src/CoarseQuantizer.mm:104-159,
   src/Internal.h:234-382). Trains nlist = min(nlist, n) L2 centroids on n
   row-major points (host memory, borrowed for the call) with the whole loop on
   the device: seeds are nlist distinct points of a uniform permutation drawn
   from mt19937(12345); training uses the first min(n, max_points_per_centroid
   * nlist) points of that permutation (0 = all points); each of `iters`
   iterations assigns every training point to its nearest centroid (lowest
   index on ties) and sets each centroid to float(double sum / count) of its
   points summed in ascending order, an empty cell taking a training point
   drawn from the same generator; a final pass assigns all n points.
   Outputs (caller-allocated; all but out_centroids nullable):
     out_centroids     nlist * dim floats
     out_assign        n cell ids
     out_cell_start    nlist + 1 offsets of each cell in out_order
     out_order         n point ids grouped by cell, ascending within a cell
     out_nlist         nlist used
   The seeds differ from the reference's (its std::shuffle draws are specific to
   its standard library); every step after seeding follows it.
   NULL points / out_centroids -> MFLAT_ERR_NULL_ARG; n, dim, nlist < 1 or
   iters, max_points_per_centroid < 0 -> MFLAT_ERR_BAD_ARG; no usable device ->
   MFLAT_ERR_NOT_READY. */
MFLAT_API mflat_status_t mflat_kmeans_train(const float* points, int n, int dim, int nlist, int iters,
        int max_points_per_centroid, float* out_centroids, int32_t* out_assign,
        int32_t* out_cell_start, int32_t* out_order, int* out_nlist);

/* ---------------- Additive: device-resident data ------------------------- */
/* No counterpart in the reference (its buffers are unified memory,
   src/FlatIndex.mm:163-171). For callers whose data already lives in HBM.
   All pointers are device pointers of the index's device; `stream` is a
   hipStream_t (NULL = the index's own stream). The call returns after the
   results are complete on the device. Same argument checks and status codes
   as mflat_flat_search / mflat_flat_add; out_ids / out_distances hold m*k
   elements with row stride k_used. */
MFLAT_API mflat_status_t mflat_flat_search_device(mflat_flat_index_t*, const float* d_queries,
        int m, int k, int32_t* d_out_ids, float* d_out_distances, int* out_k_used,
        void* stream);
MFLAT_API mflat_status_t mflat_flat_add_device(mflat_flat_index_t*, const float* d_vectors,
        int n, void* stream);

/* ---------------- Additive: allocation-free search ----------------------- */
/* No counterpart in the reference. For callers that cannot allocate device
   memory: code under HIP graph capture, tight serving loops, harnesses that
   forbid hipMalloc. As mflat_flat_search_device, but the call allocates
   nothing (no hipMalloc / hipFree, no allocating library routine): its
   workspace is a statically sized device array of 4 MiB that each GPU the
   library runs on holds until the process ends. The database must already be
   resident (mflat_flat_add / _add_device allocate as usual). Limits: m <= 16
   queries, k <= 32, dim <= 992 (fp32 storage) or 2016 (fp16 / bf16); beyond
   them MFLAT_ERR_BAD_ARG (no clamping).
   Stream-ordered: returns once the work is enqueued on `stream` (NULL = the
   index's own stream); results are complete when that stream reaches this
   point. Every call on one GPU shares that GPU's array: calls that can
   overlap on one GPU (different streams, or different threads without
   ordering) race and must be serialised by the caller. Results equal
   mflat_flat_search_device's (exact top-k, ties to the lower id). */
MFLAT_API mflat_status_t mflat_flat_search_device_noalloc(mflat_flat_index_t*, const float* d_queries,
        int m, int k, int32_t* d_out_ids, float* d_out_distances, int* out_k_used, void* stream);

/* ---------------- Additive: IVF extensions ------------------------------- */
/* No C counterpart in the reference. mflat_ivf_create_ex: as mflat_ivf_create
   with the fine scan's storage type (the rows and the queries of the fine scan
   rounded as for mflat_flat_create_ex; the coarse probe stays fp32).
   mflat_ivf_search_device: as mflat_ivf_search on device pointers (as
   mflat_flat_search_device). mflat_ivf_probe: the coarse stage alone, the
   m * nprobe nearest cells, nearest first (CoarseQuantizer::probeCells,
   src/CoarseQuantizer.mm:170-188). mflat_ivf_coarse: the coarse layer after
   build (CoarseQuantizer accessors, src/CoarseQuantizer.h): out_centroids
   nlist * dim, out_cell_start nlist + 1, out_reordered_ids size() row ids in
   cell order; each nullable. */
MFLAT_API mflat_ivf_index_t*
mflat_ivf_create_ex(int dim, mflat_metric_t metric, int nlist, mflat_storage_t storage, mflat_status_t* out_status);
MFLAT_API mflat_storage_t mflat_ivf_storage(const mflat_ivf_index_t*);
MFLAT_API mflat_status_t mflat_ivf_search_device(mflat_ivf_index_t*, const float* d_queries, int m, int k,
        int nprobe, int32_t* d_out_ids, float* d_out_distances, int* out_k_used, void* stream);
MFLAT_API mflat_status_t mflat_ivf_probe(mflat_ivf_index_t*, const float* queries, int m, int nprobe,
        int32_t* out_cells);
MFLAT_API mflat_status_t mflat_ivf_coarse(const mflat_ivf_index_t*, float* out_centroids,
        int32_t* out_cell_start, int32_t* out_reordered_ids);

/* ---------------- Additive: IVF-PQ extensions ----------------------------- */
/* No C counterpart in the reference. mflat_ivfpq_search_device: as
   mflat_ivfpq_search on device pointers. mflat_ivfpq_probe: the coarse stage
   alone (as mflat_ivf_probe). mflat_ivfpq_coarse: after build, the coarse
   layer (as mflat_ivf_coarse) and the codebook: out_pq_centroids m_sub x 256 x
   (dim / m_sub) floats, out_codes size() x m_sub bytes in cell order (the row
   slot of out_reordered_ids); each nullable. */
MFLAT_API mflat_status_t mflat_ivfpq_search_device(mflat_ivfpq_index_t*, const float* d_queries, int m, int k,
        int nprobe, int rerank, int32_t* d_out_ids, float* d_out_distances, int* out_k_used, void* stream);
MFLAT_API mflat_status_t mflat_ivfpq_probe(mflat_ivfpq_index_t*, const float* queries, int m, int nprobe,
        int32_t* out_cells);
MFLAT_API mflat_status_t mflat_ivfpq_coarse(const mflat_ivfpq_index_t*, float* out_centroids,
        int32_t* out_cell_start, int32_t* out_reordered_ids, float* out_pq_centroids, uint8_t* out_codes);

/* ---------------- Additive: kernel timing -------------------------------- */
/* No counterpart in the reference. When enabled, every launch of the library's
   kernels is bracketed with HIP events on the stream it runs on; the per-kernel
   totals accumulate process-wide until reset. name: kernel family, one of
   "scan_filter" (fused distance + threshold filter over the database, the
   hot kernel; one launch per search batch), "scan_sample" (the same kernel
   over the row sample that sets the thresholds), "scan_retry" (the same
   kernel re-run for the few queries whose threshold must be refined),
   "select" (per-query top-k select / merge), "argmin" (fused k = 1),
   "norms", "prep", "ivf_scan" (IVF fine scan over every probed cell under
   the bound, and its retries), "ivf_bound" (the IVF bound pass over a row
   sample of each query's nearest cells). Returns 0 and fills the outputs, or
   -1 for an unknown name. */
MFLAT_API void mflat_profile_enable(int on);
MFLAT_API void mflat_profile_reset(void);
MFLAT_API int  mflat_profile_read(const char* name, double* total_ms, long long* launches);

#ifdef __cplusplus
}
#endif
#endif /* MFLAT_H */
