// SPDX-License-Identifier: Apache-2.0
// ivf_index.hpp -- inverted-file (IVF) index on one MI355X (engine behind the
// mflat_ivf_* C ABI).
//
// Mirrors the reference's mflat::IvfIndex (include/metalflat/IvfIndex.h:29-62)
// and its coarse layer (src/CoarseQuantizer.h): build() trains nlist k-means
// cells and stores the database cell-major; search() probes each query's
// nprobe nearest centroids and returns the exact top-k over the rows of those
// cells. Results follow the reference's two-stage search
// (src/IvfIndex.mm:518-560, :759-879): ranking by the flat index's keys,
// ties kept in scan order (cells in probe order, rows in cell order), -1 /
// +-inf padding when the probed cells hold fewer than k rows. Not thread-safe;
// the C ABI serialises calls per handle.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <vector>

#include "flat_index.hpp"

namespace mflat_amd {

class IvfIndex {
public:
    static constexpr int kMaxK = FlatIndex::kMaxK;       // largest k
    static constexpr int kMaxProbe = FlatIndex::kMaxK;   // largest nprobe (the probe is a flat top-nprobe)

    // storage: element type of the stored rows and of the queries in the fine
    // scan (as FlatIndex); the coarse probe is always fp32.
    // pqM > 0: an IVF-PQ index (reference include/metalflat/IvfPqIndex.h:37-99):
    // rows stored as pqM one-byte residual PQ codes (pqM divides dim, <= 128;
    // L2 or Cosine), searched by asymmetric distance; storage is unused.
    IvfIndex(int dim, Metric metric, int nlist, Storage storage = kF32, int pqM = 0);
    ~IvfIndex();
    IvfIndex(const IvfIndex&) = delete;
    IvfIndex& operator=(const IvfIndex&) = delete;

    bool ready() const;        // true once build() has produced cells
    bool deviceOk() const;     // a usable gfx950 device was found
    int size() const;
    int dim() const;
    int nlist() const;         // the requested count before build(), the trained count after
    Metric metric() const;
    Storage storage() const;

    // k-means (12 iterations, at most 256 training points per centroid) over
    // the n rows, then every row goes to its cell. Host or device rows.
    void build(const float* host_rows, int n);
    void buildDevice(const float* dev_rows, int n, hipStream_t stream);

    // Top-k over each query's nprobe nearest cells. Returns k_used (0 when
    // m == 0); outputs m * k_used, row stride k_used, either nullable.
    // IVF-PQ: the ADC top-k; with rerank > k on an index built after
    // setRerank(true), the ADC top-min(rerank, size, 1024) re-ranked by exact
    // distance (reference src/IvfPqIndex.mm:552-627).
    int search(const float* host_queries, int m, int k, int nprobe, int32_t* ids, float* dists, int rerank = 0);
    int searchDevice(const float* dev_queries, int m, int k, int nprobe, int32_t* dev_ids, float* dev_dists,
                     hipStream_t stream, int rerank = 0);

    // IVF-PQ: keep the full rows for exact reranking (latched by build()).
    void setRerank(bool enable);
    int subquantizers() const;   // pqM (0: a plain IVF index)
    // IVF-PQ, after build: sub-centroids pqM x 256 x (dim / pqM); codes
    // size() x pqM in cell order (row slot of reorderedIds()).
    const std::vector<float>& pqCentroids() const;
    std::vector<uint8_t> codes() const;

    // The coarse stage alone: m x nprobe nearest cells, nearest first (host).
    void probe(const float* host_queries, int m, int nprobe, int32_t* cells);

    // The coarse layer (reference src/CoarseQuantizer.h accessors): centroids
    // nlist x dim, CSR cell starts nlist + 1, row ids in cell order.
    const std::vector<float>& centroids() const;
    const std::vector<int>& cellStart() const;
    const std::vector<int>& reorderedIds() const;

private:
    struct Impl;
    std::unique_ptr<Impl> d_;
};

}  // namespace mflat_amd
