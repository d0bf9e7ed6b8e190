// SPDX-License-Identifier: Apache-2.0
// flat_index.hpp -- exact flat index on one MI355X (engine behind the C ABI).
//
// Mirrors the reference's mflat::FlatIndex (include/metalflat/FlatIndex.h:37-77):
// add / reset / search with the same result semantics, row-major nearest-first
// output with -1 padding. The database lives in HBM from add() on (the
// reference keeps a host copy and re-uploads lazily, src/FlatIndex.mm:160-178).
// Not thread-safe; the C ABI serialises calls per handle.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <stdexcept>

#include "kernels.hpp"

namespace mflat_amd {

enum class Metric : int { L2 = 0, InnerProduct = 1, Cosine = 2 };

// Thrown by search on an index without a usable HIP device.
struct NotReady : std::runtime_error {
    using std::runtime_error::runtime_error;
};
// Thrown for arguments the engine cannot serve (e.g. more than 2^31-1 rows).
struct BadArg : std::runtime_error {
    using std::runtime_error::runtime_error;
};

class FlatIndex {
public:
    static constexpr int kMaxK = 1024;

    // storage: element type the database and the queries are held in (kF32,
    // or the reduced-precision kF16 / kBF16: fp32 inputs rounded to nearest
    // even, dots accumulated in fp32).
    FlatIndex(int dim, Metric metric, Storage storage = kF32);
    ~FlatIndex();
    FlatIndex(const FlatIndex&) = delete;
    FlatIndex& operator=(const FlatIndex&) = delete;

    bool ready() const;
    int size() const;
    int dim() const;
    Metric metric() const;
    Storage storage() const;

    // Append n rows (n * dim floats). Host or device memory.
    void add(const float* host_rows, int n);
    void addDevice(const float* dev_rows, int n, hipStream_t stream);
    void reset();

    // Exact top-k for m queries. Returns k_used (0 when m == 0). Outputs hold
    // m * k_used elements, row stride k_used; either may be null.
    int search(const float* host_queries, int m, int k, int32_t* ids, float* dists);
    int searchDevice(const float* dev_queries, int m, int k, int32_t* dev_ids, float* dev_dists,
                     hipStream_t stream);
    // As searchDevice, allocating nothing: the workspace is the GPU's static
    // scratch array (noalloc.hpp). m <= kNoAllocMaxQ, k <= kStreamTopK, and a
    // dimension whose 16-query tile fits the streaming scan's LDS (BadArg
    // otherwise). Stream-ordered: returns once the work is enqueued.
    int searchDeviceNoAlloc(const float* dev_queries, int m, int k, int32_t* dev_ids, float* dev_dists,
                            hipStream_t stream);

private:
    struct Impl;
    std::unique_ptr<Impl> d_;
};

}  // namespace mflat_amd
