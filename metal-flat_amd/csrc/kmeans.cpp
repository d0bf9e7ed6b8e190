// SPDX-License-Identifier: Apache-2.0
// kmeans.cpp -- host side of the device k-means training loop (kmeans.hpp).
// The assignment step is the flat index's fused k = 1 search (points as
// queries, centroids as the database); the update runs in kmeans_kernels.hip.
// Per iteration only the nlist cell counts cross to the host, to draw the
// reseed rows of empty cells from the same generator stream as the reference.
#include "kmeans.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "flat_index.hpp"
#include "kmeans_kernels.hpp"

namespace mflat_amd {
namespace {

void hipCheck(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) throw std::bad_alloc();
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
#define HIPC(x) hipCheck((x), #x)

struct DevMem {
    void* p = nullptr;
    explicit DevMem(size_t bytes) { HIPC(hipMalloc(&p, bytes ? bytes : 1)); }
    ~DevMem() { if (p) (void)hipFree(p); }
    DevMem(const DevMem&) = delete;
    DevMem& operator=(const DevMem&) = delete;
    template <class T> T* as() const { return static_cast<T*>(p); }
};

struct Stream {
    hipStream_t s = nullptr;
    Stream() { HIPC(hipStreamCreateWithFlags(&s, hipStreamNonBlocking)); }
    ~Stream() { if (s) (void)hipStreamDestroy(s); }
};

uint32_t bounded(std::mt19937& rng, uint32_t range) {   // uniform in [0, range)
    const uint64_t lim = (uint64_t(1) << 32) - ((uint64_t(1) << 32) % range);
    uint64_t u;
    do { u = rng(); } while (u >= lim);
    return (uint32_t)(u % range);
}

}  // namespace

int kmeansTrainDevice(const float* dData, int n, int dim, int nlistReq, int iters, int maxPointsPerCentroid,
                      float* dCentOut, int32_t* dAssignOut, int32_t* dOrderOut, int32_t* cellStart, hipStream_t s,
                      bool wrapSeeds) {
    if (n < 1 || dim < 1 || nlistReq < 1 || iters < 0 || maxPointsPerCentroid < 0)
        throw BadArg("kmeans: n, dim, nlist must be >= 1 and iters, max_points_per_centroid >= 0");
    // wrapSeeds: nlist stays nlistReq even above n, seed c being point perm[c mod n]
    // (reference src/Internal.h:241-248, the PQ sub-quantizers' 256 cells)
    const int nlist = wrapSeeds ? nlistReq : std::min(nlistReq, n);
    FlatIndex assigner(dim, Metric::L2);
    if (!assigner.ready()) throw NotReady("no usable HIP device: k-means needs a gfx950 GPU");

    // seeding (reference src/Internal.h:238-248)
    std::mt19937 rng(12345);
    std::vector<int32_t> perm((size_t)n);
    for (int i = 0; i < n; ++i) perm[(size_t)i] = i;
    for (int i = n - 1; i > 0; --i) std::swap(perm[(size_t)i], perm[bounded(rng, (uint32_t)i + 1)]);
    // training subsample: the first trainN entries of the permutation (:250-263)
    int trainN = n;
    if (maxPointsPerCentroid > 0 && (int64_t)maxPointsPerCentroid * nlist < n) trainN = maxPointsPerCentroid * nlist;

    const size_t rowB = (size_t)dim * sizeof(float);
    if (nlist > n)
        for (int c = n; c < nlist; ++c) perm.push_back(perm[(size_t)(c % n)]);
    DevMem dPerm(perm.size() * sizeof(int));
    HIPC(hipMemcpyAsync(dPerm.p, perm.data(), perm.size() * sizeof(int), hipMemcpyHostToDevice, s));
    float* dCent = dCentOut;
    launch_gather_points(dData, dPerm.as<int>(), nlist, dim, dCent, s);
    const float* dTrain = dData;
    DevMem dTrainBuf(trainN < n ? (size_t)trainN * rowB : 0);
    if (trainN < n) {
        launch_gather_points(dData, dPerm.as<int>(), trainN, dim, dTrainBuf.as<float>(), s);
        dTrain = dTrainBuf.as<float>();
    }

    DevMem dAssignBuf(dAssignOut ? 0 : (size_t)n * sizeof(int)), dOrderBuf(dOrderOut ? 0 : (size_t)n * sizeof(int));
    int* dAssign = dAssignOut ? dAssignOut : dAssignBuf.as<int>();
    int* dOrder = dOrderOut ? dOrderOut : dOrderBuf.as<int>();
    DevMem dCounts((size_t)nlist * sizeof(int));
    DevMem dStart((size_t)(nlist + 1) * sizeof(int)), dReseed((size_t)nlist * sizeof(int));
    CellGrouping grouping;
    std::vector<int> counts((size_t)nlist), start((size_t)nlist + 1), reseed((size_t)nlist);
    auto assignAll = [&](const float* pts, int m) {
        assigner.reset();
        assigner.addDevice(dCent, nlist, s);
        assigner.searchDevice(pts, m, 1, dAssign, nullptr, s);
        grouping.group(dAssign, m, nlist, dOrder, dCounts.as<int>(), s);
        HIPC(hipMemcpyAsync(counts.data(), dCounts.p, (size_t)nlist * sizeof(int), hipMemcpyDeviceToHost, s));
        HIPC(hipStreamSynchronize(s));
        start[0] = 0;
        for (int c = 0; c < nlist; ++c) start[(size_t)c + 1] = start[(size_t)c] + counts[(size_t)c];
    };

    for (int it = 0; it < iters; ++it) {
        assignAll(dTrain, trainN);
        // empty cells, in ascending order, take training point rng() % trainN
        // (reference src/Internal.h:93-98)
        for (int c = 0; c < nlist; ++c)
            reseed[(size_t)c] = counts[(size_t)c] == 0 ? (int)(rng() % (uint32_t)trainN) : -1;
        HIPC(hipMemcpyAsync(dStart.p, start.data(), start.size() * sizeof(int), hipMemcpyHostToDevice, s));
        HIPC(hipMemcpyAsync(dReseed.p, reseed.data(), reseed.size() * sizeof(int), hipMemcpyHostToDevice, s));
        launch_update_centroids(dTrain, dim, dOrder, dStart.as<int>(), dReseed.as<int>(), nlist, dCent, s);
    }
    // final assignment of every point (reference src/Internal.h:357-359) and its CSR
    // (src/CoarseQuantizer.mm:135-145)
    assignAll(dData, n);
    HIPC(hipStreamSynchronize(s));
    if (cellStart) std::copy(start.begin(), start.end(), cellStart);
    return nlist;
}

int kmeansTrain(const float* points, int n, int dim, int nlistReq, int iters, int maxPointsPerCentroid,
                float* centroids, int32_t* assign, int32_t* cellStart, int32_t* order) {
    if (n < 1 || dim < 1 || nlistReq < 1 || iters < 0 || maxPointsPerCentroid < 0)
        throw BadArg("kmeans: n, dim, nlist must be >= 1 and iters, max_points_per_centroid >= 0");
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        throw NotReady("no usable HIP device: k-means needs a gfx950 GPU");
    }
    const int nlist = std::min(nlistReq, n);
    Stream st;
    const hipStream_t s = st.s;
    const size_t rowB = (size_t)dim * sizeof(float);
    DevMem dData((size_t)n * rowB), dCent((size_t)nlist * rowB);
    DevMem dAssign(assign ? (size_t)n * sizeof(int) : 0), dOrder(order ? (size_t)n * sizeof(int) : 0);
    HIPC(hipMemcpyAsync(dData.p, points, (size_t)n * rowB, hipMemcpyHostToDevice, s));
    kmeansTrainDevice(dData.as<float>(), n, dim, nlistReq, iters, maxPointsPerCentroid, dCent.as<float>(),
                      assign ? dAssign.as<int32_t>() : nullptr, order ? dOrder.as<int32_t>() : nullptr, cellStart, s);
    HIPC(hipMemcpyAsync(centroids, dCent.p, (size_t)nlist * rowB, hipMemcpyDeviceToHost, s));
    if (assign) HIPC(hipMemcpyAsync(assign, dAssign.p, (size_t)n * sizeof(int), hipMemcpyDeviceToHost, s));
    if (order) HIPC(hipMemcpyAsync(order, dOrder.p, (size_t)n * sizeof(int), hipMemcpyDeviceToHost, s));
    HIPC(hipStreamSynchronize(s));
    return nlist;
}

}  // namespace mflat_amd
