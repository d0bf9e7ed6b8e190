// SPDX-License-Identifier: Apache-2.0
// kmeans_kernels.hpp -- device side of the k-means training loop.
#pragma once

#include <hip/hip_runtime.h>

namespace mflat_amd {

// Groups points by cell: orderOut[0, n) = point ids sorted by cell[], ascending
// id within a cell (a stable sort), countsOut[0, nlist) = points per cell.
// Keeps its scratch between calls.
struct CellGrouping {
    void* iota = nullptr;
    void* keysOut = nullptr;
    void* temp = nullptr;
    size_t tempBytes = 0;
    int cap = 0;
    ~CellGrouping();
    void release();
    void group(const int* cell, int n, int nlist, int* orderOut, int* countsOut, hipStream_t s);
};

// dst row i = src row idx[i], i < n (row-major, any dim)
void launch_gather_points(const float* src, const int* idx, int n, int dim, float* dst, hipStream_t s);

// centroids[c] = float(double sum / count) of pts rows order[cellStart[c],
// cellStart[c + 1]) in that order, or a copy of pts row reseed[c] when the
// cell is empty. pts: row-major n x dim.
void launch_update_centroids(const float* pts, int dim, const int* order, const int* cellStart, const int* reseed,
                             int nlist, float* centroids, hipStream_t s);

}  // namespace mflat_amd
