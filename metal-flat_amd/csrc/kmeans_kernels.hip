// SPDX-License-Identifier: Apache-2.0
// kmeans_kernels.hip -- device side of the k-means training loop (the
// centroid update after the fused k = 1 assignment).
//
//   group_by_cell     stable radix sort of (cell, point) pairs (primitives.hip), so the
//                     points of every cell come out in ascending point order
//   cell_counts       points per cell
//   gather_points     training subsample rows
//   update_centroids  one workgroup per cell: centroid = float(double sum /
//                     count), the sum taken over the cell's points in ascending
//                     point order -- the order and types of the reference's
//                     scalar update (src/CoarseQuantizer.mm:44-62), so a given
//                     assignment yields bit-identical centroids; an empty cell
//                     takes a copy of its reseed row (:63-66)
#include "kmeans_kernels.hpp"
#include "primitives.hpp"


#include <stdexcept>
#include <string>

namespace mflat_amd {

static void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

__global__ void iota_kernel(int* __restrict__ v, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) v[i] = i;
}

__global__ void cell_counts_kernel(const int* __restrict__ cell, int n, int* __restrict__ counts) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) atomicAdd(&counts[cell[i]], 1);
}

// dst row i = src row idx[i] (row-major, any dim)
__global__ void gather_points_kernel(const float* __restrict__ src, const int* __restrict__ idx, int n, int dim,
                                     float* __restrict__ dst) {
    const int64_t total = (int64_t)n * dim;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = e / dim;
        dst[e] = src[(int64_t)idx[i] * dim + (e - i * dim)];
    }
}

__global__ void __launch_bounds__(256) update_centroids_kernel(const float* __restrict__ pts, int dim,
                                                               const int* __restrict__ order,
                                                               const int* __restrict__ cellStart,
                                                               const int* __restrict__ reseed,
                                                               float* __restrict__ centroids) {
    const int c = blockIdx.x;
    const int beg = cellStart[c], end = cellStart[c + 1];
    float* ce = centroids + (int64_t)c * dim;
    if (end == beg) {
        const int r = reseed[c];
        for (int d = threadIdx.x; d < dim; d += blockDim.x) ce[d] = pts[(int64_t)r * dim + d];
        return;
    }
    const double cnt = (double)(end - beg);
    for (int d = threadIdx.x; d < dim; d += blockDim.x) {
        double s = 0.0;
        int e = beg;
        // loads four rows ahead; the additions stay in point order
        for (; e + 4 <= end; e += 4) {
            const float v0 = pts[(int64_t)order[e] * dim + d];
            const float v1 = pts[(int64_t)order[e + 1] * dim + d];
            const float v2 = pts[(int64_t)order[e + 2] * dim + d];
            const float v3 = pts[(int64_t)order[e + 3] * dim + d];
            s += v0;
            s += v1;
            s += v2;
            s += v3;
        }
        for (; e < end; ++e) s += pts[(int64_t)order[e] * dim + d];
        ce[d] = (float)(s / cnt);
    }
}

CellGrouping::~CellGrouping() { release(); }

void CellGrouping::release() {
    for (void** p : {&iota, &keysOut, &temp}) {
        if (*p) (void)hipFree(*p);
        *p = nullptr;
    }
    cap = 0;
    tempBytes = 0;
}

void CellGrouping::group(const int* cell, int n, int nlist, int* orderOut, int* countsOut, hipStream_t s) {
    if (n <= 0) return;
    if (n > cap) {
        release();
        check(hipMalloc(&iota, (size_t)n * sizeof(int)), "hipMalloc(iota)");
        check(hipMalloc(&keysOut, (size_t)n * sizeof(int)), "hipMalloc(keys)");
        cap = n;
    }
    int bits = 1;
    while ((1 << bits) < nlist) ++bits;
    const size_t need = radix_sort_temp_bytes(n, bits);
    if (need > tempBytes) {
        if (temp) (void)hipFree(temp);
        temp = nullptr;
        check(hipMalloc(&temp, need), "hipMalloc(sort temp)");
        tempBytes = need;
    }
    iota_kernel<<<(n + 255) / 256, 256, 0, s>>>((int*)iota, n);
    check(hipGetLastError(), "iota");
    launch_radix_sort_pairs(cell, (int*)keysOut, (const int*)iota, orderOut, n, bits, temp, s);
    check(hipMemsetAsync(countsOut, 0, (size_t)nlist * sizeof(int), s), "hipMemsetAsync(counts)");
    cell_counts_kernel<<<(n + 255) / 256, 256, 0, s>>>(cell, n, countsOut);
    check(hipGetLastError(), "cell_counts");
}

void launch_gather_points(const float* src, const int* idx, int n, int dim, float* dst, hipStream_t s) {
    if (n <= 0) return;
    int64_t g = ((int64_t)n * dim + 255) / 256;
    if (g > 65536) g = 65536;
    gather_points_kernel<<<(int)g, 256, 0, s>>>(src, idx, n, dim, dst);
    check(hipGetLastError(), "gather_points");
}

void launch_update_centroids(const float* pts, int dim, const int* order, const int* cellStart, const int* reseed,
                             int nlist, float* centroids, hipStream_t s) {
    if (nlist <= 0) return;
    update_centroids_kernel<<<nlist, 256, 0, s>>>(pts, dim, order, cellStart, reseed, centroids);
    check(hipGetLastError(), "update_centroids");
}

}  // namespace mflat_amd
