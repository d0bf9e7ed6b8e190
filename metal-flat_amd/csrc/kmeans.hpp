// SPDX-License-Identifier: Apache-2.0
// kmeans.hpp -- k-means training of an IVF coarse quantizer on one MI355X.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mflat_amd {

// Trains nlist = min(nlistReq, n) centroids on n row-major points (host
// memory) and assigns every point; the loop of the reference's
// CoarseQuantizer::train over detail::kmeansGpu (src/CoarseQuantizer.mm:104-159,
// src/Internal.h:234-382) with every step on the device:
//   seeds     centroid c = point perm[c], perm a uniform permutation of the
//             points drawn from std::mt19937(12345) by shufflePermutation;
//   training  on the first min(n, maxPointsPerCentroid * nlist) points of perm
//             (0: all points, in their own order);
//   iters x   fused k = 1 assignment (strict '<': lowest centroid on ties),
//             then centroid = float(double sum / count) over the cell's points
//             in ascending training order; an empty cell takes training point
//             rng() % trainN (cells in ascending order);
//   final     assignment of all n points and its stable CSR (cell starts and
//             point ids in cell order, ascending within a cell).
// The seeding permutation is Fisher-Yates from the top: for i = n - 1 .. 1,
// u = rng() redrawn while u >= 2^32 - 2^32 mod (i + 1), swap(perm[i],
// perm[u mod (i + 1)]) -- the reference's std::shuffle draws are specific to
// its standard library, so the seeds differ from the reference's; everything
// after the seeding follows it.
// Outputs: centroids nlist x dim; assign n (nullable); cellStart nlist + 1
// (nullable); order n (nullable). Returns nlist. Throws NotReady without a
// usable device, BadArg for bad sizes.
int kmeansTrain(const float* points, int n, int dim, int nlistReq, int iters, int maxPointsPerCentroid,
                float* centroids, int32_t* assign, int32_t* cellStart, int32_t* order);

// The same on device memory, asynchronous on s except for the per-iteration
// cell counts: points n x dim, centroids nlist x dim, assign / order n
// (nullable) are device pointers, cellStart (nlist + 1, nullable) is host
// memory. Returns nlist.
// wrapSeeds: nlist = nlistReq even above n (seeds wrap around the permutation).
int kmeansTrainDevice(const float* points, int n, int dim, int nlistReq, int iters, int maxPointsPerCentroid,
                      float* centroids, int32_t* assign, int32_t* order, int32_t* cellStart, hipStream_t s,
                      bool wrapSeeds = false);

}  // namespace mflat_amd
