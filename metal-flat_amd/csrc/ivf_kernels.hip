// SPDX-License-Identifier: Apache-2.0
// ivf_kernels.hip -- device helpers of the IVF index (ivf_kernels.hpp).
//
// The fine scan visits, for every query, the rows of its nprobe probed cells
// in probe order; a row's place in that sequence (its scan position) is the
// secondary ranking key, so ties keep the row scanned first, as the
// reference's strict '>' insertion over cells in probe order does
// (src/IvfIndex.mm:535-552). Work is cell-major: every (query, probe rank)
// entry is grouped with the other entries of its cell, and each run of up to
// 128 entries of one cell is one work item of the scan.
#include "ivf_kernels.hpp"

#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <stdexcept>
#include <string>

#include "kernels.hpp"

namespace mflat_amd {

static void check(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) throw std::bad_alloc();
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

static int grid_of(int64_t n, int block, int cap = 65536) {
    const int64_t g = (n + block - 1) / block;
    return (int)std::max<int64_t>(1, std::min<int64_t>(g, cap));
}

__global__ void scale_rows_kernel(float* __restrict__ v, int64_t n, int dim, const float* __restrict__ inv) {
    const int64_t total = n * dim;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x)
        v[e] *= inv[e / dim];
}

__global__ void gather_rows_or_zero_kernel(const float* __restrict__ src, const int* __restrict__ idx, int64_t n,
                                           int dim, float* __restrict__ dst) {
    const int64_t total = n * dim;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / dim;
        const int i = idx[r];
        dst[e] = i >= 0 ? src[(int64_t)i * dim + (e - r * dim)] : 0.0f;
    }
}

__global__ void gather_i32_kernel(const int* __restrict__ src, const int* __restrict__ idx, int n, int width,
                                  int* __restrict__ dst) {
    const int64_t total = (int64_t)n * width;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / width;
        dst[e] = src[(int64_t)idx[r] * width + (e - r * width)];
    }
}

// one thread per query: an exclusive running sum over its probe ranks
__global__ void ivf_positions_kernel(const int* __restrict__ probe, int m, int np, const int* __restrict__ cellSize,
                                     int* __restrict__ pos) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= m) return;
    const int64_t b = (int64_t)q * np;
    int run = 0;
    for (int r = 0; r < np; ++r) {
        pos[b + r] = run;
        const int c = probe[b + r];
        run += c >= 0 ? cellSize[c] : 0;   // -1: no cell (a query without finite distances)
    }
}

// entries i < m * ranks of the pass: e = (i / ranks) * np + i % ranks. An
// entry without a cell (probe -1) sorts after every cell and is never scanned.
__global__ void ivf_entries_kernel(const int* __restrict__ probe, int m, int np, int ranks, int nlist,
                                   int* __restrict__ keys, int* __restrict__ vals, int* __restrict__ counts) {
    const int64_t n = (int64_t)m * ranks;
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int q = (int)(i / ranks);
    const int e = q * np + (int)(i - (int64_t)q * ranks);
    const int c = probe[e];
    const bool ok = c >= 0 && c < nlist;
    keys[i] = ok ? c : nlist;
    vals[i] = e;
    if (ok) atomicAdd(&counts[c], 1);
}

// tiles[i] = work items of cell cellOrder[i]
__global__ void ivf_tiles_kernel(const int* __restrict__ cellOrder, const int* __restrict__ counts, int nlist,
                                 int* __restrict__ tiles) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < nlist) tiles[i] = (counts[cellOrder[i]] + kBN - 1) / kBN;
}

__global__ void ivf_work_kernel(const int* __restrict__ cellOrder, const int* __restrict__ counts,
                                const int* __restrict__ eStart, const int* __restrict__ tEnd, int nlist,
                                int4* __restrict__ work, int* __restrict__ nwork) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nlist) return;
    const int c = cellOrder[i];
    const int cnt = counts[c];
    const int nt = (cnt + kBN - 1) / kBN;
    const int t0 = tEnd[i] - nt;
    for (int t = 0; t < nt; ++t)
        work[t0 + t] = make_int4(c, eStart[c] + t * kBN, min(kBN, cnt - t * kBN), 0);
    if (i == nlist - 1) *nwork = tEnd[i];
}

__global__ void ivf_finalize_kernel(int32_t* __restrict__ ids, int m, int k, const int* __restrict__ pos,
                                    const int* __restrict__ probe, int np, const int* __restrict__ cellStart,
                                    const int* __restrict__ rid) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= (int64_t)m * k) return;
    const int p = ids[t];
    if (p < 0) return;
    const int64_t b = (t / k) * np;
    // the last rank whose first position is <= p holds p (empty cells share
    // their successor's first position and come before it)
    int lo = 0, hi = np - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (pos[b + mid] <= p) lo = mid;
        else hi = mid - 1;
    }
    ids[t] = rid[cellStart[probe[b + lo]] + (p - pos[b + lo])];
}

void launch_scale_rows(float* v, int64_t n, int dim, const float* inv, hipStream_t s) {
    if (n <= 0) return;
    scale_rows_kernel<<<grid_of(n * dim, 256), 256, 0, s>>>(v, n, dim, inv);
    check(hipGetLastError(), "scale_rows");
}

void launch_gather_rows_or_zero(const float* src, const int* idx, int64_t n, int dim, float* dst, hipStream_t s) {
    if (n <= 0) return;
    gather_rows_or_zero_kernel<<<grid_of(n * dim, 256), 256, 0, s>>>(src, idx, n, dim, dst);
    check(hipGetLastError(), "gather_rows_or_zero");
}

void launch_gather_i32(const int* src, const int* idx, int n, int width, int* dst, hipStream_t s) {
    if (n <= 0 || width <= 0) return;
    gather_i32_kernel<<<grid_of((int64_t)n * width, 256), 256, 0, s>>>(src, idx, n, width, dst);
    check(hipGetLastError(), "gather_i32");
}

void launch_ivf_positions(const int* probe, int m, int np, const int* cellSize, int* pos, hipStream_t s) {
    if (m <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    ivf_positions_kernel<<<(m + 255) / 256, 256, 0, s>>>(probe, m, np, cellSize, pos);
    prof_end(tok, s);
    check(hipGetLastError(), "ivf_positions");
}

void launch_ivf_finalize(int32_t* ids, int m, int k, const int* pos, const int* probe, int np,
                         const int* cellStart, const int* rid, hipStream_t s) {
    const int64_t n = (int64_t)m * k;
    if (n <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    ivf_finalize_kernel<<<(int)((n + 255) / 256), 256, 0, s>>>(ids, m, k, pos, probe, np, cellStart, rid);
    prof_end(tok, s);
    check(hipGetLastError(), "ivf_finalize");
}

int IvfWorkTable::maxWork(int m, int ranks, int nlist) const {
    const int64_t e = (int64_t)m * ranks;
    const int64_t w = (e + kBN - 1) / kBN + nlist;
    if (w > 0x7FFFFFFF) throw std::runtime_error("ivf: too many work items");
    return (int)w;
}

IvfWorkTable::~IvfWorkTable() { release(); }

void IvfWorkTable::release() {
    for (void** p : {(void**)&ent, (void**)&work, (void**)&nwork, (void**)&keysIn, (void**)&keysOut,
                     (void**)&valsIn, (void**)&counts, (void**)&eStart, (void**)&tiles, (void**)&tEnd, &temp}) {
        if (*p) (void)hipFree(*p);
        *p = nullptr;
    }
    tempBytes = 0;
    capE = capWork = capCells = 0;
}

void IvfWorkTable::build(const int* probe, int m, int np, int ranks, int nlist, const int* cellOrder,
                         hipStream_t s) {
    const int64_t ne64 = (int64_t)m * ranks;
    if (m <= 0 || ranks < 1 || ranks > np || nlist < 1) throw std::runtime_error("ivf work table: bad sizes");
    if (ne64 > 0x7FFFFFFF) throw std::runtime_error("ivf work table: too many entries");
    const int ne = (int)ne64;
    const int mw = maxWork(m, ranks, nlist);
    if (ne > capE) {
        for (int** p : {&ent, &keysIn, &keysOut, &valsIn}) {
            if (*p) (void)hipFree(*p);
            *p = nullptr;
        }
        for (int** p : {&ent, &keysIn, &keysOut, &valsIn}) check(hipMalloc((void**)p, (size_t)ne * sizeof(int)), "hipMalloc(entries)");
        capE = ne;
    }
    if (mw > capWork) {
        if (work) (void)hipFree(work);
        work = nullptr;
        check(hipMalloc((void**)&work, (size_t)mw * sizeof(int4)), "hipMalloc(work)");
        capWork = mw;
    }
    if (nlist > capCells) {
        for (int** p : {&counts, &eStart, &tiles, &tEnd}) {
            if (*p) (void)hipFree(*p);
            *p = nullptr;
        }
        for (int** p : {&counts, &eStart, &tiles, &tEnd})
            check(hipMalloc((void**)p, (size_t)nlist * sizeof(int)), "hipMalloc(cells)");
        capCells = nlist;
    }
    if (!nwork) check(hipMalloc((void**)&nwork, sizeof(int)), "hipMalloc(nwork)");

    int bits = 1;
    while ((1 << bits) <= nlist) ++bits;   // keys 0 .. nlist
    size_t needSort = 0, needEx = 0, needIn = 0;
    check(hipcub::DeviceRadixSort::SortPairs(nullptr, needSort, (const int*)keysIn, keysOut, (const int*)valsIn,
                                             ent, ne, 0, bits, s),
          "SortPairs (size)");
    check(hipcub::DeviceScan::ExclusiveSum(nullptr, needEx, (const int*)counts, eStart, nlist, s), "ExclusiveSum (size)");
    check(hipcub::DeviceScan::InclusiveSum(nullptr, needIn, (const int*)tiles, tEnd, nlist, s), "InclusiveSum (size)");
    const size_t need = std::max({needSort, needEx, needIn, (size_t)16});
    if (need > tempBytes) {
        if (temp) (void)hipFree(temp);
        temp = nullptr;
        check(hipMalloc(&temp, need), "hipMalloc(ivf temp)");
        tempBytes = need;
    }

    void* tok;
    prof_begin(kFamPrep, s, &tok);
    check(hipMemsetAsync(counts, 0, (size_t)nlist * sizeof(int), s), "hipMemsetAsync(counts)");
    ivf_entries_kernel<<<(int)((ne + 255) / 256), 256, 0, s>>>(probe, m, np, ranks, nlist, keysIn, valsIn, counts);
    check(hipGetLastError(), "ivf_entries");
    size_t t = tempBytes;
    check(hipcub::DeviceRadixSort::SortPairs(temp, t, (const int*)keysIn, keysOut, (const int*)valsIn, ent, ne, 0,
                                             bits, s),
          "SortPairs");
    t = tempBytes;
    check(hipcub::DeviceScan::ExclusiveSum(temp, t, (const int*)counts, eStart, nlist, s), "ExclusiveSum");
    ivf_tiles_kernel<<<(nlist + 255) / 256, 256, 0, s>>>(cellOrder, counts, nlist, tiles);
    check(hipGetLastError(), "ivf_tiles");
    t = tempBytes;
    check(hipcub::DeviceScan::InclusiveSum(temp, t, (const int*)tiles, tEnd, nlist, s), "InclusiveSum");
    ivf_work_kernel<<<(nlist + 255) / 256, 256, 0, s>>>(cellOrder, counts, eStart, tEnd, nlist, work, nwork);
    check(hipGetLastError(), "ivf_work");
    prof_end(tok, s);
}

}  // namespace mflat_amd
