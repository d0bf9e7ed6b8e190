// SPDX-License-Identifier: Apache-2.0
// ivf_kernels.hpp -- device helpers of the IVF index: the cell-major layout
// build and the per-search work tables of the fine scan (the scan itself is
// launch_scan_ivf in kernels.hpp).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <vector>

namespace mflat_amd {

// v[r][c] *= inv[r] for r < n (row-major, dim columns)
void launch_scale_rows(float* v, int64_t n, int dim, const float* inv, hipStream_t s);

// dst row r = src row idx[r], or zeros where idx[r] < 0 (row-major fp32, r < n)
void launch_gather_rows_or_zero(const float* src, const int* idx, int64_t n, int dim, float* dst, hipStream_t s);

// dst row r = src row idx[r] for r < n (int32 rows of `width` elements)
void launch_gather_i32(const int* src, const int* idx, int n, int width, int* dst, hipStream_t s);

// Scan positions: pos[q * np + r] = sum of cellSize[probe[q * np + r']] over
// r' < r -- where the probe-rank-r cell's first row falls in query q's scan
// order (cells in probe order, rows in cell order), for q < m.
void launch_ivf_positions(const int* probe, int m, int np, const int* cellSize, int* pos, hipStream_t s);

constexpr int kIvfNarrow = 32;   // entries per narrow work item (one 32-query block)

// Work table of one fine-scan pass over the entries e = q * np + r of queries
// q < m and ranks r < ranks (ranks = 1: the nearest cell only; ranks = np: all):
//   ent        the entries grouped by cell (within a cell in no particular
//              order on the device; ascending e from buildHost)
//   work[w]    wide items (cell, first entry, entries <= wideW, 0): each
//              cell's entries in runs of wideW, cells in the order cellOrder
//              gives (decreasing size)
//   workN[w]   narrow items (entries <= 32): the last n mod 128 entries of a
//              cell when at most narrowMax of them remain (else they take one
//              more wide item); narrowMax = 96 balances the two tile costs,
//              0 makes every item wide, < 0 every item narrow
//   nwork      device ints: wide, narrow item counts
// maxWork() / maxWorkNarrow() bound them (the grids of the scan launches).
// Keeps its scratch between calls.
struct IvfWorkTable {
    int wideW = 128;   // entries per wide work item (set before build)
    int* ent = nullptr;
    int4* work = nullptr;
    int4* workN = nullptr;
    int* nwork = nullptr;
    int maxWork(int m, int ranks, int nlist) const;
    int maxWorkNarrow(int m, int ranks, int nlist, int narrowMax) const;
    // pos (nullable): scan positions (launch_ivf_positions); entries whose
    // cell starts at posLimit or later are left out.
    void build(const int* probe, int m, int np, int ranks, int nlist, const int* cellOrder, int narrowMax,
               hipStream_t s, const int* pos = nullptr, int posLimit = 0);
    // The same table built on the host from host probes (m x np, all ranks)
    // and a host cell order, then uploaded: for the few queries of a retry,
    // where the device sort's fixed cost dominates.
    void buildHost(const int* probe, int m, int np, int nlist, const int* cellOrder, int narrowMax, hipStream_t s);
    ~IvfWorkTable();
    void release();

private:
    int* keysIn = nullptr;
    int* keysOut = nullptr;
    int* valsIn = nullptr;
    int* eEnd = nullptr;
    int* eStart = nullptr;
    int* tiles = nullptr;
    int* tEnd = nullptr;
    int* tilesN = nullptr;
    int* tEndN = nullptr;
    int* hist = nullptr;      // counting-sort build: per-block cell counts, cell-major
    int* histOff = nullptr;   // ... and their exclusive sums
    int64_t capHist = 0;
    void* temp = nullptr;
    size_t tempBytes = 0;
    std::vector<int> hEnt, hCnt, hStart;
    std::vector<int4> hWork, hWorkN;
    void reserve(int ne, int mw, int mn, int nlist);
    int capE = 0, capWork = 0, capWorkN = 0, capCells = 0;
};

// In place: ids[q * k + i] (a scan position, or -1) -> the original row id
// rid[cellStart[probe[q * np + r]] + position - pos[q * np + r]] of the rank r
// whose cell holds that position (q < m).
void launch_ivf_finalize(int32_t* ids, int m, int k, const int* pos, const int* probe, int np,
                         const int* cellStart, const int* rid, hipStream_t s);

}  // namespace mflat_amd
