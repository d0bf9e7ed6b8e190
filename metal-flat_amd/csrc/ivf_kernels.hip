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
#include "primitives.hpp"


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

// one wave per query: an exclusive running sum over its probe ranks, 64
// ranks at a time
__global__ void __launch_bounds__(256) ivf_positions_kernel(const int* __restrict__ probe, int m, int np,
                                                            const int* __restrict__ cellSize, int* __restrict__ pos) {
    const int q = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (q >= m) return;
    const int64_t b = (int64_t)q * np;
    int run = 0;
    for (int r0 = 0; r0 < np; r0 += 64) {
        const int r = r0 + lane;
        const int c = r < np ? probe[b + r] : -1;
        const int v = c >= 0 ? cellSize[c] : 0;   // -1: no cell (a query without finite distances)
        int x = v;
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(x, off, 64);
            if (lane >= off) x += t;
        }
        if (r < np) pos[b + r] = run + x - v;
        run += __shfl(x, 63, 64);
    }
}

// entries i < m * ranks of the pass: e = (i / ranks) * np + i % ranks. An
// entry without a cell (probe -1), or (pos non-null) whose cell starts at scan
// position posLimit or later, sorts after every cell and is never scanned.
__global__ void ivf_entries_kernel(const int* __restrict__ probe, int m, int np, int ranks, int nlist,
                                   const int* __restrict__ pos, int posLimit, int* __restrict__ keys,
                                   int* __restrict__ vals) {
    const int64_t n = (int64_t)m * ranks;
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int q = (int)(i / ranks);
    const int e = q * np + (int)(i - (int64_t)q * ranks);
    const int c = probe[e];
    const bool ok = c >= 0 && c < nlist && (pos == nullptr || pos[e] < posLimit);
    keys[i] = ok ? c : nlist;
    vals[i] = e;
}

// Each cell's run [eStart[c], eEnd[c]) in the sorted keys (both pre-zeroed:
// cells without entries keep an empty run) -- no atomics, whose contention on
// the few hot cells of a batch costs more than the sort.
__global__ void ivf_runs_kernel(const int* __restrict__ keys, int n, int nlist, int* __restrict__ eStart,
                                int* __restrict__ eEnd) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int c = keys[i];
    if (c >= nlist) return;
    if (i == 0 || keys[i - 1] != c) eStart[c] = i;
    if (i == n - 1 || keys[i + 1] != c) eEnd[c] = i + 1;
}

// A cell's n entries: wide tiles of W, then the rest in narrow tiles of
// kIvfNarrow -- unless more than narrowMax remain, which take one more wide
// tile (a tile's cost is its rows times its width; narrowMax = W - kIvfNarrow:
// up to three narrow tiles are cheaper than a wide one). narrowMax = 0: wide
// only; narrowMax < 0: narrow only.
__host__ __device__ inline void ivf_split(int n, int W, int narrowMax, int& wide, int& narrow) {
    if (narrowMax < 0) {
        wide = 0;
        narrow = (n + kIvfNarrow - 1) / kIvfNarrow;
        return;
    }
    wide = n / W;
    const int rem = n - wide * W;
    if (rem > narrowMax) {
        ++wide;
        narrow = 0;
    } else {
        narrow = (rem + kIvfNarrow - 1) / kIvfNarrow;
    }
}

// tiles of cell cellOrder[i]: wide in tilesW[i], narrow in tilesN[i]
__global__ void ivf_tiles_kernel(const int* __restrict__ cellOrder, const int* __restrict__ eStart,
                                 const int* __restrict__ eEnd, int nlist, int W, int narrowMax,
                                 int* __restrict__ tilesW, int* __restrict__ tilesN) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nlist) return;
    const int c = cellOrder[i];
    int w, nn;
    ivf_split(eEnd[c] - eStart[c], W, narrowMax, w, nn);
    tilesW[i] = w;
    tilesN[i] = nn;
}

__global__ void ivf_work_kernel(const int* __restrict__ cellOrder, const int* __restrict__ eEnd,
                                const int* __restrict__ eStart, const int* __restrict__ tEndW,
                                const int* __restrict__ tEndN, int nlist, int W, int narrowMax,
                                int4* __restrict__ work, int4* __restrict__ workN, int* __restrict__ nwork) {
    // one wave per cell: its lanes write the cell's items
    const int i = blockIdx.x * (blockDim.x / 64) + (int)(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (i >= nlist) return;
    const int c = cellOrder[i];
    const int e0 = eStart[c];
    const int cnt = eEnd[c] - e0;
    int nw, nn;
    ivf_split(cnt, W, narrowMax, nw, nn);
    const int t0 = tEndW[i] - nw;
    for (int t = lane; t < nw; t += 64) work[t0 + t] = make_int4(c, e0 + t * W, min(W, cnt - t * W), 0);
    const int n0 = tEndN[i] - nn;
    const int base = nw * W;
    for (int t = lane; t < nn; t += 64)
        workN[n0 + t] = make_int4(c, e0 + base + t * kIvfNarrow, min(kIvfNarrow, cnt - base - t * kIvfNarrow), 0);
    if (i == nlist - 1 && lane == 0) {
        nwork[0] = tEndW[i];
        nwork[1] = tEndN[i];
    }
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

// Counting-sort build of the work table (nlist <= kHistCells): block b
// counts the entries [b * chunk, (b + 1) * chunk) per cell in LDS into
// H[c * G + b]; an exclusive scan of H (cell-major) gives each block its first
// slot in every cell's run; the scatter then places the entries (their order
// within a cell follows LDS atomics). Three launches where a radix sort of the
// same keys takes a merge cascade of some twenty; two more write the items.
constexpr int kHistCells = 32768;
constexpr int kHistBlock = 1024;

__device__ __forceinline__ int ivf_entry_cell(const int* __restrict__ probe, int np, int ranks, int nlist,
                                              const int* __restrict__ pos, int posLimit, int64_t i, int& e) {
    const int q = (int)(i / ranks);
    e = q * np + (int)(i - (int64_t)q * ranks);
    const int c = probe[e];
    return (c >= 0 && c < nlist && (pos == nullptr || pos[e] < posLimit)) ? c : -1;
}

__global__ void __launch_bounds__(kHistBlock) ivf_hist_kernel(const int* __restrict__ probe, int m, int np,
                                                              int ranks, int nlist, const int* __restrict__ pos,
                                                              int posLimit, int chunk, int G, int* __restrict__ H) {
    extern __shared__ int sH[];
    for (int c = threadIdx.x; c < nlist; c += kHistBlock) sH[c] = 0;
    __syncthreads();
    const int64_t n = (int64_t)m * ranks;
    const int64_t i0 = (int64_t)blockIdx.x * chunk;
    const int64_t i1 = i0 + chunk < n ? i0 + chunk : n;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += kHistBlock) {
        int e;
        const int c = ivf_entry_cell(probe, np, ranks, nlist, pos, posLimit, i, e);
        if (c >= 0) atomicAdd(&sH[c], 1);
    }
    __syncthreads();
    for (int c = threadIdx.x; c < nlist; c += kHistBlock) H[(int64_t)c * G + blockIdx.x] = sH[c];
}

__global__ void __launch_bounds__(kHistBlock) ivf_scatter_kernel(const int* __restrict__ probe, int m, int np,
                                                                 int ranks, int nlist, const int* __restrict__ pos,
                                                                 int posLimit, int chunk, int G,
                                                                 const int* __restrict__ H, const int* __restrict__ O,
                                                                 int* __restrict__ ent, int* __restrict__ eStart,
                                                                 int* __restrict__ eEnd) {
    extern __shared__ int sCur[];
    for (int c = threadIdx.x; c < nlist; c += kHistBlock) sCur[c] = O[(int64_t)c * G + blockIdx.x];
    __syncthreads();
    const int64_t n = (int64_t)m * ranks;
    const int64_t i0 = (int64_t)blockIdx.x * chunk;
    const int64_t i1 = i0 + chunk < n ? i0 + chunk : n;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += kHistBlock) {
        int e;
        const int c = ivf_entry_cell(probe, np, ranks, nlist, pos, posLimit, i, e);
        if (c >= 0) ent[atomicAdd(&sCur[c], 1)] = e;
    }
    if (blockIdx.x == 0)
        for (int c = threadIdx.x; c < nlist; c += kHistBlock) {
            const int64_t last = (int64_t)c * G + G - 1;
            eStart[c] = O[(int64_t)c * G];
            eEnd[c] = O[last] + H[last];
        }
}

// One block: every cell's item counts (ivf_split) and their inclusive sums in
// cellOrder order (tEndW / tEndN, as the scans of the radix path give them).
__global__ void __launch_bounds__(kHistBlock) ivf_tile_sums_kernel(const int* __restrict__ cellOrder,
                                                                   const int* __restrict__ eStart,
                                                                   const int* __restrict__ eEnd, int nlist, int W,
                                                                   int narrowMax, int* __restrict__ tEndW,
                                                                   int* __restrict__ tEndN) {
    constexpr int kWaves = kHistBlock / 64;
    __shared__ int sW[kWaves], sN[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int per = (nlist + kHistBlock - 1) / kHistBlock;
    const int i0 = min(nlist, tid * per), i1 = min(nlist, i0 + per);
    int sw = 0, sn = 0;
    for (int i = i0; i < i1; ++i) {
        const int c = cellOrder[i];
        int w, nn;
        ivf_split(eEnd[c] - eStart[c], W, narrowMax, w, nn);
        sw += w;
        sn += nn;
    }
    int xw = sw, xn = sn;
    for (int off = 1; off < 64; off <<= 1) {
        const int a = __shfl_up(xw, off, 64), b = __shfl_up(xn, off, 64);
        if (lane >= off) {
            xw += a;
            xn += b;
        }
    }
    if (lane == 63) {
        sW[wave] = xw;
        sN[wave] = xn;
    }
    __syncthreads();
    int bw = xw - sw, bn = xn - sn;
    for (int w = 0; w < wave; ++w) {
        bw += sW[w];
        bn += sN[w];
    }
    for (int i = i0; i < i1; ++i) {
        const int c = cellOrder[i];
        int w, nn;
        ivf_split(eEnd[c] - eStart[c], W, narrowMax, w, nn);
        bw += w;
        bn += nn;
        tEndW[i] = bw;
        tEndN[i] = bn;
    }
}

void launch_ivf_positions(const int* probe, int m, int np, const int* cellSize, int* pos, hipStream_t s) {
    if (m <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    ivf_positions_kernel<<<(m + 3) / 4, 256, 0, s>>>(probe, m, np, cellSize, pos);
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
    const int64_t w = (e + wideW - 1) / wideW + nlist;
    if (w > 0x7FFFFFFF) throw std::runtime_error("ivf: too many work items");
    return (int)w;
}

int IvfWorkTable::maxWorkNarrow(int m, int ranks, int nlist, int narrowMax) const {
    const int64_t e = (int64_t)m * ranks;
    int64_t w = (e + kIvfNarrow - 1) / kIvfNarrow + nlist;
    if (narrowMax >= 0)   // at most ceil(min(narrowMax, wideW - 1) / kIvfNarrow) per cell
        w = std::min<int64_t>(w, (int64_t)nlist * ((std::min(narrowMax, wideW - 1) + kIvfNarrow - 1) / kIvfNarrow));
    if (w > 0x7FFFFFFF) throw std::runtime_error("ivf: too many work items");
    return (int)w;
}

IvfWorkTable::~IvfWorkTable() { release(); }

void IvfWorkTable::release() {
    for (void** p : {(void**)&ent, (void**)&work, (void**)&workN, (void**)&nwork, (void**)&keysIn, (void**)&keysOut,
                     (void**)&valsIn, (void**)&eEnd, (void**)&eStart, (void**)&tiles, (void**)&tEnd,
                     (void**)&tilesN, (void**)&tEndN, (void**)&hist, (void**)&histOff, &temp}) {
        if (*p) (void)hipFree(*p);
        *p = nullptr;
    }
    tempBytes = 0;
    capE = capWork = capWorkN = capCells = 0;
    capHist = 0;
}

void IvfWorkTable::reserve(int ne, int mw, int mn, int nlist) {
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
    if (mn > capWorkN) {
        if (workN) (void)hipFree(workN);
        workN = nullptr;
        check(hipMalloc((void**)&workN, (size_t)mn * sizeof(int4)), "hipMalloc(work)");
        capWorkN = mn;
    }
    if (nlist > capCells) {
        for (int** p : {&eEnd, &eStart, &tiles, &tEnd, &tilesN, &tEndN}) {
            if (*p) (void)hipFree(*p);
            *p = nullptr;
        }
        for (int** p : {&eEnd, &eStart, &tiles, &tEnd, &tilesN, &tEndN})
            check(hipMalloc((void**)p, (size_t)nlist * sizeof(int)), "hipMalloc(cells)");
        capCells = nlist;
    }
    if (!nwork) check(hipMalloc((void**)&nwork, 2 * sizeof(int)), "hipMalloc(nwork)");
}

void IvfWorkTable::build(const int* probe, int m, int np, int ranks, int nlist, const int* cellOrder,
                         int narrowMax, hipStream_t s, const int* pos, int posLimit) {
    const int64_t ne64 = (int64_t)m * ranks;
    if (m <= 0 || ranks < 1 || ranks > np || nlist < 1) throw std::runtime_error("ivf work table: bad sizes");
    if (ne64 > 0x7FFFFFFF) throw std::runtime_error("ivf work table: too many entries");
    const int ne = (int)ne64;
    const int mw = maxWork(m, ranks, nlist);
    const int mn = maxWorkNarrow(m, ranks, nlist, narrowMax);
    reserve(ne, mw, mn, nlist);

    if (nlist <= kHistCells) {
        const int chunk = (int)std::max<int64_t>(4096, (ne64 + 1023) / 1024);
        const int G = (int)((ne64 + chunk - 1) / chunk);
        const int64_t nh = (int64_t)nlist * G;
        if (nh > capHist) {
            for (int** p : {&hist, &histOff}) {
                if (*p) (void)hipFree(*p);
                *p = nullptr;
            }
            for (int** p : {&hist, &histOff}) check(hipMalloc((void**)p, (size_t)nh * sizeof(int)), "hipMalloc(hist)");
            capHist = nh;
        }
        const size_t need = std::max(scan_temp_bytes(nh), (size_t)16);
        if (need > tempBytes) {
            if (temp) (void)hipFree(temp);
            temp = nullptr;
            check(hipMalloc(&temp, need), "hipMalloc(ivf temp)");
            tempBytes = need;
        }
        static const bool attr = [] {
            for (const void* f : {(const void*)ivf_hist_kernel, (const void*)ivf_scatter_kernel})
                if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kHistCells * 4) != hipSuccess)
                    throw std::runtime_error("ivf work table: cannot raise the dynamic LDS limit");
            return true;
        }();
        (void)attr;
        const size_t lds = (size_t)nlist * sizeof(int);
        void* tok;
        prof_begin(kFamPrep, s, &tok);
        ivf_hist_kernel<<<G, kHistBlock, lds, s>>>(probe, m, np, ranks, nlist, pos, posLimit, chunk, G, hist);
        check(hipGetLastError(), "ivf_hist");
        launch_scan_i32(hist, histOff, nh, false, temp, s);
        ivf_scatter_kernel<<<G, kHistBlock, lds, s>>>(probe, m, np, ranks, nlist, pos, posLimit, chunk, G, hist,
                                                      histOff, ent, eStart, eEnd);
        check(hipGetLastError(), "ivf_scatter");
        ivf_tile_sums_kernel<<<1, kHistBlock, 0, s>>>(cellOrder, eStart, eEnd, nlist, wideW, narrowMax, tEnd, tEndN);
        check(hipGetLastError(), "ivf_tile_sums");
        ivf_work_kernel<<<(nlist + 3) / 4, 256, 0, s>>>(cellOrder, eEnd, eStart, tEnd, tEndN, nlist, wideW,
                                                         narrowMax, work, workN, nwork);
        check(hipGetLastError(), "ivf_work");
        prof_end(tok, s);
        return;
    }

    int bits = 1;
    while ((1 << bits) <= nlist) ++bits;   // keys 0 .. nlist
    const size_t need = std::max({radix_sort_temp_bytes(ne, bits), scan_temp_bytes(nlist), (size_t)16});
    if (need > tempBytes) {
        if (temp) (void)hipFree(temp);
        temp = nullptr;
        check(hipMalloc(&temp, need), "hipMalloc(ivf temp)");
        tempBytes = need;
    }

    void* tok;
    prof_begin(kFamPrep, s, &tok);
    check(hipMemsetAsync(eEnd, 0, (size_t)nlist * sizeof(int), s), "hipMemsetAsync(eEnd)");
    check(hipMemsetAsync(eStart, 0, (size_t)nlist * sizeof(int), s), "hipMemsetAsync(eStart)");
    ivf_entries_kernel<<<(int)((ne + 255) / 256), 256, 0, s>>>(probe, m, np, ranks, nlist, pos, posLimit, keysIn,
                                                                valsIn);
    check(hipGetLastError(), "ivf_entries");
    launch_radix_sort_pairs(keysIn, keysOut, valsIn, ent, ne, bits, temp, s);
    ivf_runs_kernel<<<(ne + 255) / 256, 256, 0, s>>>(keysOut, ne, nlist, eStart, eEnd);
    check(hipGetLastError(), "ivf_runs");
    ivf_tiles_kernel<<<(nlist + 255) / 256, 256, 0, s>>>(cellOrder, eStart, eEnd, nlist, wideW, narrowMax, tiles,
                                                          tilesN);
    check(hipGetLastError(), "ivf_tiles");
    launch_scan_i32(tiles, tEnd, nlist, true, temp, s);
    launch_scan_i32(tilesN, tEndN, nlist, true, temp, s);
    ivf_work_kernel<<<(nlist + 3) / 4, 256, 0, s>>>(cellOrder, eEnd, eStart, tEnd, tEndN, nlist, wideW, narrowMax,
                                                     work, workN, nwork);
    check(hipGetLastError(), "ivf_work");
    prof_end(tok, s);
}

void IvfWorkTable::buildHost(const int* probe, int m, int np, int nlist, const int* cellOrder, int narrowMax,
                             hipStream_t s) {
    const int64_t ne64 = (int64_t)m * np;
    if (m <= 0 || np < 1 || nlist < 1 || ne64 > 0x7FFFFFFF) throw std::runtime_error("ivf work table: bad sizes");
    const int ne = (int)ne64;
    const int mw = maxWork(m, np, nlist);
    const int mn = maxWorkNarrow(m, np, nlist, narrowMax);
    reserve(ne, mw, mn, nlist);
    // counting sort of the entries by cell, ascending entry within a cell
    hCnt.assign((size_t)nlist + 1, 0);
    for (int e = 0; e < ne; ++e)
        if (probe[e] >= 0 && probe[e] < nlist) ++hCnt[(size_t)probe[e] + 1];
    hStart.assign((size_t)nlist + 1, 0);
    for (int c = 0; c < nlist; ++c) hStart[(size_t)c + 1] = hStart[(size_t)c] + hCnt[(size_t)c + 1];
    hEnt.assign((size_t)std::max(ne, 1), 0);
    std::vector<int> cur(hStart.begin(), hStart.end() - 1);
    for (int e = 0; e < ne; ++e)
        if (probe[e] >= 0 && probe[e] < nlist) hEnt[(size_t)cur[(size_t)probe[e]]++] = e;
    hWork.clear();
    hWorkN.clear();
    for (int i = 0; i < nlist; ++i) {
        const int c = cellOrder[i];
        const int e0 = hStart[(size_t)c], cnt = hCnt[(size_t)c + 1];
        int wide, narrow;
        ivf_split(cnt, wideW, narrowMax, wide, narrow);
        for (int t = 0; t < wide; ++t)
            hWork.push_back(make_int4(c, e0 + t * wideW, std::min(wideW, cnt - t * wideW), 0));
        const int base = wide * wideW;
        for (int t = 0; t < narrow; ++t)
            hWorkN.push_back(make_int4(c, e0 + base + t * kIvfNarrow, std::min(kIvfNarrow, cnt - base - t * kIvfNarrow), 0));
    }
    if ((int)hWork.size() > mw || (int)hWorkN.size() > mn) throw std::runtime_error("ivf work table: bound exceeded");
    const int counts[2] = {(int)hWork.size(), (int)hWorkN.size()};
    check(hipMemcpyAsync(ent, hEnt.data(), (size_t)ne * sizeof(int), hipMemcpyHostToDevice, s), "hipMemcpyAsync(ent)");
    if (counts[0])
        check(hipMemcpyAsync(work, hWork.data(), hWork.size() * sizeof(int4), hipMemcpyHostToDevice, s),
              "hipMemcpyAsync(work)");
    if (counts[1])
        check(hipMemcpyAsync(workN, hWorkN.data(), hWorkN.size() * sizeof(int4), hipMemcpyHostToDevice, s),
              "hipMemcpyAsync(work)");
    check(hipMemcpyAsync(nwork, counts, sizeof counts, hipMemcpyHostToDevice, s), "hipMemcpyAsync(nwork)");
    // the host vectors are the copies' sources: wait before they can change
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
}

}  // namespace mflat_amd
