// SPDX-License-Identifier: Apache-2.0
// primitives.hip -- prefix sums and a stable LSD radix sort for gfx950.
//
// Scan: tiles of 2,048 ints (256 threads x 8 consecutive items); each tile is
// scanned in registers and LDS and its total written out; the totals are
// scanned the same way (recursively), then added back to their tiles.
//
// Radix sort: 4-bit digits, one pass per digit from the least significant.
// A pass is (1) a 16-bin histogram per tile of 1,024 elements, (2) an
// exclusive scan of the histograms in digit-major order (digit d of tile b at
// d * ntiles + b: every digit-d element of an earlier tile, and every element
// of a smaller digit, lands before), (3) a stable scatter. A tile is read in
// four rounds of 256 consecutive elements, one per thread; within a round a
// wave ranks its lanes among the lanes holding the same digit with four
// ballots (one per digit bit), the waves' per-digit counts are added in wave
// order and the tile's running counts carry over to the next round, so equal
// digits keep their input order.
#include "primitives.hpp"

#include <stdexcept>
#include <string>
#include <vector>

namespace mflat_amd {
namespace {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;
constexpr int kSortThreads = 256;
constexpr int kSortRounds = 4;
constexpr int kSortTile = kSortThreads * kSortRounds;
constexpr int kDigitBits = 4;
constexpr int kBins = 1 << kDigitBits;

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// One tile of the scan: thread-local sums of 8 items, a block scan of them,
// then the items rewritten. tile_sums (nullable) gets the tile's total.
__global__ void __launch_bounds__(kScanThreads) scan_tile_kernel(const int* __restrict__ in, int* __restrict__ out,
                                                                int64_t n, int inclusive, int* __restrict__ tile_sums) {
    __shared__ int sWave[kScanThreads / 64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)tid * kScanItems;
    int v[kScanItems];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
        v[i] = base + i < n ? in[base + i] : 0;
        sum += v[i];
    }
    int x = sum;   // inclusive scan of the thread sums within the wave
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(x, off, 64);
        if (lane >= off) x += t;
    }
    if (lane == 63) sWave[wave] = x;
    __syncthreads();
    int run = x - sum;
    for (int w = 0; w < wave; ++w) run += sWave[w];
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
        if (inclusive) run += v[i];
        if (base + i < n) out[base + i] = run;
        if (!inclusive) run += v[i];
    }
    if (tile_sums && tid == kScanThreads - 1) tile_sums[blockIdx.x] = run;
}

// out[i] += offs[tile of i]
__global__ void __launch_bounds__(kScanThreads) scan_add_kernel(int* __restrict__ out, int64_t n,
                                                               const int* __restrict__ offs) {
    const int64_t base = (int64_t)blockIdx.x * kScanTile + threadIdx.x;
    const int add = offs[blockIdx.x];
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
        const int64_t j = base + (int64_t)i * kScanThreads;
        if (j < n) out[j] += add;
    }
}

int64_t tiles_of(int64_t n) { return (n + kScanTile - 1) / kScanTile; }

void scan_rec(const int* in, int* out, int64_t n, bool inclusive, int* temp, hipStream_t s) {
    if (n <= 0) return;
    const int64_t nt = tiles_of(n);
    if (nt > 0x7FFFFFFF) throw std::runtime_error("scan: too many elements");
    int* sums = nt > 1 ? temp : nullptr;
    scan_tile_kernel<<<(int)nt, kScanThreads, 0, s>>>(in, out, n, inclusive ? 1 : 0, sums);
    check(hipGetLastError(), "scan_tile");
    if (nt > 1) {
        scan_rec(sums, sums, nt, false, temp + nt, s);   // exclusive scan of the tile totals, in place
        scan_add_kernel<<<(int)nt, kScanThreads, 0, s>>>(out, n, sums);
        check(hipGetLastError(), "scan_add");
    }
}

__global__ void __launch_bounds__(kSortThreads) radix_hist_kernel(const int* __restrict__ keys, int n, int shift,
                                                                 int ntiles, int* __restrict__ hist) {
    __shared__ int sCnt[kBins];
    const int tid = threadIdx.x;
    if (tid < kBins) sCnt[tid] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kSortTile;
    for (int r = 0; r < kSortRounds; ++r) {
        const int64_t e = base + r * kSortThreads + tid;
        if (e < n) atomicAdd(&sCnt[(keys[e] >> shift) & (kBins - 1)], 1);
    }
    __syncthreads();
    if (tid < kBins) hist[(int64_t)tid * ntiles + blockIdx.x] = sCnt[tid];
}

__global__ void __launch_bounds__(kSortThreads) radix_scatter_kernel(const int* __restrict__ keys,
                                                                    const int* __restrict__ vals, int n, int shift,
                                                                    int ntiles, const int* __restrict__ offs,
                                                                    int* __restrict__ keys_out,
                                                                    int* __restrict__ vals_out) {
    constexpr int NW = kSortThreads / 64;
    __shared__ int sBase[kBins];
    __shared__ int sWaveCnt[NW][kBins];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    if (tid < kBins) sBase[tid] = offs[(int64_t)tid * ntiles + blockIdx.x];
    if (tid < NW * kBins) sWaveCnt[tid / kBins][tid % kBins] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kSortTile;
    const unsigned long long below = (1ull << lane) - 1ull;
    for (int r = 0; r < kSortRounds; ++r) {
        const int64_t e = base + r * kSortThreads + tid;
        const bool valid = e < n;
        const int key = valid ? keys[e] : 0;
        const int val = valid ? vals[e] : 0;
        const int d = (key >> shift) & (kBins - 1);
        // lanes holding the same digit: the AND of the matching ballots of each bit
        unsigned long long peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < kDigitBits; ++b) {
            const unsigned long long ones = __ballot(valid && ((d >> b) & 1));
            peers &= ((d >> b) & 1) ? ones : ~ones;
        }
        const int rank = __popcll(peers & below);
        // the lowest lane of each digit group records the wave's count
        if (valid && rank == 0) sWaveCnt[wave][d] = __popcll(peers);
        __syncthreads();
        if (valid) {
            int pos = sBase[d] + rank;
            for (int w = 0; w < wave; ++w) pos += sWaveCnt[w][d];
            keys_out[pos] = key;
            vals_out[pos] = val;
        }
        __syncthreads();
        if (tid < kBins) {
            int t = 0;
            for (int w = 0; w < NW; ++w) t += sWaveCnt[w][tid];
            sBase[tid] += t;
        }
        __syncthreads();
        if (tid < NW * kBins) sWaveCnt[tid / kBins][tid % kBins] = 0;
        __syncthreads();
    }
}

int sort_tiles(int n) { return (n + kSortTile - 1) / kSortTile; }

}  // namespace

size_t scan_temp_bytes(int64_t n) {
    size_t words = 0;
    for (int64_t t = tiles_of(n); t > 1; t = tiles_of(t)) words += (size_t)t;
    return (words + 16) * sizeof(int);
}

void launch_scan_i32(const int* in, int* out, int64_t n, bool inclusive, void* temp, hipStream_t s) {
    scan_rec(in, out, n, inclusive, static_cast<int*>(temp), s);
}

size_t radix_sort_temp_bytes(int n, int bits) {
    (void)bits;
    const int64_t nt = sort_tiles(n);
    const int64_t nh = nt * kBins;
    // histograms, their scan, the scan's own temp, two ping-pong key/value buffers
    return (size_t)(2 * nh) * sizeof(int) + scan_temp_bytes(nh) + (size_t)4 * n * sizeof(int) + 256;
}

void launch_radix_sort_pairs(const int* keys_in, int* keys_out, const int* vals_in, int* vals_out, int n, int bits,
                             void* temp, hipStream_t s) {
    if (n <= 0) return;
    if (bits < 1 || bits > 31) throw std::runtime_error("radix sort: bits must be 1..31");
    const int nt = sort_tiles(n);
    const int64_t nh = (int64_t)nt * kBins;
    int* hist = static_cast<int*>(temp);
    int* offs = hist + nh;
    int* scanTemp = offs + nh;
    int* bufK[2];
    int* bufV[2];
    int* pp = scanTemp + scan_temp_bytes(nh) / sizeof(int);
    bufK[0] = pp; bufV[0] = pp + n; bufK[1] = pp + 2 * (int64_t)n; bufV[1] = pp + 3 * (int64_t)n;
    const int passes = (bits + kDigitBits - 1) / kDigitBits;
    const int* sk = keys_in;
    const int* sv = vals_in;
    for (int pass = 0; pass < passes; ++pass) {
        const bool last = pass + 1 == passes;
        int* dk = last ? keys_out : bufK[pass & 1];
        int* dv = last ? vals_out : bufV[pass & 1];
        const int shift = pass * kDigitBits;
        radix_hist_kernel<<<nt, kSortThreads, 0, s>>>(sk, n, shift, nt, hist);
        check(hipGetLastError(), "radix_hist");
        scan_rec(hist, offs, nh, false, scanTemp, s);
        radix_scatter_kernel<<<nt, kSortThreads, 0, s>>>(sk, sv, n, shift, nt, offs, dk, dv);
        check(hipGetLastError(), "radix_scatter");
        sk = dk;
        sv = dv;
    }
}

}  // namespace mflat_amd
