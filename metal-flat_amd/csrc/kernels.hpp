// SPDX-License-Identifier: Apache-2.0
// kernels.hpp -- device kernels of the flat-search hot path and their launchers.
//
// Storage types: the database and the queries of a search are held in one
// element type, fp32 or (reduced-precision variants) fp16 / bf16 rounded to
// nearest-even from the caller's fp32. Dots always accumulate in fp32; norms
// are double sums of the stored values.
//
// Data layout in HBM:
//   database  X, rows_pad = roundup(nb, kBM) rows of dpad = roundup(dim, 32)
//             columns in 32 x 32 chunks ordered the way MFMA lanes consume them:
//             a 32-row block occupies 32*dpad elements like a row-major block
//             would, so row offsets of blocks are unchanged, but inside it each
//             chunk (32 rows x 32 columns: 4 KB fp32, 2 KB fp16/bf16) is laid
//             out so that lane q*16 + r16 of a wave reads a 16-byte operand
//             piece of row (16 hh + r16) with one linear 1 KB load per piece:
//               fp32       [row half hh][float4 e][quarter q][row r16][4]
//                          = element (16 hh + r16, 8 q + 4 e + c)
//               fp16/bf16  [row half hh][quarter q][row r16][8]
//                          = element (16 hh + r16, 8 q + c)
//             (blk_off / blk_off_h below). Pad rows and pad columns are zero.
//   row norms xn[rows_pad]        ||x||^2, double-accumulated (reference
//                                 src/Distance.h:40-47), pad entries zero
//   queries   Q[nqb*kBN][dpad]    row-major in the storage type, zero padded;
//                                 qn[] (fp32) likewise
//   candidates cand[nq][nsplit][cap] of (key bits, id), cnt[nq][nsplit]
//
// Ranking key (smaller = nearer), the value the reference's merge kernel ranks
// on, negated (reference src/FlatIndex.mm:89-93):
//   L2:  key = max(0, (||q||^2 + ||x||^2) - 2 q.x)     reported value = key
//   IP:  key = -(q.x)                                 reported value = -key
// Results are ordered by (key, id) ascending: ties keep the lowest id, exactly
// the order the reference's strict '>' insertion produces
// (src/FlatIndex.mm:272-281).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace mflat_amd {

constexpr int kBM = 128;   // database rows per scan tile
constexpr int kBN = 128;   // queries per scan tile
constexpr int kBK = 32;    // dpad granularity; fp32 columns per LDS-staged chunk
constexpr int kSelLds = 4096;   // candidates a select block holds in LDS
constexpr int kSelLdsSmall = 1024;   // ... in its small-buffer variant (SelectParams::expect)
constexpr int kSelLdsMid = 2560;     // ... in its mid-size variant (SelectParams::expect)
constexpr int kSelLdsLarge = 12288;  // ... in its large-buffer variant (batches of <= 256 queries)
constexpr int kSelLargeMaxSplit = 4096;   // splits the large variant indexes (LDS: 96 + 8 + 16 KB)
constexpr int kTopMax = 1024;   // largest k (== MFLAT_MAX_K)
constexpr int kTopSmall = 256;   // select's winner buffer for k <= kTopSmall
constexpr int kMaxSplit = 16384;  // most database splits one select block indexes
constexpr int kSmallMaxQ = 64;                 // scan_small serves batches up to this size
constexpr size_t kSmallMaxLds = 64 * 1024;     // ... whose query tile fits this much LDS
constexpr size_t kResidentMaxLds = 68 * 1024;  // scan_resident: largest resident query tile
constexpr size_t kResidentMaxLdsNarrow = 144 * 1024;  // ... of a 32-query IVF tile (one workgroup a CU)
constexpr int kRing = 192;                     // scan_resident: staged survivors per wave
constexpr int kPoolCntStride = 32;             // ints between pooled-region counters (128 bytes)
constexpr int kRetryPlanMax = 512;             // largest retry window (the plan's LDS: 2 words a query)
constexpr int kMergeMaxSplit = 1024;   // lists merge_lists takes (one per thread)
constexpr int kStreamTopK = 32;                // streaming top-k scan: k up to this ...
constexpr int kStreamMaxQ = 16;                // ... for batches up to this many queries

// Element type of the stored database and of the queries (the ABI's
// mflat_storage_t values).
enum Storage { kF32 = 0, kF16 = 1, kBF16 = 2 };
inline int elem_bytes(int storage) { return storage == kF32 ? 4 : 2; }

enum KernelFamily {
    kFamScan = 0, kFamScanSample = 1, kFamScanRetry = 2, kFamSelect = 3, kFamArgmin = 4,
    kFamNorms = 5, kFamPrep = 6, kFamIvfScan = 7, kFamIvfBound = 8, kFamCount = 9
};
// kPassArgmin: k = 1; each query's best (key, id) goes to ScanParams::best
// (packed ordered key << 32 | id, combined with 64-bit atomicMin) instead of
// candidate regions, and the bound is each lane's running best.
enum ScanPass { kPassFull = 0, kPassSample = 1, kPassRetry = 2, kPassArgmin = 3 };

// Element offset of (row, col) of an fp32 database in the chunked layout.
__host__ __device__ inline int64_t blk_off(int64_t row, int col, int dpad) {
    const int64_t b = row >> 5;
    const int rr = (int)(row & 31);
    const int t = col >> 5, cc = col & 31;
    return ((b * (dpad >> 5) + t) << 10) +
           ((((rr >> 4) * 2 + ((cc >> 2) & 1)) * 64 + (cc >> 3) * 16 + (rr & 15)) << 2) + (cc & 3);
}
// Element offset of (row, col) of an fp16 / bf16 database in the chunked layout.
__host__ __device__ inline int64_t blk_off_h(int64_t row, int col, int dpad) {
    const int64_t b = row >> 5;
    const int rr = (int)(row & 31);
    const int t = col >> 5, cc = col & 31;
    return ((b * (dpad >> 5) + t) << 10) + ((((rr >> 4) * 4 + (cc >> 3)) * 16 + (rr & 15)) << 3) + (cc & 7);
}

struct ScanParams {
    const void* X;           // database (storage type, chunked layout above)
    const float* xnorm;      // per-row ||x||^2 (L2 only)
    float xnorm_max;         // >= every finite ||x||^2 of the pass (L2 fast-reject margin)
    int64_t nrows;           // valid rows; rows >= nrows are padding
    int64_t rows_per_split;  // largest split's rows, a multiple of kBM (split s starts at tile
                             // s * tiles / nsplit: tile counts differ by at most one)
    int nsplit;              // database splits (grid = nqb * nsplit)
    int id_stride;           // reported id = row * id_stride (sample passes)
    const void* Q;           // queries (storage type, row-major)
    const float* qnorm;      // per-query ||q||^2 (L2 only)
    int nq;                  // valid queries
    int nqb;                 // query blocks of kBN
    int qgroup;              // query blocks co-scheduled per XCD (0: the launcher's choice for the kernel)
    int dpad;                // padded dimension, multiple of kBK
    const float* tau_key;    // per-query threshold key
    const int* tau_id;       // per-query threshold id (lexicographic bound)
    uint2* cand;             // candidate regions
    int* cnt;                // per (query, split) candidate counts (may exceed cap)
    int cap;                 // entries per (query, split) region
    unsigned long long* best;  // kPassArgmin: per-query packed best, pre-filled with all ones
    // IVF fine scan (launch_scan_ivf): one workgroup per work item
    const int4* ivf_work;      // (cell, first entry, entries <= kBN, 0); items >= *ivf_nwork are idle
    const int* ivf_nwork;      // device: valid work items
    const int* ivf_ent;        // entries grouped by cell: e = query * ivf_nprobe + probe rank
    const int* ivf_pos;        // per entry: scan position of its cell's first row for its query
    const int64_t* ivf_cell_pad;   // first database row of each cell (a multiple of kBM)
    const int* ivf_cell_size;  // rows of each cell
    int ivf_nprobe;
    int ivf_nreg;              // candidate regions per query: query * nreg + rank (1, nprobe or nprobe + 1)
    int ivf_spill;             // 1: region nprobe of each query takes what overflows the others (nreg = nprobe + 1)
    int ivf_row_cap;           // > 0: scan only the first ivf_row_cap rows of each cell
    // Retry passes (kPassRetry) whose work list the device built:
    const int* nq_dev;         // nullable: valid queries = *nq_dev (<= nq); query blocks beyond exit
    // Pooled regions (kPassRetry): one region per query, cand[qoff[q] ..
    // qoff[q] + qcap[q]), slots taken with global atomics on the query's
    // counter qcnt[q * kPoolCntStride] (one per 128-byte line: counters of
    // different queries never share a line), which then holds the unclamped
    // count; cnt is not written.
    int* qcnt;
    const int64_t* qoff;
    const int* qcap;
    // Streaming top-k scan only: the caller's fp32 queries (qdim values a
    // row, nq rows), prepared by every workgroup in LDS as prep_queries would
    // (qcos: Cosine scaling first); Q and qnorm are then unused.
    const float* qraw;
    int qdim;
    int qcos;
    // fp16/bf16 at a d beyond scan_resident, batches of more than 128
    // queries: 1 runs the wide-tile kernel (256 queries a block; grid
    // ceil(nq / 256) x nsplit). The caller sets it for every pass of a batch.
    int wide;
};

// Device-built retry work lists (flat search). After a full pass's select, a
// query whose status is nonzero is retried; retry_plan decides each one's
// bound and pooled region (one per query, cand[qoff .. qoff + qcap)):
//   overflow (bit 0): the k-th best it stored, capacity = the unclamped count
//       it saw under the looser bound (total): the rerun cannot overflow, so
//       it is final;
//   too few (bit 1): the next looser bound of its ladder (the sample's j2-th,
//       then its guaranteed k-th, then none), capacity estimated for it.
// Queries are taken in ascending order while they fit rmax and the pool; the
// rest wait for the next round. All counts stay on the device.
struct RetryLists {
    int* fail;         // [mb] scratch: failing queries in ascending order
    unsigned char* lvl;   // [mb] ladder step each query has taken
    int* idx;          // [rmax] queries scheduled this round (original row)
    float* tk;         // [rmax] their bounds
    int* ti;
    int64_t* qoff;     // [rmax] pooled regions
    int* qcap;
    int* qcnt;         // [rmax * kPoolCntStride] slot counters, 128 bytes apart (cleared by the plan)
    int* counters;     // [4]: failing queries, scheduled, failed again (the select adds), spare
};
struct RetryLadder {   // per-query bounds of the "too few" ladder (nullable entries are skipped)
    const float* j2_key;
    const int* j2_id;
    const float* g_key;
    const int* g_id;
    int cap_j2, cap_g;   // pooled capacities estimated for those bounds
};

// One retry round's plan and gather (see RetryLists), run by one block
// (launch_retry_plan). Scheduled queries' rows of Q (row_bytes each) and norms
// go to dst_q / dst_qn, rows past them up to the end of their query block
// zeroed.
struct RetryPlanArgs {
    const int* status;
    int mb;
    int first;                 // 1: every query's ladder step starts at 0
    const float* tau_k_key;
    const int* tau_k_id;
    const int* total;
    RetryLadder ladder;
    int64_t pool_entries;
    int rmax;
    int all_rows;
    RetryLists lists;
    const void* Q;
    const float* qn;
    int row_bytes;
    void* dst_q;
    float* dst_qn;
    int rows_pad;
};

struct SelectParams {
    const uint2* cand;
    const int* cnt;
    int nsplit;
    int cap;
    int nq;
    int k;                   // rank to select (1..kTopMax)
    int j;                   // secondary rank for tau_j (1..k)
    int j2;                  // secondary rank for tau_j2 (1..k)
    int metric;              // 0: value = key, otherwise value = -key
    const int* qmap;         // nullable: output row of query i
    int32_t* out_ids;        // nullable
    float* out_vals;         // nullable
    int out_stride;
    float* tau_j_key;        // nullable: j-th smallest (key, id), or "no bound"
    int* tau_j_id;
    float* tau_j2_key;       // nullable: j2-th smallest (key, id), or "no bound"
    int* tau_j2_id;
    float* tau_k_key;        // nullable: k-th smallest (key, id), or "no bound"
    int* tau_k_id;
    int* status;             // nullable: bit0 = a region overflowed, bit1 = fewer than k stored
    int expect;              // stored candidates per query that (nearly) every query stays under (0:
                             // unknown): picks the smallest LDS buffer variant that holds it (more
                             // blocks per CU); a query above its buffer reads from global memory
    const int* nq_dev;       // nullable: blocks at or beyond *nq_dev exit (device-built work lists)
    const int64_t* qoff;     // nullable (nsplit == 1): pooled regions, query i at cand[qoff[i]],
    const int* qcap;         //   capacity qcap[i], count cnt[i * kPoolCntStride]
    int* total;              // nullable: unclamped candidates seen by each query (sum of its counts)
    int* fail_count;         // nullable: incremented once per query whose status is nonzero
};

// Launchers (kernels.hip). All are asynchronous on `s` and bracket the launch
// with the process-wide kernel timer when it is enabled.
// A search batch's queries in one launch: fp32 rows (dim values, n of them)
// -> out, n_pad rows of dpad elements of the storage type (zero padded;
// Cosine rows L2-normalised first, the reference's rule), qn[n_pad] = ||row||^2
// of the stored values (double sum), and, when tau_key is given, "no bound"
// (+inf, -1) for the n live rows.
void launch_prep_queries(const float* src, int64_t n, int dim, int64_t n_pad, int dpad, int storage, bool cosine,
                         void* out, float* qn, float* tau_key, int* tau_id, hipStream_t s);
// row-major fp32 (queries)
void launch_pack_rows(const float* src, int64_t n, int dim, float* dst, int64_t n_pad, int dpad,
                      hipStream_t s);
void launch_normalize_rows(float* v, int64_t n, int dpad, hipStream_t s);
// row-major storage-type rows: fp32 -> storage rounding, ||row||^2 of stored values
void launch_round_rows(const float* src, int64_t count, int storage, void* dst, hipStream_t s);
void launch_row_norms(const void* v, int64_t n, int dpad, int storage, float* out, hipStream_t s);
// inv[r] = float(1 / sqrt(sum_c src[r][c]^2)) (double sum), 1 for zero rows
void launch_row_inv_norms(const float* src, int64_t n, int dim, float* inv, hipStream_t s);
// chunked database layout: rows [row0, row0 + n) of X; inv (nullable) scales row r first
void launch_store_rows_blk(const float* src, int64_t n, int dim, const float* inv, void* X, int64_t row0,
                           int dpad, int storage, hipStream_t s);
void launch_row_norms_blk(const void* X, int64_t row0, int64_t n, int dpad, int storage, float* out,
                          hipStream_t s);
void launch_gather_rows_blk(const void* X, const int* idx, int n, int dpad, int storage, void* dst,
                            hipStream_t s);
// row-major rows of row_bytes (a multiple of 16): dst row r = src row idx[r], zero for n <= r < n_pad
void launch_gather_rows(const void* src, const int* idx, int n, int row_bytes, void* dst,
                        int64_t n_pad, hipStream_t s);
void launch_gather_f32(const float* src, const int* idx, int n, float* dst, hipStream_t s);
struct TauSources {   // three per-query bound arrays a retry can draw from
    const float* key[3];
    const int* id[3];
};
void launch_gather_tau(const TauSources& src, const int* idx, const int* sel, int n, float* ko,
                       int* io, hipStream_t s);
void launch_fill_tau_none(float* key, int* id, int n, hipStream_t s);
// (key_a, id_a)[i] = lexicographic min of itself and (key_b, id_b)[i]
void launch_tau_min(float* key_a, int* id_a, const float* key_b, const int* id_b, int n, hipStream_t s);
void launch_fill_empty(int32_t* ids, float* vals, int64_t count, float empty, hipStream_t s);
void launch_max_norm(const float* xn, int64_t n, unsigned* out, hipStream_t s);
// Dispatches to scan_small (small batches, HBM-streaming) when allowSmall and
// small_scan_fits, else to scan_resident when the 128-query tile fits in LDS
// (resident_scan_fits), else to the LDS-tiled scan_filter. scan_resident and
// scan_filter compute bit-identical keys (same MFMA shape and column order);
// scan_small's accumulation order differs, so passes whose bounds feed each
// other must not mix it with the other two (allowSmall = false).
bool small_scan_fits(int nq, int dpad, int storage);
bool resident_scan_fits(int dpad, int storage);
// The IVF fine scan's 32-query scan_resident tile fits LDS (fp32 dim <= 1120,
// fp16/bf16 dim <= 2272).
bool ivf_narrow_fits(int dpad, int storage);
// Workgroups of the scan that launch_scan_filter runs (outside scan_small's
// range) that fit the current device at once (occupancy x CUs); 0 if unknown.
int scan_concurrency(int dpad, int storage, int metric, int pass, bool wide = false);
// Whether a batch of nq queries takes the wide-tile kernel (fp16/bf16, a d
// beyond scan_resident's LDS, more than 128 queries).
bool wide_scan_applies(int nq, int dpad, int storage);
void launch_scan_filter(const ScanParams& p, int metric, int pass, int storage, hipStream_t s,
                        bool allowSmall = true);
// IVF fine scan (scan_resident over the work items of ScanParams::ivf_*; the
// 128-query tile must fit, resident_scan_fits): pass kPassSample or kPassFull,
// work items of up to tileQueries (128 or 32) entries, grid = an upper bound of
// the work items. Both tile widths compute bit-identical keys.
void launch_scan_ivf(const ScanParams& p, int metric, int pass, int storage, int tileQueries, int grid,
                     hipStream_t s);
void launch_select(const SelectParams& p, hipStream_t s);
// Streaming top-k scan (batches of <= kStreamMaxQ queries, k = p.cap <=
// kStreamTopK): one workgroup per split keeps each wave's exact top-k of the
// rows it reads and writes the split's top-k of every query (cand regions of
// p.cap entries, cnt = entries written); launch_merge_lists finishes the
// search. No bound, sample or retry: exact by construction. The split count
// wants to be the number of workgroups resident at once (topk_concurrency).
// Queries: prepared rows (Q, qnorm) or the caller's fp32 rows (qraw), which
// every workgroup prepares itself (no separate preparation launch).
void launch_scan_topk(const ScanParams& p, int metric, int storage, hipStream_t s);
int topk_concurrency(int dpad, int storage, int metric);
// The streaming scan's exact top-k per query from its ascending per-split
// lists (cand / cnt / nsplit <= kMergeMaxSplit / cap of launch_scan_topk;
// k <= cap; out_ids / out_vals / out_stride / metric / qmap as for
// launch_select). Rows missing when the database holds fewer than k: id -1
// and the empty value.
void launch_merge_lists(const SelectParams& p, hipStream_t s);
// One retry round's plan and gather in one block (RetryPlanArgs).
void launch_retry_plan(const RetryPlanArgs& a, hipStream_t s);
void launch_argmin_finalize(const unsigned long long* best, int nq, int metric, int32_t* ids, float* vals,
                            hipStream_t s);
void launch_fill_u64(unsigned long long* p, int64_t n, unsigned long long v, hipStream_t s);

// Kernel timer (profile.cpp).
void prof_begin(int fam, hipStream_t s, void** token);
void prof_end(void* token, hipStream_t s);
void prof_suppress(bool on);   // on: this thread's launches create no timer events (nests)

}  // namespace mflat_amd
