// SPDX-License-Identifier: Apache-2.0
// flat_index.cpp -- host side of the flat-search hot path on one MI355X.
//
// Search = threshold filtering on the GPU, in levels (reference loop it
// replaces: src/FlatIndex.mm:294-421):
//
//   L0  sample:  exact top-k of every query over a strided sample of R0
//                database rows (scan_filter with no bound, then select). Its
//                k-th (key, id) is a GUARANTEED bound: the k-th best over any
//                subset is never better than the k-th best over the whole
//                database. Its j-th (j <= k, from a Poisson tail estimate) is a
//                SPECULATIVE bound expected to admit ~j*nb/R0 rows.
//   L1  full:    scan_filter over all rows with the speculative bound, then
//                select. The result is exact iff no candidate region overflowed
//                and at least k rows passed (every row that did not pass ranks
//                after all k that did).
//   retry:       queries failing that test rerun L1 alone, with the guaranteed
//                bound (too few passed) or with the k-th best of what was stored
//                (a region overflowed); a query overflowing again reruns once
//                more under its new k-th with one region sized by its count,
//                which cannot overflow. The device builds these work lists, so
//                a search is a fixed launch sequence (retries()). Exactness
//                never depends on the estimate, only the amount of work does.
//
// Small databases (nb <= max(2*R0, kSelLds)) skip the levels: one unbounded pass.
#include "flat_index.hpp"

#include <algorithm>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "log.hpp"
#include "noalloc.hpp"

namespace mflat_amd {
namespace {

// MFLAT_TRACE=1 in the environment prints per-search plans and bound
// refinements to stderr (diagnostics only; results are unaffected).
bool traceOn() {
    static const bool on = [] {
        const char* v = std::getenv("MFLAT_TRACE");
        return v && *v && *v != '0';
    }();
    return on;
}

void hipCheck(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) throw std::bad_alloc();
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
#define HIPC(x) hipCheck((x), #x)

constexpr int64_t kTargetWG = 2048;             // scan_filter workgroups wanted per launch
constexpr int64_t kTargetWGSmall = 4096;        // scan_small workgroups (HBM streaming)
constexpr size_t kCandBudget = size_t(1536) << 20;  // candidate workspace per batch
constexpr size_t kStageBytes = size_t(256) << 20;   // host->device staging chunk
constexpr int64_t kRetryMinTiles = 2;   // tiles per split in the retries of a large batch
constexpr int kRetryMax = 256;          // queries one device-built retry window takes (large batches)

int64_t roundUp(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    void ensure(size_t b) {
        if (b <= bytes) return;
        release();
        const size_t want = std::max(b, bytes + bytes / 2);
        HIPC(hipMalloc(&p, want));
        bytes = want;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
    template <class T> T* as() const { return static_cast<T*>(p); }
};

// Two ints of pinned host memory: the counters a batch reads back at its end.
struct PinnedInts {
    int* p = nullptr;
    void ensure() {
        if (!p) HIPC(hipHostMalloc((void**)&p, 4 * sizeof(int), hipHostMallocDefault));
    }
    void release() {
        if (p) (void)hipHostFree(p);
        p = nullptr;
    }
};

// Device storage of the retry work lists (kernels.hpp RetryLists).
struct RetryStore {
    DevBuf fail, lvl, idx, tk, ti, qoff, qcap, qcnt, counters;
    void ensure(int mb, int rmax, hipStream_t s) {
        fail.ensure((size_t)mb * 4);
        lvl.ensure((size_t)mb);
        for (DevBuf* b : {&idx, &tk, &ti, &qcap}) b->ensure((size_t)rmax * 4);
        qcnt.ensure((size_t)rmax * kPoolCntStride * 4);
        qoff.ensure((size_t)rmax * sizeof(int64_t));
        (void)s;
        counters.ensure(4 * sizeof(int));
    }
    RetryLists lists() const {
        RetryLists l;
        l.fail = fail.as<int>(); l.lvl = lvl.as<unsigned char>();
        l.idx = idx.as<int>(); l.tk = tk.as<float>(); l.ti = ti.as<int>();
        l.qoff = qoff.as<int64_t>(); l.qcap = qcap.as<int>(); l.qcnt = qcnt.as<int>();
        l.counters = counters.as<int>();
        return l;
    }
    void release() {
        for (DevBuf* b : {&fail, &lvl, &idx, &tk, &ti, &qoff, &qcap, &qcnt, &counters}) b->release();
    }
};

// Smallest j in [1, k] with P(Poisson(lambda) >= j) <= tail: the chance that a
// speculative bound taken at the sample's j-th best admits fewer than k rows.
int chooseJ(int k, double lambda, double tail) {
    double term = std::exp(-lambda), cdf = term;
    for (int j = 1; j <= k; ++j) {
        if (1.0 - cdf <= tail) return j;
        term *= lambda / j;
        cdf += term;
    }
    return k;
}

// nq: queries of the launch (small batches go to scan_small, which streams the
// database and wants many more, smaller workgroups).
// minTiles: fewest kBM-row tiles per split (a scan_resident workgroup needs
// two tiles to give each of its four waves a 64-row slice).
// concurrent (> 0): workgroups of the MFMA scan that run at once
// (scan_concurrency). The launch's nqb x nsplit workgroups run in rounds of
// that many; a last round of a few leaves the chip idle for most of a round
// (C1: 8 x 196 = 1,568 workgroups in rounds of 512, a fourth round of 32).
// Splits share the tiles as evenly as possible (split s starts at tile
// s * ntiles / nsplit), so any split count is possible: it is chosen in
// [want / 4, 3 want] to minimise rounds x (tiles of the largest split + 1),
// a partial round of fraction f costing 0.5 + 0.5 f of a full one (its
// workgroups run alone, faster). rowsPerSplit is the largest split's rows.
void splitPlan(int64_t nrows, int nq, int dpad, int storage, int64_t& rowsPerSplit, int& nsplit,
               bool allowSmall = true, int64_t minTiles = 1, int concurrent = 0) {
    const int nqb = (nq + kBN - 1) / kBN;
    const int64_t ntiles = std::max<int64_t>(1, (nrows + kBM - 1) / kBM);
    const int64_t target = allowSmall && small_scan_fits(nq, dpad, storage) ? kTargetWGSmall : kTargetWG;
    int64_t want = std::max<int64_t>(1, (target + nqb - 1) / nqb);
    // keep a split's bytes addressable with 32-bit offsets
    const int64_t maxTiles =
        std::max<int64_t>(1, ((int64_t)1 << 31) / ((int64_t)kBM * dpad * elem_bytes(storage)) - 1);
    const int64_t fewest = std::min<int64_t>(kMaxSplit, (ntiles + maxTiles - 1) / maxTiles);
    want = std::max(want, fewest);
    want = std::min<int64_t>(want, kMaxSplit);
    want = std::min(want, std::max<int64_t>(1, ntiles / minTiles));
    want = std::min(want, ntiles);
    if (concurrent > 0 && !(allowSmall && small_scan_fits(nq, dpad, storage))) {
        const int64_t lo = std::max<int64_t>({1, fewest, want / 4});
        const int64_t hi = std::min<int64_t>({3 * want, kMaxSplit, std::max<int64_t>(1, ntiles / minTiles), ntiles});
        auto cost = [&](int64_t ns) {
            const int64_t tps = (ntiles + ns - 1) / ns;
            const int64_t w = (int64_t)nqb * ns;
            const int64_t full = w / concurrent, rem = w % concurrent;
            const double rounds = (double)full + (rem ? 0.5 + 0.5 * (double)rem / concurrent : 0.0);
            return rounds * ((double)tps + 1.0);
        };
        int64_t best = want;
        double bestCost = cost(want);
        for (int64_t ns = lo; ns <= hi; ++ns) {
            const double c = cost(ns);
            if (c < bestCost - 1e-9) {
                bestCost = c;
                best = ns;
            }
        }
        want = best;
    }
    nsplit = (int)want;
    rowsPerSplit = (ntiles + want - 1) / want * kBM;
}

int pow2ceil(int64_t x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

struct Plan {
    bool stream = false;  // streaming top-k scan (small batch, small k): no sample, no retries
    bool wide = false;    // every pass on the wide-tile kernel (wideBatch)
    bool direct = true;
    int64_t R0 = 0;       // sample rows
    int stride = 1;       // sample row r is database row r*stride
    int j = 1;            // speculative rank
    int j2 = 1;           // looser speculative rank (first retry of a query with too few rows)
    int64_t rps0 = 0;
    int nsplit0 = 1, cap0 = 1;
    // optional second sample (0 rows: none), scanned with the first one's
    // speculative bound; its jb-th best is the full pass's speculative bound
    int64_t Rb = 0;
    int strideb = 1;
    int jb = 1;
    int jb2 = 0;          // its looser rank (0: none): the retries' first bound, with j2's

    int64_t rpsb = 0;
    int nsplitb = 1, capb = 1;
    int64_t rps1 = 0;
    int nsplit1 = 1, cap1 = 1;
    double e1 = 0.0;      // expected full-pass survivors per query
    size_t perQuery = 0;  // candidate entries per query (max over levels)
};

}  // namespace

struct FlatIndex::Impl {
    int dim = 0, dpad = 0;
    Metric metric = Metric::L2;
    int storage = kF32;   // element type of the database and of the queries
    int esize = 4;
    int device = -1;
    bool ready = false;
    bool warnedK = false;
    hipStream_t stream = nullptr;

    int64_t nb = 0;
    int64_t capRows = 0;
    DevBuf X, xn;
    float xnMax = 0.0f;   // max finite-or-inf ||x||^2 over the database
    DevBuf maxBits;

    // strided sample of the database (L0)
    // strided samples of the database (L0, and the optional second level)
    struct RowSample {
        DevBuf X, xn, idx;
        int64_t R = 0;
        int stride = 0;
        int64_t nb = -1;   // database size it was gathered at
        void release() { X.release(); xn.release(); idx.release(); nb = -1; }
    };
    RowSample smp[2];

    // per-search workspace
    DevBuf stage, inv, qin, outIds, outVals;
    DevBuf qbuf, qh, qnorm, cand, cnt;
    DevBuf tauSk, tauSi, tauS2k, tauS2i, tauGk, tauGi, tauKk, tauKi, tauBk, tauBi, tauB2k, tauB2i, status;
    DevBuf cQ, cQn;
    DevBuf best, total;
    RetryStore rl;
    PinnedInts hostCounters;
    // Diagnostics knobs, read once when the index is created: MFLAT_RETRY_WINDOW
    // = n limits a device-built retry window to n queries, MFLAT_RETRY_POOL = n
    // the retry pool to n entries (0 = not set). They exercise the host's
    // fallback windows; results never depend on them, only the work done.
    int retryWindow = 0;
    int64_t retryPool = 0;
    // MFLAT_STREAM_MAXQ = n: batches of up to n queries (0: none) take the
    // streaming top-k scan; MFLAT_STREAM_SPLITS = n: its split count.
    // Default: up to 2 queries with fp32 storage, 1 with fp16 / bf16. The
    // streaming scan loses to the bound filter's as queries are added (each
    // wave's bound starts unbounded, so its lists take ~k (1 + ln(rows / k))
    // insertions a query) but saves the sample path's launches and selects.
    // Whole search at C4 (10M x 96, k 10), streaming / sample path, ms: fp32
    // nq 1 0.601 / 0.640, nq 2 0.623 / 0.643, nq 4 0.652 / 0.653, nq 8 0.703 /
    // 0.656, nq 16 0.790 / 0.665; fp16 nq 1 0.329 / 0.372, nq 4 0.381 / 0.367.
    int streamMaxQ = -1;   // -1: the storage type's default
    int streamSplits = 0;
    // MFLAT_QGROUP = n: query blocks co-scheduled per XCD by the MFMA scans
    // (0: each kernel's default).
    int qgroupKnob = 0;

    int kernMetric() const { return metric == Metric::L2 ? 0 : 1; }
    float emptyValue() const { return metric == Metric::L2 ? INFINITY : -INFINITY; }

    // Workgroups of each pass's MFMA scan that fit the device at once (the
    // split plan's tail rule), queried once per pass.
    mutable int conc[2][4] = {{-1, -1, -1, -1}, {-1, -1, -1, -1}};
    int concurrency(int pass, bool wide = false) const {
        int& c = conc[wide ? 1 : 0][pass];
        if (c < 0) c = scan_concurrency(dpad, storage, kernMetric(), pass, wide);
        return c;
    }
    // fp16/bf16 batches of more than 128 queries at a d beyond scan_resident
    // run their sample and full passes on the wide-tile kernel, their retry
    // window on the 128-query tiled kernel (same keys); MFLAT_WIDE=0 (read
    // when the index is created) keeps every pass on the tiled kernel. Split
    // plans of wide passes count 256-query blocks: they get half the query count.
    int wideKnob = 1;
    bool wideBatch(int64_t mb) const {
        return wideKnob && wide_scan_applies((int)std::min<int64_t>(mb, 1 << 30), dpad, storage);
    }
    int planQ(int64_t mb) const { return (int)(wideBatch(mb) ? (mb + 1) / 2 : mb); }
    int planConc(int pass, int64_t mb) const { return concurrency(pass, wideBatch(mb)); }
    bool curWide = false;   // the batch being searched runs the wide-tile kernel

    void setDevice() const {
        if (device >= 0) HIPC(hipSetDevice(device));
    }

    // The streaming top-k scan's plan: one workgroup per split, as many
    // splits as run at once; each streams its rows once and hands k candidates
    // per query to the select, whose LDS buffer holds them all.
    // maxSplits: a workspace bound (the allocation-free path's scratch).
    void setStreamPlan(Plan& pl, int k, int64_t maxSplits = kMergeMaxSplit) const {
        pl.stream = true;
        const int64_t ntiles = std::max<int64_t>(1, (nb + kBM - 1) / kBM);
        int64_t want = streamSplits > 0 ? streamSplits : topkConcurrency();
        if (want <= 0) want = 1024;
        want = std::max<int64_t>(1, std::min<int64_t>({want, ntiles, kMergeMaxSplit, maxSplits}));
        const int64_t tps = (ntiles + want - 1) / want;
        pl.nsplit1 = (int)((ntiles + tps - 1) / tps);
        pl.rps1 = tps * kBM;
        pl.cap1 = k;
        pl.perQuery = (size_t)pl.nsplit1 * k;
    }

    // Small batches with a small k: the streaming top-k scan.
    bool streamPath(int64_t mb, int k) const {
        const int maxq = streamMaxQ >= 0 ? streamMaxQ : storage == kF32 ? 2 : 1;
        return mb <= std::min(maxq, kStreamMaxQ) && k <= kStreamTopK && small_scan_fits((int)mb, dpad, storage);
    }
    mutable int topkConc = -1;
    int topkConcurrency() const {
        if (topkConc < 0) topkConc = topk_concurrency(dpad, storage, kernMetric());
        return topkConc;
    }

    // k = 1 on a batch too large for scan_small: one fused argmin pass.
    bool argminPath(int64_t mb, int k) const {
        return k == 1 && !small_scan_fits((int)std::min<int64_t>(mb, 1 << 30), dpad, storage);
    }

    Plan plan(int64_t mb, int k) const {
        Plan pl;
        if (argminPath(mb, k)) {
            pl.perQuery = 1;
            return pl;
        }
        if (streamPath(mb, k)) {
            setStreamPlan(pl, k);
            return pl;
        }
        int64_t r = (int64_t)std::ceil(std::sqrt(16.0 * (double)nb));
        // Small batches stream the database once whatever the bound; a sample of
        // at most kSelLds rows keeps its per-query select inside LDS.
        if (mb <= kSmallMaxQ) r = std::min<int64_t>(r, kSelLds);
        r = std::max<int64_t>(r, std::max<int64_t>(4LL * k, 256));
        r = roundUp(r, kBM);
        // A database whose every row fits one select block's LDS (e.g. an IVF
        // coarse quantizer's centroids) takes one unbounded pass: cheaper than
        // a sample level and its select.
        if (nb <= std::max<int64_t>(2 * r, kSelLds)) {
            pl.direct = true;
            pl.wide = wideBatch(mb);
            splitPlan(nb, planQ(mb), dpad, storage, pl.rps1, pl.nsplit1, true, 1, planConc(kPassFull, mb));
            pl.cap1 = (int)pl.rps1;
            pl.perQuery = (size_t)pl.nsplit1 * pl.cap1;
            return pl;
        }
        pl.direct = false;
        pl.wide = wideBatch(mb);
        setFirstSample(pl, mb, k, r);
        splitPlan(nb, planQ(mb), dpad, storage, pl.rps1, pl.nsplit1, true, 1, planConc(kPassFull, mb));
        const double e1 = (double)pl.j * (double)nb / (double)r;   // expected survivors
        pl.e1 = e1;
        const int64_t perSplit = (int64_t)(2.0 * e1 / pl.nsplit1) + 64;
        pl.cap1 = std::max<int>({2 * k, 64, pow2ceil(perSplit)});
        planSecondSample(pl, mb, k, r);
        pl.perQuery = std::max({(size_t)pl.nsplit0 * pl.cap0, (size_t)pl.nsplit1 * pl.cap1,
                                pl.Rb ? (size_t)pl.nsplitb * pl.capb : (size_t)0});
        return pl;
    }

    // First sample level of r rows: every row is stored (the select takes the
    // j-th, j2-th and k-th best of each query).
    void setFirstSample(Plan& pl, int64_t mb, int k, int64_t r) const {
        pl.R0 = r;
        pl.stride = (int)(nb / r);
        const double lambda = (double)k * (double)r / (double)nb;
        pl.j = chooseSpeculativeRank(k, lambda, mb, nb, r);
        pl.j2 = chooseJ(k, lambda, 1e-9);
        splitPlan(r, planQ(mb), dpad, storage, pl.rps0, pl.nsplit0, true, 1, planConc(kPassSample, mb));
        pl.cap0 = (int)pl.rps0;
    }

    // Speculative rank j. A tighter rank means fewer survivors in the full
    // pass (~j nb / R0 a query, each an exact test and a store in the scan
    // epilogue); a query whose j-th sample bound admits fewer than k rows
    // (probability P(Poisson(lambda) >= j), floored at 3e-4: the sample is a
    // fixed stride, so a few queries miss at every j) is retried, and retries
    // cost per batch, not per query: a host round trip (~130 us of idle
    // device) plus a pass over the database per retried block of kBN queries.
    // j minimises the expected sum, with the measured rates of this part
    // (C1-C3 shapes): ~0.12 ns a survivor fp32 (0.16 fp16/bf16), ~120 (700)
    // TFLOP/s a pass; never below the rank of a 1% miss rate (the second
    // sample level's plan assumes it). Measured sweeps: C1 j = 2 / 3 / 4 / 5
    // -> 1.61 / 2.13 / 2.11 / 1.51 M QPS (6 / 0 / 0 / 1 queries retried), the
    // rule picks 3; C3 j = 3 / 4 / 5 -> 122.3 / 122.6 / 123.0 ms, it picks 3.
    int chooseSpeculativeRank(int k, double lambda, int64_t mb, int64_t nbRows, int64_t r) const {
        const bool f32 = storage == kF32;
        const double tSurv = f32 ? 0.12e-9 : 0.16e-9;
        const double tBlock = (double)nbRows * kBN * dpad * 2.0 / (f32 ? 120e12 : 700e12);
        const double tTrip = 130e-6;
        const double perJ = (double)mb * ((double)nbRows / (double)r) * tSurv;
        int best = k;
        double bestCost = 1e300;
        double term = std::exp(-lambda), cdf = term;   // P(X = j - 1), P(X <= j - 1)
        for (int j = 1; j <= k; ++j) {
            const double pj = std::min(std::max(3e-4, 1.0 - cdf), 1.0 - 1e-16);   // P(X >= j), floored
            const double pAny = -std::expm1((double)mb * std::log1p(-pj));
            const double blocks = std::max(1.0, std::ceil((double)mb * pj / kBN));
            const double cost = perJ * j + pAny * (tTrip + blocks * tBlock);
            if (cost < bestCost) {
                bestCost = cost;
                best = j;
            }
            if (perJ * j > bestCost) break;   // survivors alone exceed the best
            term *= lambda / j;
            cdf += term;
        }
        return std::max(best, chooseJ(k, lambda, 0.01));
    }

    // Second sample level. The full pass's survivors scale with the speculative
    // bound's rank over its sample size (j nb / R0 per query); a larger sample
    // Rb, scanned with the first sample's bound (few candidates), gives the
    // rank jb for Rb and ~jb nb / Rb survivors. It pays where a survivor's exact
    // test and store cost more than the extra MFMA work: fp16/bf16 storage at
    // small d. The cost model uses measured rates of this part (C2 shape):
    // fp32 ~60 TMAC/s, fp16/bf16 ~420 TMAC/s resident (~330 tiled), ~0.15 ns
    // per survivor, ~15 ns per query for the extra select.
    void planSecondSample(Plan& pl, int64_t mb, int k, int64_t r) const {
        if (small_scan_fits((int)std::min<int64_t>(mb, 1 << 30), dpad, storage)) {
            planSecondSampleSmall(pl, mb, k, r);
            return;
        }
        const double tMac = storage == kF32 ? 1.0 / 60e12
                            : resident_scan_fits(dpad, storage) ? 1.0 / 420e12 : 1.0 / 330e12;
        const double tSurv = 0.15e-9, tSelQ = 15e-9;
        double best = 0.0;
        for (int f = 2; f <= 16; f *= 2) {
            const int64_t Rb = roundUp(f * r, kBM);
            if (2 * Rb > nb) break;
            const int jb = chooseJ(k, (double)k * (double)Rb / (double)nb, 0.01);
            const double saved = (double)mb * ((double)pl.j * nb / r - (double)jb * nb / Rb) * tSurv;
            const double cost = (double)mb * (double)Rb * dpad * tMac + (double)mb * tSelQ;
            if (saved > 1.5 * cost && saved - cost > best) {   // clear wins only: the rates are estimates
                best = saved - cost;
                pl.Rb = Rb;
                pl.jb = jb;
            }
        }
        if (!pl.Rb) return;
        // With a second level, the first one only seeds that level's bound
        // (~j Rb / R0 candidates a query) and the retries' fallback bounds: a
        // first sample of max(4 k, 1,024) rows keeps its select, over every
        // sample row, in the 1,024-entry buffer (~8 blocks per CU, not 3).
        const int64_t r1 = roundUp(std::max<int64_t>(4LL * k, kSelLdsSmall), kBM);
        if (r1 < r) {
            r = r1;
            setFirstSample(pl, mb, k, r);
        }
        finishSecondSample(pl, mb, k, r);
    }

    // Second sample level of a small batch. Small batches stream the database
    // once whatever the bound, so the bound only sets how many survivors the
    // full pass stores for the per-query select: ~j nb / R0 (R0 is capped at
    // the select's LDS buffer), spread as the j-th order statistic of the
    // sample, P(count > C) ~ P(Gamma(j, 1) > C R0 / nb). A query above the
    // select's LDS buffer reads its candidates from global memory on every
    // select pass (measured ~230 us at 10M x 96, against ~25 us in LDS); a
    // second sample of Rb = f R0 rows under the first bound (one more small
    // scan and select, ~30 us) gives ~jb nb / Rb survivors, jb at a 1e-5 miss
    // rate (a miss costs another pass over the database).
    void planSecondSampleSmall(Plan& pl, int64_t mb, int k, int64_t r) const {
        const int buf = pl.nsplit1 <= kSelLargeMaxSplit ? kSelLdsLarge : kSelLds;
        const double x = (double)buf * (double)r / (double)nb;
        double term = std::exp(-x), tail = term;
        for (int i = 1; i < pl.j; ++i) {
            term *= x / i;
            tail += term;
        }
        const double pAny = -std::expm1((double)mb * std::log1p(-std::min(tail, 1.0 - 1e-16)));
        if (pAny * 230e-6 <= 30e-6) return;
        for (int f = 4; f <= 64; f *= 2) {
            const int64_t Rb = roundUp(f * r, kBM);
            if (2 * Rb > nb) break;
            pl.Rb = Rb;
            pl.jb = chooseJ(k, (double)k * (double)Rb / (double)nb, 1e-5);
            if ((double)pl.jb * (double)nb / (double)Rb <= kSelLds / 4) break;
        }
        if (!pl.Rb) return;
        finishSecondSample(pl, mb, k, r);
    }

    void finishSecondSample(Plan& pl, int64_t mb, int k, int64_t r) const {
        pl.strideb = (int)(nb / pl.Rb);
        splitPlan(pl.Rb, planQ(mb), dpad, storage, pl.rpsb, pl.nsplitb, true, 1, planConc(kPassSample, mb));
        const double eb = (double)pl.j * (double)pl.Rb / (double)r;   // expected stored per query
        pl.capb = std::max<int>(32, pow2ceil((int64_t)(4.0 * eb / pl.nsplitb) + 16));
        // the full pass now expects jb nb / Rb survivors
        const double e1 = (double)pl.jb * (double)nb / (double)pl.Rb;
        pl.e1 = e1;
        pl.cap1 = std::max<int>({2 * k, 64, pow2ceil((int64_t)(2.0 * e1 / pl.nsplit1) + 64)});
        // A query with too few rows under the jb-th best reruns first under
        // the tighter of the first sample's j2-th best (~j2 nb / R0 rows) and
        // this sample's jb2-th best (~jb2 nb / Rb rows, where it stored that
        // many), both at a 1e-9 miss rate.
        const int jb2 = chooseJ(k, (double)k * (double)pl.Rb / (double)nb, 1e-9);
        pl.jb2 = jb2 > pl.jb && pl.j2 > pl.j ? jb2 : 0;
    }

    void growRows(int64_t need, hipStream_t s) {
        if (need <= capRows) return;
        const int64_t newCap = std::max(need, roundUp(capRows + capRows / 2, kBM));
        void* nx = nullptr;
        void* nn = nullptr;
        HIPC(hipMalloc(&nx, (size_t)newCap * dpad * esize));
        hipError_t e = hipMalloc(&nn, (size_t)newCap * sizeof(float));
        if (e != hipSuccess) { (void)hipFree(nx); hipCheck(e, "hipMalloc(norms)"); }
        HIPC(hipMemsetAsync(nx, 0, (size_t)newCap * dpad * esize, s));
        HIPC(hipMemsetAsync(nn, 0, (size_t)newCap * sizeof(float), s));
        if (nb > 0) {
            // whole 32-row blocks: the chunked layout interleaves a block's rows
            HIPC(hipMemcpyAsync(nx, X.p, (size_t)roundUp(nb, 32) * dpad * esize,
                                hipMemcpyDeviceToDevice, s));
            HIPC(hipMemcpyAsync(nn, xn.p, (size_t)nb * sizeof(float), hipMemcpyDeviceToDevice, s));
        }
        HIPC(hipStreamSynchronize(s));
        X.release();
        xn.release();
        X.p = nx; X.bytes = (size_t)newCap * dpad * esize;
        xn.p = nn; xn.bytes = (size_t)newCap * sizeof(float);
        capRows = newCap;
    }

    void append(const float* src, int n, hipMemcpyKind kind, hipStream_t s) {
        if (n <= 0) return;
        if (nb + (int64_t)n > (int64_t)INT_MAX) throw BadArg("database would exceed 2^31-1 rows");
        if (!ready) { nb += n; return; }
        setDevice();
        growRows(roundUp(nb + n, kBM), s);
        // rows go to the chunked database layout (kernels.hpp, blk_off), Cosine
        // rows normalised in fp32 (reference src/FlatIndex.mm:241-242) and then
        // rounded to the storage type
        const int64_t chunk = std::max<int64_t>(1, (int64_t)(kStageBytes / (sizeof(float) * dim)));
        for (int64_t r0 = 0; r0 < n; r0 += chunk) {
            const int64_t rn = std::min<int64_t>(chunk, n - r0);
            const float* from = src + r0 * dim;
            if (kind != hipMemcpyDeviceToDevice) {
                stage.ensure((size_t)rn * dim * sizeof(float));
                HIPC(hipMemcpyAsync(stage.p, from, (size_t)rn * dim * sizeof(float), kind, s));
                from = stage.as<float>();
            }
            const float* scale = nullptr;
            if (metric == Metric::Cosine) {
                inv.ensure((size_t)rn * sizeof(float));
                launch_row_inv_norms(from, rn, dim, inv.as<float>(), s);
                scale = inv.as<float>();
            }
            launch_store_rows_blk(from, rn, dim, scale, X.p, nb + r0, dpad, storage, s);
        }
        launch_row_norms_blk(X.p, nb, n, dpad, storage, xn.as<float>() + nb, s);
        maxBits.ensure(sizeof(unsigned));
        HIPC(hipMemsetAsync(maxBits.p, 0, sizeof(unsigned), s));
        launch_max_norm(xn.as<float>() + nb, n, maxBits.as<unsigned>(), s);
        float m = 0.0f;
        HIPC(hipMemcpyAsync(&m, maxBits.p, sizeof(float), hipMemcpyDeviceToHost, s));
        HIPC(hipStreamSynchronize(s));
        if (m > xnMax) xnMax = m;
        nb += n;
    }

    // Sample row r is database row r * stride (R is a multiple of kBM).
    void ensureSample(RowSample& sm, int64_t R, int stride, hipStream_t s) {
        if (sm.nb == nb && sm.R == R && sm.stride == stride) return;
        std::vector<int> idx((size_t)R);
        for (int64_t r = 0; r < R; ++r) idx[(size_t)r] = (int)(r * stride);
        sm.idx.ensure(idx.size() * sizeof(int));
        sm.X.ensure((size_t)R * dpad * esize);
        sm.xn.ensure((size_t)R * sizeof(float));
        HIPC(hipMemcpyAsync(sm.idx.p, idx.data(), idx.size() * sizeof(int), hipMemcpyHostToDevice, s));
        launch_gather_rows_blk(X.p, sm.idx.as<int>(), (int)R, dpad, storage, sm.X.p, s);
        launch_gather_f32(xn.as<float>(), sm.idx.as<int>(), (int)R, sm.xn.as<float>(), s);
        HIPC(hipStreamSynchronize(s));
        sm.nb = nb;
        sm.R = R;
        sm.stride = stride;
    }

    ScanParams scanParams(const void* Xs, const float* xns, int64_t nrows, int64_t rps, int nsplit, int idStride,
                          const void* Q, const float* qn, int nq, const float* tk, const int* ti, int cap) const {
        ScanParams p;
        std::memset(&p, 0, sizeof p);
        p.X = Xs; p.xnorm = xns; p.xnorm_max = xnMax; p.nrows = nrows; p.rows_per_split = rps; p.nsplit = nsplit;
        p.id_stride = idStride;
        p.Q = Q; p.qnorm = qn; p.nq = nq; p.nqb = (nq + kBN - 1) / kBN; p.dpad = dpad;
        p.tau_key = tk; p.tau_id = ti;
        p.cand = cand.as<uint2>(); p.cnt = cnt.as<int>(); p.cap = cap;
        p.qgroup = qgroupKnob;
        p.wide = curWide ? 1 : 0;
        return p;
    }

    void scan(const void* Xs, const float* xns, int64_t nrows, int64_t rps, int nsplit, int idStride,
              const void* Q, const float* qn, int nq, const float* tk, const int* ti, int cap,
              hipStream_t s, int pass = kPassFull, bool allowSmall = true) {
        cand.ensure((size_t)nq * nsplit * cap * sizeof(uint2));
        cnt.ensure((size_t)nq * nsplit * sizeof(int));
        const ScanParams p = scanParams(Xs, xns, nrows, rps, nsplit, idStride, Q, qn, nq, tk, ti, cap);
        launch_scan_filter(p, kernMetric(), pass, storage, s, allowSmall);
    }

    SelectParams selectParams(int nq, int nsplit, int cap, int k, int j) const {
        SelectParams sp;
        std::memset(&sp, 0, sizeof sp);
        sp.cand = cand.as<uint2>(); sp.cnt = cnt.as<int>();
        sp.nsplit = nsplit; sp.cap = cap; sp.nq = nq; sp.k = k; sp.j = j; sp.j2 = j;
        sp.metric = kernMetric();
        sp.out_stride = k;
        return sp;
    }

    // The streaming top-k search of mb raw fp32 queries (device rows of dim
    // values; the scan prepares them itself): two launches, no staging.
    // cd / cn: mb * nsplit1 * k entries and mb * nsplit1 counts.
    void streamBatch(const float* dq, int mb, int k, const Plan& pl, uint2* cd, int* cn, int32_t* oIds,
                     float* oVals, hipStream_t s) {
        ScanParams p = scanParams(X.p, xn.as<float>(), nb, pl.rps1, pl.nsplit1, 1, nullptr, nullptr, mb, nullptr,
                                  nullptr, k);
        p.cand = cd; p.cnt = cn;
        p.qraw = dq; p.qdim = dim; p.qcos = metric == Metric::Cosine ? 1 : 0;
        launch_scan_topk(p, kernMetric(), storage, s);
        SelectParams sp = selectParams(mb, pl.nsplit1, k, k, 1);
        sp.cand = cd; sp.cnt = cn;
        sp.out_ids = oIds; sp.out_vals = oVals;
        launch_merge_lists(sp, s);
    }

    // Search mb staged queries (storage type, qh or qbuf; norms in qnorm) and
    // write rows [0, mb) of the outputs.
    void searchBatch(int mb, int k, const Plan& pl, int32_t* oIds, float* oVals, hipStream_t s) {
        curWide = pl.wide;
        const void* Q = storage == kF32 ? qbuf.p : qh.p;
        const float* qn = qnorm.as<float>();
        if (argminPath(mb, k)) {
            best.ensure((size_t)mb * sizeof(unsigned long long));
            launch_fill_u64(best.as<unsigned long long>(), mb, ~0ull, s);
            ScanParams p;
            std::memset(&p, 0, sizeof p);
            p.X = X.p; p.xnorm = xn.as<float>(); p.xnorm_max = xnMax; p.nrows = nb;
            splitPlan(nb, mb, dpad, storage, p.rows_per_split, p.nsplit, true, 1, concurrency(kPassArgmin));
            p.id_stride = 1;
            p.Q = Q; p.qnorm = qn; p.nq = mb; p.nqb = (mb + kBN - 1) / kBN; p.dpad = dpad;
            p.cap = 1;
            p.best = best.as<unsigned long long>();
            launch_scan_filter(p, kernMetric(), kPassArgmin, storage, s);
            launch_argmin_finalize(best.as<unsigned long long>(), mb, kernMetric(), oIds, oVals, s);
            return;
        }
        tauSk.ensure((size_t)mb * 4); tauSi.ensure((size_t)mb * 4);
        tauS2k.ensure((size_t)mb * 4); tauS2i.ensure((size_t)mb * 4);
        total.ensure((size_t)mb * 4);
        tauGk.ensure((size_t)mb * 4); tauGi.ensure((size_t)mb * 4);
        tauKk.ensure((size_t)mb * 4); tauKi.ensure((size_t)mb * 4);
        status.ensure((size_t)mb * 4);

        // tauS holds "no bound" from the query preparation
        if (pl.direct) {
            scan(X.p, xn.as<float>(), nb, pl.rps1, pl.nsplit1, 1, Q, qn, mb,
                 tauSk.as<float>(), tauSi.as<int>(), pl.cap1, s);
            SelectParams sp = selectParams(mb, pl.nsplit1, pl.cap1, k, 1);
            sp.out_ids = oIds; sp.out_vals = oVals;
            sp.expect = (int)std::min<int64_t>(nb, INT_MAX);   // every row is stored
            launch_select(sp, s);
            return;
        }

        // the retry round's buffers -- and the candidate pool every pass
        // shares -- are sized before any pass writes candidates
        RetryRound rr = retryPrepare(mb, k, pl, Q, qn, s);
        ensureSample(smp[0], pl.R0, pl.stride, s);
        if (pl.Rb) ensureSample(smp[1], pl.Rb, pl.strideb, s);
        if (traceOn())
            std::fprintf(stderr, "[mflat trace] mb=%d k=%d nb=%lld R0=%lld stride=%d j=%d "
                         "L0 %dx%d Rb=%lld jb=%d L1 splits=%d cap=%d\n", mb, k, (long long)nb, (long long)pl.R0,
                         pl.stride, pl.j, pl.nsplit0, pl.cap0, (long long)pl.Rb, pl.jb, pl.nsplit1, pl.cap1);
        // L0: sample, no bound -> speculative (j-th) and guaranteed (k-th) bounds
        scan(smp[0].X.p, smp[0].xn.as<float>(), pl.R0, pl.rps0, pl.nsplit0, pl.stride, Q, qn, mb,
             tauSk.as<float>(), tauSi.as<int>(), pl.cap0, s, kPassSample);
        {
            SelectParams sp = selectParams(mb, pl.nsplit0, pl.cap0, k, pl.j);
            sp.expect = (int)pl.R0;   // the sample is stored whole
            sp.j2 = pl.j2;
            sp.tau_j_key = tauSk.as<float>(); sp.tau_j_id = tauSi.as<int>();
            sp.tau_j2_key = tauS2k.as<float>(); sp.tau_j2_id = tauS2i.as<int>();
            sp.tau_k_key = tauGk.as<float>(); sp.tau_k_id = tauGi.as<int>();
            launch_select(sp, s);
        }
        // L0b (optional): the second sample under the first one's speculative
        // bound; its jb-th best, where it stored that many, tightens the bound
        if (pl.Rb) {
            scan(smp[1].X.p, smp[1].xn.as<float>(), pl.Rb, pl.rpsb, pl.nsplitb, pl.strideb, Q, qn, mb,
                 tauSk.as<float>(), tauSi.as<int>(), pl.capb, s, kPassSample);
            tauBk.ensure((size_t)mb * 4); tauBi.ensure((size_t)mb * 4);
            SelectParams sp = selectParams(mb, pl.nsplitb, pl.capb, pl.jb2 ? pl.jb2 : pl.jb, pl.jb);
            if (pl.jb2) {
                tauB2k.ensure((size_t)mb * 4); tauB2i.ensure((size_t)mb * 4);
                sp.tau_j_key = tauBk.as<float>(); sp.tau_j_id = tauBi.as<int>();
                sp.tau_k_key = tauB2k.as<float>(); sp.tau_k_id = tauB2i.as<int>();
            } else {
                sp.tau_k_key = tauBk.as<float>(); sp.tau_k_id = tauBi.as<int>();
            }
            // ~j Rb / R0 candidates a query, spread as an order statistic
            sp.expect = (int)std::min(3.0 * (double)pl.j * (double)pl.Rb / (double)pl.R0 + 64.0, 1e9);
            launch_select(sp, s);
            launch_tau_min(tauSk.as<float>(), tauSi.as<int>(), tauBk.as<float>(), tauBi.as<int>(), mb, s);
            if (pl.jb2)
                launch_tau_min(tauS2k.as<float>(), tauS2i.as<int>(), tauB2k.as<float>(), tauB2i.as<int>(), mb, s);
        }
        // L1: full database with the speculative bound
        scan(X.p, xn.as<float>(), nb, pl.rps1, pl.nsplit1, 1, Q, qn, mb,
             tauSk.as<float>(), tauSi.as<int>(), pl.cap1, s);
        {
            SelectParams sp = selectParams(mb, pl.nsplit1, pl.cap1, k, k);
            sp.out_ids = oIds; sp.out_vals = oVals;
            sp.tau_k_key = tauKk.as<float>(); sp.tau_k_id = tauKi.as<int>();
            sp.status = status.as<int>();
            sp.total = total.as<int>();
            // survivors per query spread as the bound's order statistic
            // (Gamma(j) / R0 of the rows): ~99% of queries stay under 3x the mean
            // for j >= 3
            sp.expect = (int)std::min(3.0 * pl.e1 + 64.0, 1e9);
            launch_select(sp, s);
        }

        retries(mb, k, rr, Q, qn, oIds, oVals, s);
    }

    // Verification and retries, as a fixed launch sequence whose work list the
    // device builds (no host round trip): a query is exact unless its
    // full-pass select reported an overflow or fewer than k stored rows. One
    // round (retry_plan: bounds, pooled regions and the rerun queries' rows in
    // one block; pooled scan; select) reruns up to rmax of them, each with
    // one candidate region of its own:
    //   overflow: under the k-th best it stored, the region sized by the rows
    //             it saw under its looser bound -- a subset, so the rerun is
    //             final;
    //   too few:  under the sample's j2-th best (rarely still too few), then
    //             its guaranteed k-th, the region sized for that bound (if it
    //             overflows, the next round is the final kind above).
    // Launches with an empty list exit at once. Three counters come back with
    // the batch's final synchronisation; only if a query is left (more than
    // rmax failed, a region did not fit the pool, a rerun failed again) does
    // the host run further rounds before returning.
    // Every rerun either ends a query or moves it up its bound ladder, so the
    // rounds terminate.
    struct RetryRound {
        bool batchSmall = false;
        int rmax = 1, rowsPad = kBN, rowBytes = 0;
        int64_t rps = 0;
        int nsplit = 1;
        RetryLadder lad{};
        int k = 1;
        double expect = 0.0;
    };

    RetryRound retryPrepare(int mb, int k, const Plan& pl, const void* Q, const float* qn, hipStream_t s) {
        (void)Q;
        (void)qn;
        RetryRound rr;
        rr.k = k;
        rr.batchSmall = small_scan_fits(mb, dpad, storage);
        // pooled capacities of the ladder's bounds: ~rank nb / R0 rows
        // admitted, three times that (and at least k, so an overflowing rerun
        // keeps a k-th best) before the final kind of rerun takes over
        auto capFor = [&](int rank) {
            const double e = (double)rank * (double)nb / std::max<double>(1.0, (double)pl.R0);
            return (int)std::min<double>((double)std::max<int64_t>(nb, 1), std::max(3.0 * e + 256.0, (double)k));
        };
        std::memset(&rr.lad, 0, sizeof rr.lad);
        if (pl.j2 > pl.j) {
            rr.lad.j2_key = tauS2k.as<float>(); rr.lad.j2_id = tauS2i.as<int>();
            rr.lad.cap_j2 = capFor(pl.j2);
        }
        rr.lad.g_key = tauGk.as<float>(); rr.lad.g_id = tauGi.as<int>();
        rr.lad.cap_g = capFor(k);
        // a window of rmax queries whose regions fit the candidate budget
        int rmax = std::max(1, std::min({mb, retryWindow > 0 ? retryWindow : rr.batchSmall ? kSmallMaxQ : kRetryMax,
                                         kRetryPlanMax}));
        const size_t perQ = (size_t)std::max(rr.lad.cap_g, rr.lad.cap_j2) * sizeof(uint2);
        while (rmax > 1 && (size_t)rmax * perQ > kCandBudget) rmax = (rmax + 1) / 2;
        rr.rmax = rmax;
        rr.rowsPad = (int)roundUp(rmax, kBN);
        rr.rowBytes = dpad * esize;
        // Retries run the kernel family of the passes their bounds came from
        // (the whole batch's), so every bound is compared with keys computed
        // the same way (a guaranteed bound must admit its own rows); a wide
        // batch's window runs the 128-query tiled kernel, whose keys are the
        // wide kernel's, so a window of up to 128 queries costs one 128-query
        // block. Pooled regions do not depend on the split plan: it only
        // spreads the work, made for one block of queries (a window rarely
        // holds more: the launch covers rmax, and blocks past the device's
        // count exit at once).
        splitPlan(nb, std::min(rmax, kBN), dpad, storage, rr.rps, rr.nsplit, rr.batchSmall,
                  rr.batchSmall ? 1 : kRetryMinTiles, concurrency(kPassRetry, false));
        // j2 reruns, the usual kind: ~j2 nb / R0 candidates
        rr.expect = 1.5 * std::max(pl.j2, 2) * (double)nb / std::max<double>(1.0, (double)pl.R0) + 2.0 * k;
        if (pl.jb2) rr.expect = 1.5 * pl.jb2 * (double)nb / (double)pl.Rb + 2.0 * k;

        rl.ensure(mb, rmax, s);
        cQ.ensure((size_t)rr.rowsPad * rr.rowBytes);
        cQn.ensure((size_t)rr.rowsPad * 4);
        // one buffer for every pass's candidates and the retry pool, sized now
        // so no later pass reallocates it under another's candidates
        cand.ensure(std::max((size_t)rmax * perQ, (size_t)mb * pl.perQuery * sizeof(uint2)));
        return rr;
    }

    RetryPlanArgs retryArgs(int mb, const RetryRound& rr, const void* Q, const float* qn, bool first,
                            bool drain = false) const {
        RetryPlanArgs a;
        std::memset(&a, 0, sizeof a);
        a.status = status.as<int>();
        a.mb = mb;
        a.first = first ? 1 : 0;
        a.tau_k_key = tauKk.as<float>();
        a.tau_k_id = tauKi.as<int>();
        a.total = total.as<int>();
        a.ladder = rr.lad;
        a.pool_entries = (int64_t)(cand.bytes / sizeof(uint2));
        // drain: the host's fallback, whose pool always holds one query's region
        if (retryPool > 0 && !drain) a.pool_entries = std::min<int64_t>(a.pool_entries, retryPool);
        a.rmax = rr.rmax;
        a.all_rows = (int)std::max<int64_t>(nb, 1);
        a.lists = rl.lists();
        a.Q = Q;
        a.qn = qn;
        a.row_bytes = rr.rowBytes;
        a.dst_q = cQ.p;
        a.dst_qn = cQn.as<float>();
        a.rows_pad = rr.rowsPad;
        return a;
    }

    void retries(int mb, int k, const RetryRound& rr, const void* Q, const float* qn, int32_t* oIds, float* oVals,
                 hipStream_t s) {
        const RetryLists L = rl.lists();
        auto round = [&](bool first, bool drain) {
            launch_retry_plan(retryArgs(mb, rr, Q, qn, first, drain), s);
            ScanParams p = scanParams(X.p, xn.as<float>(), nb, rr.rps, rr.nsplit, 1, cQ.p, cQn.as<float>(), rr.rmax,
                                      L.tk, L.ti, 1);
            p.nq_dev = L.counters + 1;
            p.qcnt = L.qcnt; p.qoff = L.qoff; p.qcap = L.qcap;
            p.wide = 0;   // the tiled kernel (same keys as the wide one)
            launch_scan_filter(p, kernMetric(), kPassRetry, storage, s, rr.batchSmall);
            SelectParams sp = selectParams(rr.rmax, 1, 1, k, k);
            sp.cnt = L.qcnt;
            sp.qoff = L.qoff; sp.qcap = L.qcap;
            sp.nq_dev = L.counters + 1;
            sp.qmap = L.idx;
            sp.out_ids = oIds; sp.out_vals = oVals;
            sp.tau_k_key = tauKk.as<float>(); sp.tau_k_id = tauKi.as<int>();
            sp.status = status.as<int>();
            sp.total = total.as<int>();
            sp.fail_count = L.counters + 2;
            sp.expect = (int)std::min(rr.expect, 1e9);
            launch_select(sp, s);
            hostCounters.ensure();
            HIPC(hipMemcpyAsync(hostCounters.p, L.counters, 3 * sizeof(int), hipMemcpyDeviceToHost, s));
            HIPC(hipStreamSynchronize(s));
            return hostCounters.p[0] - hostCounters.p[1] + hostCounters.p[2];   // queries left
        };
        int left = round(true, false);
        if (traceOn())
            std::fprintf(stderr, "[mflat trace] retries: %d of %d queries failed the full pass, %d rerun, %d left\n",
                         hostCounters.p[0], mb, hostCounters.p[1], left);
        // Host fallback: a pool of nb entries holds any single region, so
        // every round schedules at least one query.
        const int64_t limit = 4 * ((int64_t)mb / rr.rmax + 2) + 3LL * mb;
        for (int64_t r = 0; left > 0; ++r) {
            if (r > limit) throw std::runtime_error("flat search: retries did not converge");
            cand.ensure((size_t)std::max<int64_t>(nb, 1) * sizeof(uint2));
            left = round(false, true);
        }
    }

    // The allocation-free search: the streaming top-k scan with its workspace
    // (queries, norms, per-split counts and candidates) carved out of the
    // device's scratch array. Stream-ordered: returns once the work is
    // enqueued on s. Nothing here allocates: no DevBuf, no timer events.
    int searchNoAlloc(const float* dq, int m, int k, int32_t* ids, float* vals, hipStream_t s) {
        if (!ready) throw NotReady("no usable HIP device: flat search needs a gfx950 GPU");
        if (m > kNoAllocMaxQ)
            throw BadArg("allocation-free search: at most " + std::to_string(kNoAllocMaxQ) + " queries per call (got " +
                         std::to_string(m) + ")");
        if (k > kStreamTopK)
            throw BadArg("allocation-free search: k at most " + std::to_string(kStreamTopK) + " (got " +
                         std::to_string(k) + ")");
        if (dim > kNoAllocMaxDim || !small_scan_fits(kNoAllocMaxQ, dpad, storage))
            throw BadArg("allocation-free search: dimension " + std::to_string(dim) +
                         " too large (at most 992 for fp32 storage, 2016 for fp16 / bf16)");
        if (m <= 0) return 0;
        if (k < 1) k = 1;
        setDevice();
        prof_suppress(true);
        struct Unsuppress {
            ~Unsuppress() { prof_suppress(false); }
        } unsuppress;
        if (nb == 0) {
            launch_fill_empty(ids, vals, (int64_t)m * k, emptyValue(), s);
            return k;
        }
        char* base = static_cast<char*>(noalloc_scratch(device));
        Plan pl;
        // the split lists and counts of m queries must fit the scratch (with
        // 256-byte alignment slack for both carves)
        setStreamPlan(pl, k, (int64_t)((kNoAllocScratchBytes - 512) / ((size_t)m * ((size_t)k * sizeof(uint2) + sizeof(int)))));
        auto carve = [&](size_t& at, size_t bytes) {
            const size_t off = at;
            at = (at + bytes + 255) / 256 * 256;
            return base + off;
        };
        size_t at = 0;
        int* cn = reinterpret_cast<int*>(carve(at, (size_t)m * pl.nsplit1 * sizeof(int)));
        uint2* cd = reinterpret_cast<uint2*>(carve(at, (size_t)m * pl.nsplit1 * k * sizeof(uint2)));
        if (at > kNoAllocScratchBytes)
            throw BadArg("allocation-free search: workspace of " + std::to_string(at) + " bytes exceeds the " +
                         std::to_string(kNoAllocScratchBytes) + "-byte scratch");
        streamBatch(dq, m, k, pl, cd, cn, ids, vals, s);
        return k;
    }

    int searchDev(const float* dq, int m, int k, int32_t* ids, float* vals, hipStream_t s) {
        if (!ready) throw NotReady("no usable HIP device: flat search needs a gfx950 GPU");
        if (m <= 0) return 0;
        if (k < 1) k = 1;
        if (k > kMaxK) {
            if (!warnedK) {
                MFLAT_LOG_WARN("k=%d clamped to MFLAT_MAX_K=%d", k, kMaxK);
                warnedK = true;
            }
            k = kMaxK;
        }
        setDevice();
        if (nb == 0) {
            launch_fill_empty(ids, vals, (int64_t)m * k, emptyValue(), s);
            HIPC(hipStreamSynchronize(s));
            return k;
        }
        // batch the queries so the candidate workspace stays bounded
        int64_t mb = m;
        Plan pl = plan(mb, k);
        for (int it = 0; it < 4 && (size_t)mb * pl.perQuery * sizeof(uint2) > kCandBudget; ++it) {
            mb = (int64_t)(kCandBudget / (pl.perQuery * sizeof(uint2)));
            mb = std::max<int64_t>(kBN, mb / kBN * kBN);
            pl = plan(mb, k);
        }
        for (int64_t b0 = 0; b0 < m; b0 += mb) {
            const int n = (int)std::min<int64_t>(mb, m - b0);
            const Plan pb = (n == mb) ? pl : plan(n, k);
            if (pb.stream) {
                cand.ensure((size_t)n * pb.nsplit1 * k * sizeof(uint2));
                cnt.ensure((size_t)n * pb.nsplit1 * sizeof(int));
                streamBatch(dq + b0 * dim, n, k, pb, cand.as<uint2>(), cnt.as<int>(), ids ? ids + b0 * k : nullptr,
                            vals ? vals + b0 * k : nullptr, s);
                continue;
            }
            const int64_t nPad = roundUp(n, kBN);
            // queries in the database's element type (Cosine normalised first),
            // their norms, and every query's first bound, in one launch
            DevBuf& qs = storage == kF32 ? qbuf : qh;
            qs.ensure((size_t)nPad * dpad * esize);
            qnorm.ensure((size_t)nPad * sizeof(float));
            const bool bounded = !argminPath(n, k);
            if (bounded) {
                tauSk.ensure((size_t)n * 4);
                tauSi.ensure((size_t)n * 4);
            }
            launch_prep_queries(dq + b0 * dim, n, dim, nPad, dpad, storage, metric == Metric::Cosine, qs.p,
                                qnorm.as<float>(), bounded ? tauSk.as<float>() : nullptr,
                                bounded ? tauSi.as<int>() : nullptr, s);
            searchBatch(n, k, pb, ids ? ids + b0 * k : nullptr, vals ? vals + b0 * k : nullptr, s);
        }
        HIPC(hipStreamSynchronize(s));
        return k;
    }
};

FlatIndex::FlatIndex(int dim, Metric metric, Storage storage) : d_(new Impl) {
    if (storage != kF32 && storage != kF16 && storage != kBF16) throw BadArg("unknown storage type");
    d_->dim = dim;
    d_->dpad = (int)roundUp(dim, kBK);
    d_->metric = metric;
    d_->storage = storage;
    d_->esize = elem_bytes(storage);
    if (const char* v = std::getenv("MFLAT_RETRY_WINDOW")) d_->retryWindow = std::max(0, std::atoi(v));
    if (const char* v = std::getenv("MFLAT_RETRY_POOL")) d_->retryPool = std::max<long long>(0, std::atoll(v));
    if (const char* v = std::getenv("MFLAT_STREAM_MAXQ")) d_->streamMaxQ = std::max(0, std::atoi(v));
    if (const char* v = std::getenv("MFLAT_STREAM_SPLITS")) d_->streamSplits = std::max(0, std::atoi(v));
    if (const char* v = std::getenv("MFLAT_QGROUP")) d_->qgroupKnob = std::max(0, std::atoi(v));
    if (const char* v = std::getenv("MFLAT_WIDE")) d_->wideKnob = std::atoi(v) != 0 ? 1 : 0;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        MFLAT_LOG_INFO("no HIP device - flat search unavailable on this index");
        return;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        MFLAT_LOG_ERROR("device %d is %s; this build targets gfx950 only", dev, prop.gcnArchName);
        return;
    }
    if (hipStreamCreateWithFlags(&d_->stream, hipStreamNonBlocking) != hipSuccess) {
        MFLAT_LOG_ERROR("hipStreamCreate failed");
        return;
    }
    d_->device = dev;
    d_->ready = true;
}

FlatIndex::~FlatIndex() {
    if (!d_) return;
    if (d_->device >= 0) (void)hipSetDevice(d_->device);
    if (d_->stream) (void)hipStreamSynchronize(d_->stream);
    for (auto& sm : d_->smp) sm.release();
    for (DevBuf* b : {&d_->X, &d_->xn, &d_->stage, &d_->inv, &d_->qin, &d_->outIds,
                      &d_->outVals, &d_->qbuf, &d_->qh, &d_->qnorm, &d_->cand, &d_->cnt, &d_->tauSk, &d_->tauSi, &d_->tauS2k, &d_->tauS2i, &d_->maxBits,
                      &d_->tauGk, &d_->tauGi, &d_->tauKk, &d_->tauKi, &d_->tauBk, &d_->tauBi, &d_->tauB2k, &d_->tauB2i, &d_->status, &d_->cQ, &d_->cQn,
                      &d_->best, &d_->total})
        b->release();
    d_->rl.release();
    d_->hostCounters.release();
    if (d_->stream) (void)hipStreamDestroy(d_->stream);
}

bool FlatIndex::ready() const { return d_->ready; }
int FlatIndex::size() const { return (int)d_->nb; }
int FlatIndex::dim() const { return d_->dim; }
Metric FlatIndex::metric() const { return d_->metric; }
Storage FlatIndex::storage() const { return static_cast<Storage>(d_->storage); }

void FlatIndex::add(const float* rows, int n) {
    d_->append(rows, n, hipMemcpyHostToDevice, d_->stream);
}

void FlatIndex::addDevice(const float* rows, int n, hipStream_t s) {
    d_->append(rows, n, hipMemcpyDeviceToDevice, s ? s : d_->stream);
}

void FlatIndex::reset() {
    if (d_->ready) {
        d_->setDevice();
        HIPC(hipStreamSynchronize(d_->stream));
    }
    d_->X.release();
    d_->xn.release();
    d_->capRows = 0;
    d_->nb = 0;
    d_->xnMax = 0.0f;
    for (auto& sm : d_->smp) sm.nb = -1;
}

int FlatIndex::search(const float* q, int m, int k, int32_t* ids, float* dists) {
    Impl& I = *d_;
    if (!I.ready) throw NotReady("no usable HIP device: flat search needs a gfx950 GPU");
    if (m <= 0) return 0;
    const int kk = std::min(std::max(k, 1), kMaxK);
    I.setDevice();
    hipStream_t s = I.stream;
    I.qin.ensure((size_t)m * I.dim * sizeof(float));
    I.outIds.ensure((size_t)m * kk * sizeof(int32_t));
    I.outVals.ensure((size_t)m * kk * sizeof(float));
    HIPC(hipMemcpyAsync(I.qin.p, q, (size_t)m * I.dim * sizeof(float), hipMemcpyHostToDevice, s));
    const int used = I.searchDev(I.qin.as<float>(), m, k, I.outIds.as<int32_t>(), I.outVals.as<float>(), s);
    if (ids) HIPC(hipMemcpyAsync(ids, I.outIds.p, (size_t)m * used * sizeof(int32_t), hipMemcpyDeviceToHost, s));
    if (dists) HIPC(hipMemcpyAsync(dists, I.outVals.p, (size_t)m * used * sizeof(float), hipMemcpyDeviceToHost, s));
    HIPC(hipStreamSynchronize(s));
    return used;
}

int FlatIndex::searchDevice(const float* q, int m, int k, int32_t* ids, float* dists, hipStream_t s) {
    return d_->searchDev(q, m, k, ids, dists, s ? s : d_->stream);
}

int FlatIndex::searchDeviceNoAlloc(const float* q, int m, int k, int32_t* ids, float* dists, hipStream_t s) {
    return d_->searchNoAlloc(q, m, k, ids, dists, s ? s : d_->stream);
}

}  // namespace mflat_amd
