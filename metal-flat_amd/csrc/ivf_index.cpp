// SPDX-License-Identifier: Apache-2.0
// ivf_index.cpp -- host side of the IVF index on one MI355X.
//
// Build (reference src/IvfIndex.mm:480-516, src/CoarseQuantizer.mm:104-159):
// Cosine rows normalised; device k-means (kmeansTrainDevice: 12 iterations,
// 256 training points per centroid); the rows stored cell-major in the flat
// scan's chunked layout, each cell padded to a multiple of kBM rows (zero rows,
// never reported); the centroids go to an fp32 L2 FlatIndex, the coarse probe.
//
// Search of a batch (reference src/IvfIndex.mm:759-879 and searchCpu :518-560):
//   probe    the coarse FlatIndex's top-nprobe over the centroids (nearest
//            first, ties to the lower cell id: the reference's FlatIndex probe
//            and its partial_sort over (distance, cell), CoarseQuantizer.mm:170-188)
//   A bound  each query's nearest cells, up to the first that brings its scan
//            to k rows (at most kBoundRanks), no bound; the k-th best (key,
//            scan position) of what it stored is a GUARANTEED bound -- the k-th
//            best over a subset of the probed rows is never better than the
//            k-th best over all of them (skipped for nprobe = 1)
//   A2       (IVF-PQ, when a cell outgrows the sample) A's cells in full under
//            A's bound; the smaller of the two bounds stays
//   B scan   all probed cells with that bound, into one region per (query,
//            cell) plus a spill region per query for what overflows them;
//            select the k best of the stored survivors. Exact unless the spill
//            overflowed too.
//   retry    those queries rerun B with the k-th best of what they stored as
//            the bound, into regions that hold a whole cell each (no overflow
//            is possible), so one retry is final.
//   finalize scan positions -> original row ids.
// The ranking key and the bound test are the flat index's (kernels.hpp), so a
// row's key is the same in every pass of a search.
#include "ivf_index.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <numeric>
#include <string>
#include <vector>

#include "ivf_kernels.hpp"
#include "kernels.hpp"
#include "kmeans.hpp"
#include "log.hpp"
#include "pq_kernels.hpp"

namespace mflat_amd {
namespace {

void hipCheck(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) throw std::bad_alloc();
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
#define HIPC(x) hipCheck((x), #x)

constexpr int kTrainIters = 12;            // reference src/IvfIndex.mm:493
constexpr int kPointsPerCentroid = 256;    // reference src/CoarseQuantizer.mm:116-117
constexpr size_t kCandBudget = size_t(3) << 30;   // candidate regions per batch
constexpr int kBoundRanks = 4;             // bound pass: most cells per query
constexpr int kMaxSubquantizers = 128;     // PQ: M x 256 floats of one query's table fit LDS
constexpr int64_t kHostTableMax = 1 << 17;  // retries of at most this many entries build their table on the host

int64_t roundUp(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

int pow2ceil(int64_t x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() { release(); }
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

}  // namespace

struct IvfIndex::Impl {
    int dim = 0, dpad = 0;
    Metric metric = Metric::L2;
    int storage = kF32;
    int esize = 4;
    int nlistReq = 1;
    int nlist = 0;
    int64_t n = 0;
    int64_t rowsPad = 0;   // stored rows, cells padded to kBM
    int maxCell = 0;
    bool built = false;
    bool devOk = false;
    bool warnedK = false;
    int device = -1;
    hipStream_t stream = nullptr;

    // IVF-PQ (pqM > 0): residual product quantization instead of stored rows
    int pqM = 0, dsub = 0;
    // Diagnostics knobs, read once when the index is created (never during a
    // search): MFLAT_IVF_TILES = 128 / 32 makes every work item wide / narrow,
    // MFLAT_IVF_CAP_B = n overrides the full pass's region capacity. Results
    // never depend on them, only the work done; 0 = not set.
    int tilesKnob = 0, capBKnob = 0;
    bool trace = false;   // MFLAT_TRACE: per-search survivor statistics on stderr
    bool rerankReq = false;    // keep the full rows for exact reranking (set before build)
    bool fullStored = false;   // ... latched at build
    DevBuf dCodes, dPqc, dNorms, dT, dCentD, dFull;
    std::vector<float> hPqc;
    bool pq() const { return pqM > 0; }

    std::unique_ptr<FlatIndex> coarse;
    DevBuf X, xn, maxBits;
    float xnMax = 0.0f;
    DevBuf dCellSize, dCellPad, dCellStart, dRid, dCellOrder;
    std::vector<float> hCent;
    std::vector<int> hStart, hRid, hCellOrder;

    // per-search workspace
    DevBuf qin, outIds, outVals, qbuf, qh, qnorm, qrm, probe, pos, posOut, cand, cnt;
    DevBuf tauAk, tauAi, tauKk, tauKi, tauRk, tauRi, status;
    DevBuf cQ, cQn, cTk, cTi, cIdx, cProbe, cPos;
    DevBuf lut, base, cLut, cBase, shortIds, rrCand, rrCnt, rrSel;
    IvfWorkTable wt;
    std::vector<int> hProbe;

    int kernMetric() const { return metric == Metric::L2 ? 0 : 1; }
    float emptyValue() const { return metric == Metric::L2 ? INFINITY : -INFINITY; }
    void setDevice() const {
        if (device >= 0) HIPC(hipSetDevice(device));
    }

    void buildFrom(const float* src, int nrows, hipMemcpyKind kind, hipStream_t s) {
        if (nrows <= 0) return;   // reference src/IvfIndex.mm:481: nothing to build
        if (!devOk) throw NotReady("no usable HIP device: IVF build needs a gfx950 GPU");
        setDevice();
        const size_t rowB = (size_t)dim * sizeof(float);
        // the caller's rows are borrowed: a device copy, normalised for Cosine
        // (reference src/IvfIndex.mm:486-487, src/Distance.h:50-60)
        DevBuf data, inv;
        data.ensure((size_t)nrows * rowB);
        HIPC(hipMemcpyAsync(data.p, src, (size_t)nrows * rowB, kind, s));
        if (metric == Metric::Cosine) {
            inv.ensure((size_t)nrows * sizeof(float));
            launch_row_inv_norms(data.as<float>(), nrows, dim, inv.as<float>(), s);
            launch_scale_rows(data.as<float>(), nrows, dim, inv.as<float>(), s);
        }
        // coarse quantizer: k-means and the CSR of the final assignment
        const int nlMax = std::min(nlistReq, nrows);
        DevBuf cent, order;
        cent.ensure((size_t)nlMax * rowB);
        order.ensure((size_t)nrows * sizeof(int));
        std::vector<int> start((size_t)nlMax + 1);
        const int nl = kmeansTrainDevice(data.as<float>(), nrows, dim, nlistReq, kTrainIters, kPointsPerCentroid,
                                         cent.as<float>(), nullptr, order.as<int>(), start.data(), s);
        std::vector<int> rid((size_t)nrows);
        std::vector<float> centH((size_t)nl * dim);
        HIPC(hipMemcpyAsync(rid.data(), order.p, (size_t)nrows * sizeof(int), hipMemcpyDeviceToHost, s));
        HIPC(hipMemcpyAsync(centH.data(), cent.p, centH.size() * sizeof(float), hipMemcpyDeviceToHost, s));
        HIPC(hipStreamSynchronize(s));

        // cell-major layout: cell c at rows [pad[c], pad[c] + size[c]) of X
        std::vector<int> size((size_t)nl), cellOrder((size_t)nl);
        std::vector<int64_t> pad((size_t)nl);
        int64_t P = 0;
        int mc = 0;
        for (int c = 0; c < nl; ++c) {
            size[(size_t)c] = start[(size_t)c + 1] - start[(size_t)c];
            pad[(size_t)c] = P;
            P += roundUp(size[(size_t)c], kBM);
            mc = std::max(mc, size[(size_t)c]);
        }
        P = std::max<int64_t>(P, kBM);
        std::vector<int> slotSrc((size_t)P, -1);
        for (int c = 0; c < nl; ++c)
            for (int i = 0; i < size[(size_t)c]; ++i)
                slotSrc[(size_t)(pad[(size_t)c] + i)] = rid[(size_t)start[(size_t)c] + i];
        // work items run in decreasing cell size (the largest first), ties by cell
        std::iota(cellOrder.begin(), cellOrder.end(), 0);
        std::stable_sort(cellOrder.begin(), cellOrder.end(),
                         [&](int a, int b) { return size[(size_t)a] > size[(size_t)b]; });

        DevBuf slot, tmp;
        float xm = 0.0f;
        X.release();
        xn.release();
        if (!pq()) {
            slot.ensure((size_t)P * sizeof(int));
            tmp.ensure((size_t)P * rowB);
            HIPC(hipMemcpyAsync(slot.p, slotSrc.data(), (size_t)P * sizeof(int), hipMemcpyHostToDevice, s));
            launch_gather_rows_or_zero(data.as<float>(), slot.as<int>(), P, dim, tmp.as<float>(), s);
            X.ensure((size_t)P * dpad * esize);
            xn.ensure((size_t)P * sizeof(float));
            HIPC(hipMemsetAsync(X.p, 0, (size_t)P * dpad * esize, s));
            launch_store_rows_blk(tmp.as<float>(), P, dim, nullptr, X.p, 0, dpad, storage, s);
            launch_row_norms_blk(X.p, 0, P, dpad, storage, xn.as<float>(), s);
            maxBits.ensure(sizeof(unsigned));
            HIPC(hipMemsetAsync(maxBits.p, 0, sizeof(unsigned), s));
            launch_max_norm(xn.as<float>(), P, maxBits.as<unsigned>(), s);
            HIPC(hipMemcpyAsync(&xm, maxBits.p, sizeof(float), hipMemcpyDeviceToHost, s));
        }

        dCellSize.ensure((size_t)nl * sizeof(int));
        dCellPad.ensure((size_t)nl * sizeof(int64_t));
        dCellStart.ensure(((size_t)nl + 1) * sizeof(int));
        dRid.ensure((size_t)nrows * sizeof(int));
        dCellOrder.ensure((size_t)nl * sizeof(int));
        HIPC(hipMemcpyAsync(dCellSize.p, size.data(), (size_t)nl * sizeof(int), hipMemcpyHostToDevice, s));
        HIPC(hipMemcpyAsync(dCellPad.p, pad.data(), (size_t)nl * sizeof(int64_t), hipMemcpyHostToDevice, s));
        HIPC(hipMemcpyAsync(dCellStart.p, start.data(), ((size_t)nl + 1) * sizeof(int), hipMemcpyHostToDevice, s));
        HIPC(hipMemcpyAsync(dRid.p, order.p, (size_t)nrows * sizeof(int), hipMemcpyDeviceToDevice, s));
        HIPC(hipMemcpyAsync(dCellOrder.p, cellOrder.data(), (size_t)nl * sizeof(int), hipMemcpyHostToDevice, s));

        if (pq()) buildPq(data.as<float>(), cent.as<float>(), nrows, nl, s);

        coarse.reset(new FlatIndex(dim, Metric::L2, kF32));
        coarse->addDevice(cent.as<float>(), nl, s);
        HIPC(hipStreamSynchronize(s));

        xnMax = xm;
        nlist = nl;
        n = nrows;
        rowsPad = P;
        maxCell = mc;
        hCent.swap(centH);
        start.resize((size_t)nl + 1);
        hStart.swap(start);
        hRid.swap(rid);
        hCellOrder.swap(cellOrder);
        built = true;
    }

    // Residual product quantization of the rows (reference src/IvfPqIndex.mm:
    // 286-327, src/PqTrainer.h:37-66): per sub-space, k-means of the residuals
    // x - c (12 iterations, 256 cells, every row trains, seeds wrapping when
    // fewer rows than cells); the codes are the final assignments, stored in
    // cell order; the per-cell cross table T and the sub-centroid norms follow.
    // data: the (Cosine-normalised) rows; the CSR arrays are on the device.
    void buildPq(const float* data, const float* cent, int nrows, int nl, hipStream_t s) {
        const size_t rowB = (size_t)dim * sizeof(float);
        fullStored = rerankReq;
        dFull.release();
        if (fullStored) {   // exact rerank rows, original order, before the residual subtraction
            dFull.ensure((size_t)nrows * rowB);
            HIPC(hipMemcpyAsync(dFull.p, data, (size_t)nrows * rowB, hipMemcpyDeviceToDevice, s));
        }
        DevBuf assign, r, sub, subAssign;
        assign.ensure((size_t)nrows * sizeof(int));
        r.ensure((size_t)nrows * rowB);
        launch_cell_assign(dCellStart.as<int>(), dRid.as<int>(), nl, assign.as<int>(), s);
        launch_residuals(data, cent, assign.as<int>(), nrows, dim, r.as<float>(), s);
        dPqc.ensure((size_t)pqM * kPqKsub * dsub * sizeof(float));
        dNorms.ensure((size_t)pqM * kPqKsub * sizeof(float));
        dCodes.ensure((size_t)nrows * pqM);
        sub.ensure((size_t)nrows * dsub * sizeof(float));
        subAssign.ensure((size_t)nrows * sizeof(int));
        for (int mm = 0; mm < pqM; ++mm) {
            launch_subspace(r.as<float>(), nrows, dim, mm * dsub, dsub, sub.as<float>(), s);
            kmeansTrainDevice(sub.as<float>(), nrows, dsub, kPqKsub, kTrainIters, 0,
                              dPqc.as<float>() + (size_t)mm * kPqKsub * dsub, subAssign.as<int>(), nullptr, nullptr,
                              s, true);
            launch_pq_codes(subAssign.as<int>(), dRid.as<int>(), nrows, pqM, mm, dCodes.as<uint8_t>(), s);
        }
        launch_pq_norms(dPqc.as<float>(), pqM, dsub, dNorms.as<float>(), s);
        dT.ensure((size_t)nl * pqM * kPqKsub * sizeof(float));
        launch_pq_cell_table(cent, nl, dim, dPqc.as<float>(), pqM, dsub, dT.as<float>(), s);
        dCentD.ensure((size_t)nl * rowB);
        HIPC(hipMemcpyAsync(dCentD.p, cent, (size_t)nl * rowB, hipMemcpyDeviceToDevice, s));
        hPqc.resize((size_t)pqM * kPqKsub * dsub);
        HIPC(hipMemcpyAsync(hPqc.data(), dPqc.p, hPqc.size() * sizeof(float), hipMemcpyDeviceToHost, s));
        HIPC(hipStreamSynchronize(s));
    }

    // One fine-scan pass over the work table wt (built for nq queries).
    // The queries of a pass: storage-type rows and norms (flat rows), or the
    // lookup tables and per-entry coarse terms (PQ).
    struct QueryRefs {
        const void* Q;
        const float* qn;
        const float* lut;
        const float* base;
    };

    void scanPass(int pass, int nq, int ranks, int nprobe, int nreg, int cap, const QueryRefs& qr, const float* tk,
                  const int* ti, const int* posb, hipStream_t s, bool spill = false, int rowCap = 0) {
        cand.ensure((size_t)nq * nreg * cap * sizeof(uint2));
        cnt.ensure((size_t)nq * nreg * sizeof(int));
        // every region a work item covers gets its count from it; the others
        // (entries without a cell) stay empty
        HIPC(hipMemsetAsync(cnt.p, 0, (size_t)nq * nreg * sizeof(int), s));
        if (pq()) {
            AdcParams a;
            std::memset(&a, 0, sizeof a);
            a.codes = dCodes.as<uint8_t>(); a.cellStart = dCellStart.as<int>();
            a.lut = qr.lut; a.T = dT.as<float>(); a.base = qr.base;
            a.work = wt.work; a.nwork = wt.nwork; a.ent = wt.ent; a.pos = posb;
            a.tau_key = tk; a.tau_id = ti;
            a.cand = cand.as<uint2>(); a.cnt = cnt.as<int>(); a.cap = cap;
            a.M = pqM; a.nprobe = nprobe; a.nreg = nreg; a.spill = spill ? 1 : 0; a.rowCap = rowCap;
            a.tq = adc_tile_queries(pqM);
            launch_adc_scan(a, pass, wt.maxWork(nq, ranks, nlist), s);
            return;
        }
        const void* Q = qr.Q;
        const float* qn = qr.qn;
        ScanParams p;
        std::memset(&p, 0, sizeof p);
        p.X = X.p; p.xnorm = xn.as<float>(); p.xnorm_max = xnMax; p.nrows = rowsPad;
        p.rows_per_split = kBM; p.nsplit = 1; p.id_stride = 1;
        p.Q = Q; p.qnorm = qn; p.nq = nq; p.nqb = (nq + kBN - 1) / kBN; p.dpad = dpad;
        p.tau_key = tk; p.tau_id = ti;
        p.cand = cand.as<uint2>(); p.cnt = cnt.as<int>(); p.cap = cap;
        p.ivf_ent = wt.ent; p.ivf_pos = posb;
        p.ivf_cell_pad = dCellPad.as<int64_t>(); p.ivf_cell_size = dCellSize.as<int>();
        p.ivf_nprobe = nprobe; p.ivf_nreg = nreg; p.ivf_spill = spill ? 1 : 0; p.ivf_row_cap = rowCap;
        p.ivf_work = wt.work; p.ivf_nwork = wt.nwork;
        if (narrowMax() >= 0) launch_scan_ivf(p, kernMetric(), pass, storage, kBN, wt.maxWork(nq, ranks, nlist), s);
        p.ivf_work = wt.workN; p.ivf_nwork = wt.nwork + 1;
        launch_scan_ivf(p, kernMetric(), pass, storage, kIvfNarrow, wt.maxWorkNarrow(nq, ranks, nlist, narrowMax()),
                        s);
    }

    // Tile widths of the work tables: MFLAT_IVF_TILES = 128 / 32 (diagnostics)
    // makes every work item wide / narrow; both compute the same keys, so the
    // results never depend on it.
    // PQ work items: adc_tile_queries(M) queries, wide only.
    // Large d (a 128-query tile beyond scan_resident's LDS): the 128-query
    // items run the LDS-tiled kernel, the 32-query ones scan_resident where
    // their tile fits (else every item is wide). The two kernels issue the
    // same MFMA sequence per (query, row) pair, so their keys are
    // bit-identical and passes may mix them.
    int narrowMax() const {
        if (pq()) return 0;
        if (tilesKnob == 128) return 0;
        if (tilesKnob == 32 && ivf_narrow_fits(dpad, storage)) return -1;
        if (!resident_scan_fits(dpad, storage) && !ivf_narrow_fits(dpad, storage)) return 0;
        return kBN - kIvfNarrow;
    }
    int wideWidth() const { return pq() ? adc_tile_queries(pqM) : kBN; }

    SelectParams selectParams(int nq, int nsplit, int cap, int k) const {
        SelectParams sp;
        std::memset(&sp, 0, sizeof sp);
        sp.cand = cand.as<uint2>(); sp.cnt = cnt.as<int>();
        sp.nsplit = nsplit; sp.cap = cap; sp.nq = nq; sp.k = k; sp.j = k; sp.j2 = k;
        sp.metric = pq() ? 0 : kernMetric();   // PQ values are ADC squared distances for every metric
        sp.out_stride = k;
        return sp;
    }

    // Region capacities. capA: bound pass, per query; capB: full pass, per
    // (query, probe rank) -- a whole cell when nprobe = 1 (no bound, every row
    // stored); capR: retries, a whole cell.
    // Bound pass rows per cell: >= k (so a cell of at least k rows yields a
    // bound by itself), and few enough that the pass stays a small fraction
    // of the full one; the full pass then admits ~k * size / sampleRows rows of
    // the nearest cell.
    static int sampleRows(int k) { return std::max(4 * k, 1024); }
    int capA(int k) const {
        return (int)roundUp(std::max(1, std::min(maxCell, sampleRows(k))), 64);
    }
    int capR() const { return (int)roundUp(std::max(maxCell, 1), 64); }
    // MFLAT_IVF_CAP_B (diagnostics) overrides capB to exercise the retries;
    // the results never depend on it, only the work done.
    int capB(int k, int nprobe) const {
        if (capBKnob >= 1) return capBKnob;
        if (nprobe == 1) return capR();
        // PQ: the bound is the k-th of the whole nearest cell (A covers it, or
        // A2 does), so that cell's region holds at most k survivors and the
        // others rarely more than a few
        return pq() ? pow2ceil(std::max(2 * k, 128)) : pow2ceil(std::max(4 * k, 256));
    }

    // Search mb staged queries (qbuf / qh, norms in qnorm, probes in probe).
    void searchBatch(int mb, int k, int nprobe, int32_t* oIds, float* oVals, hipStream_t s) {
        const void* Q = storage == kF32 ? qbuf.p : qh.p;
        const float* qn = qnorm.as<float>();
        const QueryRefs qr{Q, qn, lut.as<float>(), base.as<float>()};
        wt.wideW = wideWidth();
        pos.ensure((size_t)mb * nprobe * sizeof(int));
        launch_ivf_positions(probe.as<int>(), mb, nprobe, dCellSize.as<int>(), pos.as<int>(), s);
        tauAk.ensure((size_t)mb * 4); tauAi.ensure((size_t)mb * 4);
        tauKk.ensure((size_t)mb * 4); tauKi.ensure((size_t)mb * 4);
        status.ensure((size_t)mb * 4);
        launch_fill_tau_none(tauAk.as<float>(), tauAi.as<int>(), mb, s);
        if (nprobe > 1) {
            // A: the first sampleRows(k) rows (ascending id within a cell: a
            // uniform sample) of each query's nearest cells, no bound, up to the
            // first cell that brings its scan to k rows (at most kBoundRanks)
            // -> a guaranteed bound: the k-th best of what was stored
            const int sr = sampleRows(k);
            const int ca = capA(k);
            const int ra = std::min(nprobe, kBoundRanks);
            wt.build(probe.as<int>(), mb, nprobe, ra, nlist, dCellOrder.as<int>(), narrowMax(), s, pos.as<int>(), k);
            scanPass(kPassSample, mb, ra, nprobe, ra, ca, qr, tauAk.as<float>(), tauAi.as<int>(), pos.as<int>(), s,
                     false, sr);
            SelectParams sp = selectParams(mb, ra, ca, k);
            sp.tau_k_key = tauAk.as<float>(); sp.tau_k_id = tauAi.as<int>();
            sp.expect = std::min(sr, std::max(maxCell, 1));
            launch_select(sp, s);
            if (pq() && maxCell > sr) {
                // A2 (PQ): A's cells in full under A's bound (A's work table),
                // one region of capB rows per (query, rank) (rows past it are
                // dropped: the k-th of any k stored rows is still a bound); the
                // smaller bound stays. ADC keys repeat where rows share codes,
                // so a sample of a large cell can miss a whole group of equal
                // keys and leave a bound that admits most probed rows; A2 costs
                // one more scan of the nearest cells.
                const int cr = capB(k, nprobe);
                tauRk.ensure((size_t)mb * 4); tauRi.ensure((size_t)mb * 4);
                scanPass(kPassSample, mb, ra, nprobe, ra, cr, qr, tauAk.as<float>(), tauAi.as<int>(), pos.as<int>(),
                         s);
                SelectParams sr2 = selectParams(mb, ra, cr, k);
                sr2.tau_k_key = tauRk.as<float>(); sr2.tau_k_id = tauRi.as<int>();
                sr2.expect = cr;
                launch_select(sr2, s);
                launch_tau_min(tauAk.as<float>(), tauAi.as<int>(), tauRk.as<float>(), tauRi.as<int>(), mb, s);
            }
        }
        // B: every probed cell under the bound
        const int cb = capB(k, nprobe);
        int32_t* posIds = oIds;
        if (!posIds) {
            posOut.ensure((size_t)mb * k * sizeof(int32_t));
            posIds = posOut.as<int32_t>();
        }
        // regions: one per (query, probe rank), plus a spill region per query
        wt.build(probe.as<int>(), mb, nprobe, nprobe, nlist, dCellOrder.as<int>(), narrowMax(), s);
        scanPass(kPassFull, mb, nprobe, nprobe, nprobe + 1, cb, qr, tauAk.as<float>(), tauAi.as<int>(),
                 pos.as<int>(), s, true);
        if (trace) {
            std::vector<int> c((size_t)mb * (nprobe + 1));
            HIPC(hipMemcpyAsync(c.data(), cnt.p, c.size() * sizeof(int), hipMemcpyDeviceToHost, s));
            HIPC(hipStreamSynchronize(s));
            int64_t tot = 0, spilt = 0;
            std::vector<int64_t> perq((size_t)mb, 0);
            for (size_t i = 0; i < c.size(); ++i) {
                tot += c[i];
                perq[i / (size_t)(nprobe + 1)] += c[i];
                if (i % (size_t)(nprobe + 1) == (size_t)nprobe) spilt += c[i];
            }
            const int worst = (int)(std::max_element(perq.begin(), perq.end()) - perq.begin());
            float wk = 0.0f;
            int wi = 0;
            HIPC(hipMemcpyAsync(&wk, tauAk.as<float>() + worst, 4, hipMemcpyDeviceToHost, s));
            HIPC(hipMemcpyAsync(&wi, tauAi.as<int>() + worst, 4, hipMemcpyDeviceToHost, s));
            HIPC(hipStreamSynchronize(s));
            std::fprintf(stderr, "[mflat trace] ivf: most survivors at batch query %d, bound (%g, %d)\n", worst,
                         (double)wk, wi);
            std::sort(perq.begin(), perq.end());
            std::fprintf(stderr,
                         "[mflat trace] ivf: full pass stored %.1f survivors per query (%.1f spilled; median %lld, "
                         "p99 %lld, max %lld), k %d\n",
                         (double)tot / mb, (double)spilt / mb, (long long)perq[(size_t)mb / 2],
                         (long long)perq[(size_t)mb * 99 / 100], (long long)perq[(size_t)mb - 1], k);
        }
        {
            SelectParams sp = selectParams(mb, nprobe + 1, cb, k);
            sp.out_ids = posIds; sp.out_vals = oVals;
            sp.tau_k_key = tauKk.as<float>(); sp.tau_k_id = tauKi.as<int>();
            sp.status = status.as<int>();
            // the bound is the k-th of the nearest cell: survivors ~ a few k
            // (all rows when nprobe = 1)
            sp.expect = nprobe > 1 ? 4 * k : std::min(cb, maxCell);
            launch_select(sp, s);
        }
        std::vector<int> st((size_t)mb);
        HIPC(hipMemcpyAsync(st.data(), status.p, (size_t)mb * 4, hipMemcpyDeviceToHost, s));
        HIPC(hipStreamSynchronize(s));
        std::vector<int> over;
        for (int i = 0; i < mb; ++i)
            if (st[(size_t)i] & 1) over.push_back(i);
        if (!over.empty()) {
            // retries: bound = k-th of the stored survivors, whole-cell regions
            const int cr = capR();
            const size_t perQ = (size_t)nprobe * cr * sizeof(uint2);
            const int chunk = (int)std::max<size_t>(1, std::min<size_t>(over.size(), kCandBudget / perQ));
            if (trace)
                std::fprintf(stderr, "[mflat trace] ivf: %d of %d queries overflowed (cap %d), retried with cap %d\n",
                             (int)over.size(), mb, cb, cr);
            for (size_t o = 0; o < over.size(); o += (size_t)chunk) {
                const int nf = (int)std::min<size_t>((size_t)chunk, over.size() - o);
                const int nfPad = (int)roundUp(nf, kBN);
                cIdx.ensure((size_t)nf * 4);
                cQ.ensure((size_t)nfPad * dpad * esize); cQn.ensure((size_t)nfPad * 4);
                cTk.ensure((size_t)nf * 4); cTi.ensure((size_t)nf * 4);
                cProbe.ensure((size_t)nf * nprobe * 4); cPos.ensure((size_t)nf * nprobe * 4);
                HIPC(hipMemcpyAsync(cIdx.p, over.data() + o, (size_t)nf * 4, hipMemcpyHostToDevice, s));
                QueryRefs cr_{cQ.p, cQn.as<float>(), nullptr, nullptr};
                if (pq()) {   // the compact batch's lookup tables and coarse terms
                    const int tab = pqM * kPqKsub;
                    cLut.ensure((size_t)nf * tab * sizeof(float));
                    cBase.ensure((size_t)nf * nprobe * sizeof(float));
                    launch_gather_rows(lut.p, cIdx.as<int>(), nf, tab * (int)sizeof(float), cLut.p, nf, s);
                    launch_gather_i32(base.as<int>(), cIdx.as<int>(), nf, nprobe, cBase.as<int>(), s);
                    cr_.lut = cLut.as<float>();
                    cr_.base = cBase.as<float>();
                } else {
                    launch_gather_rows(Q, cIdx.as<int>(), nf, dpad * esize, cQ.p, nfPad, s);
                    launch_gather_f32(qn, cIdx.as<int>(), nf, cQn.as<float>(), s);
                }
                launch_gather_f32(tauKk.as<float>(), cIdx.as<int>(), nf, cTk.as<float>(), s);
                launch_gather_i32(tauKi.as<int>(), cIdx.as<int>(), nf, 1, cTi.as<int>(), s);
                launch_gather_i32(probe.as<int>(), cIdx.as<int>(), nf, nprobe, cProbe.as<int>(), s);
                launch_gather_i32(pos.as<int>(), cIdx.as<int>(), nf, nprobe, cPos.as<int>(), s);
                if ((int64_t)nf * nprobe <= kHostTableMax) {   // few entries: the table on the host
                    hProbe.resize((size_t)nf * nprobe);
                    HIPC(hipMemcpyAsync(hProbe.data(), cProbe.p, hProbe.size() * sizeof(int), hipMemcpyDeviceToHost,
                                        s));
                    HIPC(hipStreamSynchronize(s));
                    wt.buildHost(hProbe.data(), nf, nprobe, nlist, hCellOrder.data(), narrowMax(), s);
                } else {
                    wt.build(cProbe.as<int>(), nf, nprobe, nprobe, nlist, dCellOrder.as<int>(), narrowMax(), s);
                }
                scanPass(kPassFull, nf, nprobe, nprobe, nprobe, cr, cr_, cTk.as<float>(), cTi.as<int>(), cPos.as<int>(),
                         s);
                SelectParams sp = selectParams(nf, nprobe, cr, k);
                sp.expect = 4 * k;
                sp.qmap = cIdx.as<int>();
                sp.out_ids = posIds; sp.out_vals = oVals;
                launch_select(sp, s);
                HIPC(hipStreamSynchronize(s));
            }
        }
        if (oIds)
            launch_ivf_finalize(oIds, mb, k, pos.as<int>(), probe.as<int>(), nprobe, dCellStart.as<int>(),
                                dRid.as<int>(), s);
    }

    int searchDev(const float* dq, int m, int k, int nprobe, int rerank, int32_t* ids, float* vals, hipStream_t s) {
        if (!devOk) throw NotReady("no usable HIP device: IVF search needs a gfx950 GPU");
        if (!built) throw NotReady("IVF index is not built");
        if (m <= 0) return 0;
        if (k < 1) k = 1;
        if (k > kMaxK) {
            if (!warnedK) {
                MFLAT_LOG_WARN("k=%d clamped to MFLAT_MAX_K=%d", k, kMaxK);
                warnedK = true;
            }
            k = kMaxK;
        }
        // reference src/IvfIndex.mm:766-767, src/IvfPqIndex.mm:557-559
        if (nprobe < 1) nprobe = 1;
        if (nprobe > nlist) nprobe = nlist;
        if (nprobe > kMaxProbe) throw BadArg("IVF search: nprobe above 1024 is not supported");
        // PQ rerank (src/IvfPqIndex.mm:583-585): a PQ shortlist of kRun rows,
        // re-ranked by exact distance, when rerank > k and the rows were kept
        const bool doRerank = pq() && rerank > k && fullStored;
        const int kRun = doRerank ? (int)std::min<int64_t>({(int64_t)rerank, n, (int64_t)kMaxK}) : k;
        setDevice();
        // batch the queries so the candidate regions stay bounded
        size_t perQuery = std::max<size_t>(nprobe > 1 ? (size_t)std::min(nprobe, kBoundRanks) * capA(kRun) : 0,
                                           (size_t)(nprobe + 1) * capB(kRun, nprobe)) *
                          sizeof(uint2);
        if (pq()) perQuery += (size_t)pqM * kPqKsub * sizeof(float) + (size_t)nprobe * sizeof(float) +
                              (size_t)kRun * (sizeof(uint2) + sizeof(int));
        int64_t mb = std::max<int64_t>(1, (int64_t)(kCandBudget / perQuery));
        if (mb >= kBN) mb = mb / kBN * kBN;
        mb = std::min<int64_t>(mb, m);
        for (int64_t b0 = 0; b0 < m; b0 += mb) {
            const int nb = (int)std::min<int64_t>(mb, m - b0);
            const int64_t nPad = roundUp(nb, kBN);
            const float* src = dq + b0 * dim;
            int32_t* bIds = ids ? ids + b0 * k : nullptr;
            float* bVals = vals ? vals + b0 * k : nullptr;
            probe.ensure((size_t)nb * nprobe * sizeof(int));
            const float* probeQ = src;
            if (metric == Metric::Cosine) {
                // normalised queries (reference src/IvfIndex.mm:773-780) for the
                // probe (row-major, dim columns) and the fine scan
                qrm.ensure((size_t)nb * dim * sizeof(float));
                launch_pack_rows(src, nb, dim, qrm.as<float>(), nb, dim, s);
                launch_normalize_rows(qrm.as<float>(), nb, dim, s);
                probeQ = qrm.as<float>();
            }
            coarse->searchDevice(probeQ, nb, nprobe, probe.as<int32_t>(), nullptr, s);
            if (pq()) {
                lut.ensure((size_t)nb * pqM * kPqKsub * sizeof(float));
                base.ensure((size_t)nb * nprobe * sizeof(float));
                launch_pq_lut(probeQ, nb, dim, dPqc.as<float>(), dNorms.as<float>(), pqM, dsub, lut.as<float>(), s);
                launch_pq_base(probeQ, nb, dim, dCentD.as<float>(), probe.as<int>(), nprobe, base.as<float>(), s);
                if (!doRerank) {
                    searchBatch(nb, k, nprobe, bIds, bVals, s);
                    continue;
                }
                shortIds.ensure((size_t)nb * kRun * sizeof(int));
                searchBatch(nb, kRun, nprobe, shortIds.as<int32_t>(), nullptr, s);
                // exact keys of the shortlist, ties in shortlist order
                // (src/IvfPqIndex.mm:600-625)
                rrCand.ensure((size_t)nb * kRun * sizeof(uint2));
                rrCnt.ensure((size_t)nb * sizeof(int));
                rrSel.ensure((size_t)nb * k * sizeof(int));
                const int rm = metric == Metric::L2 ? 0 : 1;
                launch_rerank_keys(probeQ, nb, dim, dFull.as<float>(), shortIds.as<int>(), kRun, rm,
                                   rrCand.as<uint2>(), rrCnt.as<int>(), s);
                SelectParams sp;
                std::memset(&sp, 0, sizeof sp);
                sp.cand = rrCand.as<uint2>(); sp.cnt = rrCnt.as<int>();
                sp.nsplit = 1; sp.cap = kRun; sp.nq = nb; sp.k = k; sp.j = k; sp.j2 = k;
                sp.metric = rm;
                sp.out_ids = rrSel.as<int32_t>(); sp.out_vals = bVals; sp.out_stride = k;
                sp.expect = kRun;
                launch_select(sp, s);
                if (bIds) launch_rerank_ids(shortIds.as<int>(), kRun, rrSel.as<int>(), nb, k, bIds, s);
                continue;
            }
            qbuf.ensure((size_t)nPad * dpad * sizeof(float));
            qnorm.ensure((size_t)nPad * sizeof(float));
            launch_pack_rows(src, nb, dim, qbuf.as<float>(), nPad, dpad, s);
            if (metric == Metric::Cosine) launch_normalize_rows(qbuf.as<float>(), nb, dpad, s);
            const void* qs = qbuf.p;
            if (storage != kF32) {
                qh.ensure((size_t)nPad * dpad * esize);
                launch_round_rows(qbuf.as<float>(), nPad * dpad, storage, qh.p, s);
                qs = qh.p;
            }
            if (metric == Metric::L2) launch_row_norms(qs, nb, dpad, storage, qnorm.as<float>(), s);
            searchBatch(nb, k, nprobe, bIds, bVals, s);
        }
        HIPC(hipStreamSynchronize(s));
        return k;
    }
};

IvfIndex::IvfIndex(int dim, Metric metric, int nlist, Storage storage, int pqM) : d_(new Impl) {
    if (dim <= 0 || nlist <= 0) throw BadArg("IVF index: dim and nlist must be >= 1");
    if (storage != kF32 && storage != kF16 && storage != kBF16) throw BadArg("unknown storage type");
    if (pqM < 0 || (pqM > 0 && (dim % pqM != 0 || pqM > kMaxSubquantizers)))
        throw BadArg("IVF-PQ index: m must divide dim and be at most 128");
    if (pqM > 0 && metric == Metric::InnerProduct) throw BadArg("IVF-PQ index: inner product is not supported");
    d_->pqM = pqM;
    d_->dsub = pqM > 0 ? dim / pqM : 0;
    d_->dim = dim;
    d_->dpad = (int)roundUp(dim, kBK);
    d_->metric = metric;
    d_->storage = storage;
    d_->esize = elem_bytes(storage);
    d_->nlistReq = nlist;
    auto knob = [](const char* name) {
        const char* v = std::getenv(name);
        return v ? std::atoi(v) : 0;
    };
    d_->tilesKnob = knob("MFLAT_IVF_TILES");
    d_->capBKnob = knob("MFLAT_IVF_CAP_B");
    d_->trace = knob("MFLAT_TRACE") != 0;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        MFLAT_LOG_INFO("no HIP device - IVF index unavailable");
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
    d_->devOk = true;
}

IvfIndex::~IvfIndex() {
    if (!d_) return;
    if (d_->device >= 0) (void)hipSetDevice(d_->device);
    if (d_->stream) (void)hipStreamSynchronize(d_->stream);
    d_->coarse.reset();
    d_->wt.release();
    if (d_->stream) (void)hipStreamDestroy(d_->stream);
}

bool IvfIndex::ready() const { return d_->built; }
bool IvfIndex::deviceOk() const { return d_->devOk; }
int IvfIndex::size() const { return (int)d_->n; }
int IvfIndex::dim() const { return d_->dim; }
int IvfIndex::nlist() const { return d_->built ? d_->nlist : d_->nlistReq; }
Metric IvfIndex::metric() const { return d_->metric; }
Storage IvfIndex::storage() const { return static_cast<Storage>(d_->storage); }

void IvfIndex::build(const float* rows, int n) { d_->buildFrom(rows, n, hipMemcpyHostToDevice, d_->stream); }

void IvfIndex::buildDevice(const float* rows, int n, hipStream_t s) {
    d_->buildFrom(rows, n, hipMemcpyDeviceToDevice, s ? s : d_->stream);
}

void IvfIndex::setRerank(bool enable) { d_->rerankReq = enable; }
int IvfIndex::subquantizers() const { return d_->pqM; }
const std::vector<float>& IvfIndex::pqCentroids() const { return d_->hPqc; }

std::vector<uint8_t> IvfIndex::codes() const {
    Impl& I = *d_;
    std::vector<uint8_t> out;
    if (!I.built || !I.pq()) return out;
    I.setDevice();
    out.resize((size_t)I.n * I.pqM);
    HIPC(hipMemcpy(out.data(), I.dCodes.p, out.size(), hipMemcpyDeviceToHost));
    return out;
}

int IvfIndex::search(const float* q, int m, int k, int nprobe, int32_t* ids, float* dists, int rerank) {
    Impl& I = *d_;
    if (!I.devOk) throw NotReady("no usable HIP device: IVF search needs a gfx950 GPU");
    if (!I.built) throw NotReady("IVF index is not built");
    if (m <= 0) return 0;
    const int kk = std::min(std::max(k, 1), kMaxK);
    I.setDevice();
    hipStream_t s = I.stream;
    I.qin.ensure((size_t)m * I.dim * sizeof(float));
    I.outIds.ensure((size_t)m * kk * sizeof(int32_t));
    I.outVals.ensure((size_t)m * kk * sizeof(float));
    HIPC(hipMemcpyAsync(I.qin.p, q, (size_t)m * I.dim * sizeof(float), hipMemcpyHostToDevice, s));
    const int used = I.searchDev(I.qin.as<float>(), m, k, nprobe, rerank, ids ? I.outIds.as<int32_t>() : nullptr,
                                 dists ? I.outVals.as<float>() : nullptr, s);
    if (ids) HIPC(hipMemcpyAsync(ids, I.outIds.p, (size_t)m * used * sizeof(int32_t), hipMemcpyDeviceToHost, s));
    if (dists) HIPC(hipMemcpyAsync(dists, I.outVals.p, (size_t)m * used * sizeof(float), hipMemcpyDeviceToHost, s));
    HIPC(hipStreamSynchronize(s));
    return used;
}

int IvfIndex::searchDevice(const float* q, int m, int k, int nprobe, int32_t* ids, float* dists, hipStream_t s,
                           int rerank) {
    return d_->searchDev(q, m, k, nprobe, rerank, ids, dists, s ? s : d_->stream);
}

void IvfIndex::probe(const float* q, int m, int nprobe, int32_t* cells) {
    Impl& I = *d_;
    if (!I.devOk) throw NotReady("no usable HIP device: IVF probe needs a gfx950 GPU");
    if (!I.built) throw NotReady("IVF index is not built");
    if (m <= 0) return;
    if (nprobe < 1) nprobe = 1;
    if (nprobe > I.nlist) nprobe = I.nlist;
    if (nprobe > kMaxProbe) throw BadArg("IVF probe: nprobe above 1024 is not supported");
    I.setDevice();
    hipStream_t s = I.stream;
    I.qin.ensure((size_t)m * I.dim * sizeof(float));
    I.probe.ensure((size_t)m * nprobe * sizeof(int));
    HIPC(hipMemcpyAsync(I.qin.p, q, (size_t)m * I.dim * sizeof(float), hipMemcpyHostToDevice, s));
    const float* pq = I.qin.as<float>();
    if (I.metric == Metric::Cosine) {
        I.qrm.ensure((size_t)m * I.dim * sizeof(float));
        launch_pack_rows(pq, m, I.dim, I.qrm.as<float>(), m, I.dim, s);
        launch_normalize_rows(I.qrm.as<float>(), m, I.dim, s);
        pq = I.qrm.as<float>();
    }
    I.coarse->searchDevice(pq, m, nprobe, I.probe.as<int32_t>(), nullptr, s);
    HIPC(hipMemcpyAsync(cells, I.probe.p, (size_t)m * nprobe * sizeof(int), hipMemcpyDeviceToHost, s));
    HIPC(hipStreamSynchronize(s));
}

const std::vector<float>& IvfIndex::centroids() const { return d_->hCent; }
const std::vector<int>& IvfIndex::cellStart() const { return d_->hStart; }
const std::vector<int>& IvfIndex::reorderedIds() const { return d_->hRid; }

}  // namespace mflat_amd
