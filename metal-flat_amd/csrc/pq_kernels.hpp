// SPDX-License-Identifier: Apache-2.0
// pq_kernels.hpp -- device side of the IVF-PQ index: residual product
// quantization tables and the ADC (asymmetric distance) fine scan.
//
// Residual PQ (reference src/PqTrainer.h, src/IvfIndex.mm's ivfpq_adc): a row x
// of cell c is stored as M one-byte codes, code m the nearest of 256
// sub-centroids pqc[m][.] of the residual's m-th sub-vector (dsub = dim / M
// columns). Its ADC distance to a query q is
//   dist = ||q - c||^2 + sum_m (lut[m][code_m] + T[c][m][code_m])
//   lut[m][j]  = ||pqc[m][j]||^2 - 2 q_m . pqc[m][j]     (per query)
//   T[c][m][j] = 2 c_m . pqc[m][j]                       (per cell)
// with every dot, square norm and ||q - c||^2 an fp32 sum in ascending column
// order and no fused multiply-add (the reference's scalar C++ loops), and the
// sum over m in ascending m, each term's two table entries added first.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace mflat_amd {

constexpr int kPqKsub = 256;   // sub-centroids per sub-quantizer (8-bit codes)

// assign[rid[slot]] = c for slot in [cellStart[c], cellStart[c + 1])
void launch_cell_assign(const int* cellStart, const int* rid, int nlist, int* assign, hipStream_t s);
// r[i] = x[i] - cent[assign[i]] (row-major, dim columns)
void launch_residuals(const float* x, const float* cent, const int* assign, int64_t n, int dim, float* r,
                      hipStream_t s);
// sub[i][d] = r[i][off + d], d < dsub
void launch_subspace(const float* r, int64_t n, int dim, int off, int dsub, float* sub, hipStream_t s);
// norms[m][j] = ||pqc[m][j]||^2 (pqc: M x 256 x dsub)
void launch_pq_norms(const float* pqc, int M, int dsub, float* norms, hipStream_t s);
// T[c][m][j] = 2 cent[c]_m . pqc[m][j] for c < nlist
void launch_pq_cell_table(const float* cent, int nlist, int dim, const float* pqc, int M, int dsub, float* T,
                          hipStream_t s);
// codes[slot][mm] = subAssign[rid[slot]] for slot < n (cell order)
void launch_pq_codes(const int* subAssign, const int* rid, int64_t n, int M, int mm, uint8_t* codes, hipStream_t s);

// lut[i][m][j] for queries i < nq (row-major, dim columns)
void launch_pq_lut(const float* q, int nq, int dim, const float* pqc, const float* norms, int M, int dsub, float* lut,
                   hipStream_t s);
// base[e] = ||q_i - cent[probe[e]]||^2, e = i * np + r (+inf for probe -1)
void launch_pq_base(const float* q, int nq, int dim, const float* cent, const int* probe, int np, float* base,
                    hipStream_t s);

// The ADC fine scan over work items of one cell and up to tq queries (the IVF
// work tables), filter and survivor regions as the MFMA IVF scan: a row
// survives when (dist, scan position) <= the query's bound, lexicographically.
struct AdcParams {
    const uint8_t* codes;     // n x M, cell order (row slot of the CSR)
    const int* cellStart;     // CSR starts (nlist + 1)
    const float* lut;         // nq x M x 256
    const float* T;           // nlist x M x 256
    const float* base;        // per entry: ||q - c||^2
    const int4* work;         // (cell, first entry, entries <= tq, 0)
    const int* nwork;         // device: valid work items
    const int* ent;           // entries e = q * nprobe + rank, grouped by cell
    const int* pos;           // per entry: scan position of the cell's first row
    const float* tau_key;     // per query bound (key, id)
    const int* tau_id;
    uint2* cand;              // regions (q * nreg + rank) x cap
    int* cnt;
    int cap;
    int M;
    int nprobe;
    int nreg;
    int spill;                // region nprobe of each query takes what overflows the others
    int rowCap;               // > 0: only the first rowCap rows of each cell
    int tq;                   // queries per work item (<= 16)
};
// LDS of one work item: tq combined tables of M x 256 floats
int adc_tile_queries(int M);
void launch_adc_scan(const AdcParams& p, int pass, int grid, hipStream_t s);

// Rerank: keys of the shortlist of each query (nq x kRun ids, -1 padding at
// the end): L2 -> ||q - full[id]||^2, otherwise -(q . full[id]); region i of
// query q holds (key, shortlist index), cnt[q] = valid entries.
void launch_rerank_keys(const float* q, int nq, int dim, const float* full, const int* shortIds, int kRun, int metric,
                        uint2* cand, int* cnt, hipStream_t s);
// ids[i][j] = shortIds[i][sel[i][j]] (sel -1 -> -1), j < k
void launch_rerank_ids(const int* shortIds, int kRun, const int* sel, int nq, int k, int* ids, hipStream_t s);

}  // namespace mflat_amd
