// SPDX-License-Identifier: Apache-2.0
// pq_kernels.hip -- device side of the IVF-PQ index (pq_kernels.hpp).
//
// The PQ tables and the coarse term restate the reference's scalar fp32 loops
// (src/PqTrainer.h:84-116, src/Distance.h:26-37,86-88, src/IvfPqIndex.mm:500-520)
// with contraction off, so each value is the same float the reference's CPU
// computes: ascending-order sums, a separate multiply and add per term.
//
// adc_scan: one workgroup per work item (a cell and up to tq of the queries
// probing it). It first adds the cell's cross table to each query's lookup
// table in LDS (one combined M x 256 table per query: the two entries of a
// term are added before the term joins the sum, as the reference does), then
// each thread takes rows of the cell -- one coalesced load of the row's M
// code bytes -- and sums M table lookups per query: the scan is bound by LDS
// gathers (M per candidate), not by HBM (M bytes per row per work item).
#include "pq_kernels.hpp"

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
    return (int)(g < 1 ? 1 : g > cap ? cap : g);
}

// fp32 restatements, no fused multiply-add (reference src/Distance.h:26-37);
// 16-byte aligned operands of a length divisible by 4 load as float4, the
// terms still accumulate one at a time in ascending order.
__device__ __forceinline__ bool vec4_ok(const float* a, const float* b, int n) {
    return ((((uintptr_t)a | (uintptr_t)b) & 15u) == 0) && (n & 3) == 0;
}
__device__ __forceinline__ float dot_seq(const float* a, const float* b, int n) {
#pragma clang fp contract(off)
    float acc = 0.0f;
    if (vec4_ok(a, b, n)) {
        const float4* a4 = (const float4*)a;
        const float4* b4 = (const float4*)b;
        for (int i = 0; i < n / 4; ++i) {
            const float4 x = a4[i], y = b4[i];
            acc += x.x * y.x;
            acc += x.y * y.y;
            acc += x.z * y.z;
            acc += x.w * y.w;
        }
        return acc;
    }
    for (int i = 0; i < n; ++i) acc += a[i] * b[i];
    return acc;
}
__device__ __forceinline__ float sql2_seq(const float* a, const float* b, int n) {
#pragma clang fp contract(off)
    float acc = 0.0f;
    if (vec4_ok(a, b, n)) {
        const float4* a4 = (const float4*)a;
        const float4* b4 = (const float4*)b;
        for (int i = 0; i < n / 4; ++i) {
            const float4 x = a4[i], y = b4[i];
            const float e0 = x.x - y.x, e1 = x.y - y.y, e2 = x.z - y.z, e3 = x.w - y.w;
            acc += e0 * e0;
            acc += e1 * e1;
            acc += e2 * e2;
            acc += e3 * e3;
        }
        return acc;
    }
    for (int i = 0; i < n; ++i) {
        const float e = a[i] - b[i];
        acc += e * e;
    }
    return acc;
}

__global__ void cell_assign_kernel(const int* __restrict__ cellStart, const int* __restrict__ rid, int nlist,
                                   int* __restrict__ assign) {
    const int c = blockIdx.x;
    if (c >= nlist) return;
    for (int s = cellStart[c] + (int)threadIdx.x; s < cellStart[c + 1]; s += blockDim.x) assign[rid[s]] = c;
}

__global__ void residuals_kernel(const float* __restrict__ x, const float* __restrict__ cent,
                                 const int* __restrict__ assign, int64_t n, int dim, float* __restrict__ r) {
#pragma clang fp contract(off)
    const int64_t total = n * dim;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = e / dim;
        const int d = (int)(e - i * dim);
        r[e] = x[e] - cent[(int64_t)assign[i] * dim + d];
    }
}

__global__ void subspace_kernel(const float* __restrict__ r, int64_t n, int dim, int off, int dsub,
                                float* __restrict__ sub) {
    const int64_t total = n * dsub;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = e / dsub;
        sub[e] = r[i * dim + off + (e - i * dsub)];
    }
}

__global__ void pq_norms_kernel(const float* __restrict__ pqc, int M, int dsub, float* __restrict__ norms) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= M * kPqKsub) return;
    const float* c = pqc + (int64_t)e * dsub;
    norms[e] = dot_seq(c, c, dsub);
}

// T[c][m][j] = 2 * dot(cent_c[m], pqc[m][j])
__global__ void pq_cell_table_kernel(const float* __restrict__ cent, int nlist, int dim,
                                     const float* __restrict__ pqc, int M, int dsub, float* __restrict__ T) {
#pragma clang fp contract(off)
    const int tab = M * kPqKsub;
    const int64_t total = (int64_t)nlist * tab;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(e / tab);
        const int o = (int)(e - (int64_t)c * tab);
        const int m = o / kPqKsub;
        T[e] = 2.0f * dot_seq(cent + (int64_t)c * dim + m * dsub, pqc + (int64_t)o * dsub, dsub);
    }
}

__global__ void pq_codes_kernel(const int* __restrict__ subAssign, const int* __restrict__ rid, int64_t n, int M,
                                int mm, uint8_t* __restrict__ codes) {
    for (int64_t s = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; s < n; s += (int64_t)gridDim.x * blockDim.x)
        codes[s * M + mm] = (uint8_t)subAssign[rid[s]];
}

// lut[i][m][j] = norms[m][j] - 2 * dot(q_i[m], pqc[m][j]) (src/Distance.h:86-88).
// One block per (16 queries, sub-space m): thread j keeps sub-centroid j in
// registers and writes entry j of the 16 queries' tables (coalesced rows); the
// queries' sub-vectors sit in LDS. dsub <= 32 here; larger sub-spaces take
// pq_lut_wide_kernel.
constexpr int kLutQ = 16;
constexpr int kLutMaxDsub = 32;
__global__ void __launch_bounds__(kPqKsub) pq_lut_kernel(const float* __restrict__ q, int nq, int dim,
                                                          const float* __restrict__ pqc,
                                                          const float* __restrict__ norms, int M, int dsub,
                                                          float* __restrict__ lut) {
#pragma clang fp contract(off)
    __shared__ float sq[kLutQ * kLutMaxDsub];
    const int m = blockIdx.y;
    const int i0 = blockIdx.x * kLutQ;
    const int j = threadIdx.x;
    for (int e = j; e < kLutQ * dsub; e += kPqKsub) {
        const int t = e / dsub, c = e - t * dsub;
        sq[e] = i0 + t < nq ? q[(int64_t)(i0 + t) * dim + m * dsub + c] : 0.0f;
    }
    float pc[kLutMaxDsub];
    const float* cj = pqc + ((int64_t)m * kPqKsub + j) * dsub;
#pragma unroll
    for (int c = 0; c < kLutMaxDsub; ++c) pc[c] = c < dsub ? cj[c] : 0.0f;
    const float nj = norms[m * kPqKsub + j];
    __syncthreads();
    const int64_t tab = (int64_t)M * kPqKsub;
    for (int t = 0; t < kLutQ && i0 + t < nq; ++t) {
        const float* qs = sq + t * dsub;
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < kLutMaxDsub; ++c)
            if (c < dsub) acc += qs[c] * pc[c];
        lut[(int64_t)(i0 + t) * tab + m * kPqKsub + j] = nj - 2.0f * acc;
    }
}

__global__ void pq_lut_wide_kernel(const float* __restrict__ q, int nq, int dim, const float* __restrict__ pqc,
                                   const float* __restrict__ norms, int M, int dsub, float* __restrict__ lut) {
#pragma clang fp contract(off)
    const int tab = M * kPqKsub;
    const int64_t total = (int64_t)nq * tab;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = e / tab;
        const int o = (int)(e - i * tab);
        const int m = o / kPqKsub;
        const float d = dot_seq(q + i * dim + m * dsub, pqc + (int64_t)o * dsub, dsub);
        lut[e] = norms[o] - 2.0f * d;
    }
}

__global__ void pq_base_kernel(const float* __restrict__ q, int nq, int dim, const float* __restrict__ cent,
                               const int* __restrict__ probe, int np, float* __restrict__ base) {
    const int64_t total = (int64_t)nq * np;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int c = probe[e];
        base[e] = c >= 0 ? sql2_seq(q + (e / np) * dim, cent + (int64_t)c * dim, dim) : INFINITY;
    }
}

constexpr int kAdcMaxTq = 16;
constexpr int kAdcBlock = 512;   // threads of an ADC work item (M x 64 float4 of a table: a multiple of it for M >= 8)

int adc_tile_queries(int M) {
    const int t = (64 * 1024) / (M * kPqKsub * (int)sizeof(float));
    return t < 1 ? 1 : t > kAdcMaxTq ? kAdcMaxTq : t;
}

// One lookup of a combined table: byte offset a of the code's entry plus a
// compile-time offset (query tile slot and sub-space), which the compiler folds
// into the ds_read immediate.
__device__ __forceinline__ float lds_at(const float* base, uint32_t a, int off) {
    return *(const float*)((const char*)base + a + off);
}

// MV: M known at compile time (codes loaded with vector loads, TQ = 64 / MV
// query slots unrolled: the M byte offsets of a row are computed once and
// serve every query), 0: any M (runtime loops)
template <int PASS, int MV>
__global__ void __launch_bounds__(kAdcBlock) adc_scan_kernel(AdcParams p) {
    extern __shared__ float sL[];   // [tq][M][256]
    __shared__ int sQi[kAdcMaxTq], sReg[kAdcMaxTq], sPos[kAdcMaxTq], sCnt[kAdcMaxTq], sTi[kAdcMaxTq];
    __shared__ float sBase[kAdcMaxTq], sTk[kAdcMaxTq];
    if ((int)blockIdx.x >= *p.nwork) return;
    const int4 wk = p.work[blockIdx.x];
    const int c = wk.x, ne = wk.z;
    const int tid = threadIdx.x;
    const int M = MV > 0 ? MV : p.M;
    if (tid < kAdcMaxTq) {
        const int e = tid < ne ? p.ent[wk.y + tid] : -1;
        const int q = e >= 0 ? e / p.nprobe : -1;
        sQi[tid] = q;
        sReg[tid] = e >= 0 ? q * p.nreg + (e - q * p.nprobe) : -1;
        sPos[tid] = e >= 0 ? p.pos[e] : 0;
        sBase[tid] = e >= 0 ? p.base[e] : 0.0f;
        sTk[tid] = e >= 0 ? p.tau_key[q] : 0.0f;
        sTi[tid] = e >= 0 ? p.tau_id[q] : -1;
        sCnt[tid] = 0;
    }
    __syncthreads();
    // combined tables: lut of the query + the cell's cross table (tab floats
    // each, a multiple of 4: float4 copies)
    const int tab = M * kPqKsub;
    const int tab4 = tab / 4;
    const float4* Tc = (const float4*)(p.T + (int64_t)c * tab);
    float4* sL4 = (float4*)sL;
    auto add4 = [](float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); };
    if constexpr (MV > 0) {
        // every load of the thread's share in flight at once: PER float4 of
        // the cross table, reused by the TQ queries (empty slots copy slot 0's)
        constexpr int TQ = 64 / MV, PER = MV * 64 / kAdcBlock;
        static_assert(PER >= 1 && PER * kAdcBlock == MV * 64, "table share per thread");
        float4 tv[PER], lv[TQ][PER];
#pragma unroll
        for (int j = 0; j < PER; ++j) tv[j] = Tc[tid + j * kAdcBlock];
#pragma unroll
        for (int t = 0; t < TQ; ++t) {
            const float4* lq = (const float4*)(p.lut + (int64_t)sQi[t < ne ? t : 0] * tab);
#pragma unroll
            for (int j = 0; j < PER; ++j) lv[t][j] = lq[tid + j * kAdcBlock];
        }
#pragma unroll
        for (int t = 0; t < TQ; ++t)
#pragma unroll
            for (int j = 0; j < PER; ++j) sL4[t * tab4 + tid + j * kAdcBlock] = add4(lv[t][j], tv[j]);
    } else {
        for (int t = 0; t < ne; ++t) {
            const float4* lq = (const float4*)(p.lut + (int64_t)sQi[t] * tab);
            for (int o = tid; o < tab4; o += kAdcBlock) sL4[t * tab4 + o] = add4(lq[o], Tc[o]);
        }
    }
    __syncthreads();

    const int beg = p.cellStart[c];
    int rows = p.cellStart[c + 1] - beg;
    if (p.rowCap > 0 && rows > p.rowCap) rows = p.rowCap;
    auto emit = [&](int t, float key, int id) {
        const uint2 v = make_uint2(__float_as_uint(key), (unsigned)id);
        const int slot = atomicAdd(&sCnt[t], 1);
        if (slot < p.cap) {
            p.cand[(int64_t)sReg[t] * p.cap + slot] = v;
        } else if (p.spill) {
            const int64_t sr = (int64_t)sQi[t] * p.nreg + p.nprobe;
            const int sp = atomicAdd(&p.cnt[sr], 1);
            if (sp < p.cap) p.cand[sr * p.cap + sp] = v;
        }
    };
    if constexpr (MV > 0) {
        constexpr int TQ = 64 / MV;   // == adc_tile_queries(MV); slots >= ne are computed, never emitted
        constexpr int NW = MV / 4;    // code words per row
        // the next row's codes load while the current row is summed
        auto load_codes = [&](int r, uint32_t* cw) {
            const uint8_t* src = p.codes + (int64_t)(beg + r) * MV;
            if constexpr (NW == 2) {
                const uint2 v = *(const uint2*)src;
                cw[0] = v.x; cw[1] = v.y;
            } else {
#pragma unroll
                for (int w = 0; w < NW; w += 4) {
                    const uint4 v = *(const uint4*)(src + w * 4);
                    cw[w] = v.x; cw[w + 1] = v.y; cw[w + 2] = v.z; cw[w + 3] = v.w;
                }
            }
        };
        uint32_t nx[NW];
        if (tid < rows) load_codes(tid, nx);
        for (int r = tid; r < rows; r += kAdcBlock) {
            uint32_t cw[NW];
#pragma unroll
            for (int w = 0; w < NW; ++w) cw[w] = nx[w];
            if (r + kAdcBlock < rows) load_codes(r + kAdcBlock, nx);
            uint32_t a[MV];   // byte offset of the row's entry in table m (without m * 1 KiB)
#pragma unroll
            for (int m = 0; m < MV; ++m) a[m] = ((cw[m >> 2] >> ((m & 3) * 8)) & 255u) * 4u;
            float dist[TQ];
#pragma unroll
            for (int t = 0; t < TQ; ++t) dist[t] = sBase[t];
#pragma unroll
            for (int m = 0; m < MV; ++m) {
#pragma unroll
                for (int t = 0; t < TQ; ++t)
                    dist[t] = dist[t] + lds_at(sL, a[m], (t * MV + m) * kPqKsub * (int)sizeof(float));
            }
#pragma unroll
            for (int t = 0; t < TQ; ++t) {
                if (t >= ne) break;
                const int id = sPos[t] + r;
                if (dist[t] < sTk[t] || (dist[t] == sTk[t] && id <= sTi[t])) emit(t, dist[t], id);
            }
        }
    } else {
        for (int r = tid; r < rows; r += kAdcBlock) {
            const uint8_t* code = p.codes + (int64_t)(beg + r) * M;
            for (int t = 0; t < ne; ++t) {
                const float* L = sL + t * tab;
                float dist = sBase[t];
                for (int m = 0; m < M; ++m) dist = dist + L[m * kPqKsub + code[m]];
                const int id = sPos[t] + r;
                if (dist < sTk[t] || (dist == sTk[t] && id <= sTi[t])) emit(t, dist, id);
            }
        }
    }
    __syncthreads();
    if (tid < ne) p.cnt[sReg[tid]] = p.spill && sCnt[tid] > p.cap ? p.cap : sCnt[tid];
}

// One block per 256 (query, shortlist slot) pairs. The rows go through LDS
// in chunks of 32 columns (coalesced: 32 lanes read one row's chunk), padded
// to 33 floats a row so the summing threads -- one per pair, columns in
// ascending order across the chunks -- read distinct banks.
constexpr int kRrCols = 32;
__global__ void __launch_bounds__(256) rerank_keys_kernel(const float* __restrict__ q, int nq, int dim,
                                                          const float* __restrict__ full,
                                                          const int* __restrict__ shortIds, int kRun, int metric,
                                                          uint2* __restrict__ cand, int* __restrict__ cnt) {
#pragma clang fp contract(off)
    __shared__ float sX[256 * (kRrCols + 1)];
    __shared__ int sId[256];
    const int64_t total = (int64_t)nq * kRun;
    const int64_t e0 = (int64_t)blockIdx.x * 256;
    const int tid = threadIdx.x;
    const int64_t e = e0 + tid;
    sId[tid] = e < total ? shortIds[e] : -1;
    const int64_t i = e < total ? e / kRun : 0;
    const float* qq = q + i * dim;
    float acc = 0.0f;
    for (int c0 = 0; c0 < dim; c0 += kRrCols) {
        const int w = min(kRrCols, dim - c0);
        float qv[kRrCols];   // the query's chunk, loaded in one batch
#pragma unroll
        for (int j = 0; j < kRrCols; ++j) qv[j] = j < w ? qq[c0 + j] : 0.0f;
        __syncthreads();   // sId visible; the previous chunk consumed
#pragma unroll 8
        for (int f = tid; f < 256 * kRrCols; f += 256) {
            const int r = f / kRrCols, col = f - r * kRrCols;
            const int id = sId[r];
            sX[r * (kRrCols + 1) + col] = (id >= 0 && col < w) ? full[(int64_t)id * dim + c0 + col] : 0.0f;
        }
        __syncthreads();
        const float* x = sX + tid * (kRrCols + 1);
        if (metric == 0) {
#pragma unroll
            for (int j = 0; j < kRrCols; ++j)
                if (j < w) {
                    const float d = qv[j] - x[j];
                    acc += d * d;
                }
        } else {
#pragma unroll
            for (int j = 0; j < kRrCols; ++j)
                if (j < w) acc += qv[j] * x[j];
        }
    }
    if (e >= total || sId[tid] < 0) return;
    const int j = (int)(e - i * kRun);
    const float key = metric == 0 ? acc : -acc;
    cand[e] = make_uint2(__float_as_uint(key + 0.0f), (unsigned)j);
    if (j == kRun - 1 || shortIds[e + 1] < 0) cnt[i] = j + 1;   // padding sits at the end
}

// dim % 4 == 0: one wave per 64 (query, slot) pairs. The 64 shortlist rows
// load in 64-column blocks as float4 lanes (16 lanes a row, four rows an
// instruction), go to LDS column-major with a 65-float stride (lane i then
// reads column j of its row from bank (i + j) mod 32) and each lane sums its
// pair's columns in ascending order.
constexpr int kRrBlk = 64;
__global__ void __launch_bounds__(64) rerank_rows_kernel(const float* __restrict__ q, int nq, int dim,
                                                         const float* __restrict__ full,
                                                         const int* __restrict__ shortIds, int kRun, int metric,
                                                         uint2* __restrict__ cand, int* __restrict__ cnt) {
#pragma clang fp contract(off)
    __shared__ float sX[kRrBlk * 65];
    const int lane = threadIdx.x;
    const int64_t total = (int64_t)nq * kRun;
    const int64_t e = (int64_t)blockIdx.x * 64 + lane;
    const bool live = e < total;
    const int myId = live ? shortIds[e] : -1;
    const int64_t i = live ? e / kRun : 0;
    const float* qq = q + i * dim;
    const int quarter = lane >> 4, c4 = (lane & 15) * 4;
    float acc = 0.0f;
    for (int c0 = 0; c0 < dim; c0 += kRrBlk) {
        const int w = min(kRrBlk, dim - c0);
        float4 v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int id = __shfl(myId, 4 * u + quarter, 64);
            v[u] = (id >= 0 && c4 < w) ? *(const float4*)(full + (int64_t)id * dim + c0 + c4)
                                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        __syncthreads();   // the previous block's columns are summed
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int row = 4 * u + quarter;
            sX[(c4 + 0) * 65 + row] = v[u].x;
            sX[(c4 + 1) * 65 + row] = v[u].y;
            sX[(c4 + 2) * 65 + row] = v[u].z;
            sX[(c4 + 3) * 65 + row] = v[u].w;
        }
        __syncthreads();
        if (metric == 0) {
#pragma unroll 16
            for (int j = 0; j < w; ++j) {
                const float d = qq[c0 + j] - sX[j * 65 + lane];
                acc += d * d;
            }
        } else {
#pragma unroll 16
            for (int j = 0; j < w; ++j) acc += qq[c0 + j] * sX[j * 65 + lane];
        }
    }
    if (!live || myId < 0) return;
    const int j = (int)(e - i * kRun);
    const float key = metric == 0 ? acc : -acc;
    cand[e] = make_uint2(__float_as_uint(key + 0.0f), (unsigned)j);
    if (j == kRun - 1 || shortIds[e + 1] < 0) cnt[i] = j + 1;   // padding sits at the end
}

__global__ void count_zero_kernel(int* __restrict__ cnt, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) cnt[i] = 0;
}

__global__ void rerank_ids_kernel(const int* __restrict__ shortIds, int kRun, const int* __restrict__ sel, int nq,
                                  int k, int* __restrict__ ids) {
    const int64_t total = (int64_t)nq * k;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = e / k;
        const int s = sel[e];
        ids[e] = s >= 0 ? shortIds[i * kRun + s] : -1;
    }
}

void launch_cell_assign(const int* cellStart, const int* rid, int nlist, int* assign, hipStream_t s) {
    if (nlist <= 0) return;
    cell_assign_kernel<<<nlist, 256, 0, s>>>(cellStart, rid, nlist, assign);
    check(hipGetLastError(), "cell_assign");
}

void launch_residuals(const float* x, const float* cent, const int* assign, int64_t n, int dim, float* r,
                      hipStream_t s) {
    if (n <= 0) return;
    residuals_kernel<<<grid_of(n * dim, 256), 256, 0, s>>>(x, cent, assign, n, dim, r);
    check(hipGetLastError(), "residuals");
}

void launch_subspace(const float* r, int64_t n, int dim, int off, int dsub, float* sub, hipStream_t s) {
    if (n <= 0) return;
    subspace_kernel<<<grid_of(n * dsub, 256), 256, 0, s>>>(r, n, dim, off, dsub, sub);
    check(hipGetLastError(), "subspace");
}

void launch_pq_norms(const float* pqc, int M, int dsub, float* norms, hipStream_t s) {
    pq_norms_kernel<<<(M * kPqKsub + 255) / 256, 256, 0, s>>>(pqc, M, dsub, norms);
    check(hipGetLastError(), "pq_norms");
}

void launch_pq_cell_table(const float* cent, int nlist, int dim, const float* pqc, int M, int dsub, float* T,
                          hipStream_t s) {
    if (nlist <= 0) return;
    pq_cell_table_kernel<<<grid_of((int64_t)nlist * M * kPqKsub, 256), 256, 0, s>>>(cent, nlist, dim, pqc, M, dsub,
                                                                                   T);
    check(hipGetLastError(), "pq_cell_table");
}

void launch_pq_codes(const int* subAssign, const int* rid, int64_t n, int M, int mm, uint8_t* codes, hipStream_t s) {
    if (n <= 0) return;
    pq_codes_kernel<<<grid_of(n, 256), 256, 0, s>>>(subAssign, rid, n, M, mm, codes);
    check(hipGetLastError(), "pq_codes");
}

void launch_pq_lut(const float* q, int nq, int dim, const float* pqc, const float* norms, int M, int dsub, float* lut,
                   hipStream_t s) {
    if (nq <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    if (dsub <= kLutMaxDsub && (nq + kLutQ - 1) / kLutQ <= 0x7FFFFFFF && M <= 65535)
        pq_lut_kernel<<<dim3((unsigned)((nq + kLutQ - 1) / kLutQ), (unsigned)M), kPqKsub, 0, s>>>(q, nq, dim, pqc,
                                                                                              norms, M, dsub, lut);
    else
        pq_lut_wide_kernel<<<grid_of((int64_t)nq * M * kPqKsub, 256), 256, 0, s>>>(q, nq, dim, pqc, norms, M, dsub,
                                                                                 lut);
    prof_end(tok, s);
    check(hipGetLastError(), "pq_lut");
}

void launch_pq_base(const float* q, int nq, int dim, const float* cent, const int* probe, int np, float* base,
                    hipStream_t s) {
    if (nq <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    pq_base_kernel<<<grid_of((int64_t)nq * np, 256), 256, 0, s>>>(q, nq, dim, cent, probe, np, base);
    prof_end(tok, s);
    check(hipGetLastError(), "pq_base");
}

template <int PASS>
static void launch_adc_p(const AdcParams& p, int grid, size_t lds, hipStream_t s) {
    // the specialised kernels hold 64 / M query slots
    const int M = p.tq == adc_tile_queries(p.M) ? p.M : 0;
    switch (M) {
        case 8: adc_scan_kernel<PASS, 8><<<grid, kAdcBlock, lds, s>>>(p); break;
        case 16: adc_scan_kernel<PASS, 16><<<grid, kAdcBlock, lds, s>>>(p); break;
        case 32: adc_scan_kernel<PASS, 32><<<grid, kAdcBlock, lds, s>>>(p); break;
        case 64: adc_scan_kernel<PASS, 64><<<grid, kAdcBlock, lds, s>>>(p); break;
        default: adc_scan_kernel<PASS, 0><<<grid, kAdcBlock, lds, s>>>(p); break;
    }
}

void launch_adc_scan(const AdcParams& p, int pass, int grid, hipStream_t s) {
    if (grid <= 0) return;
    if (p.M < 1 || p.tq < 1 || p.tq > kAdcMaxTq || p.cap < 1 || p.nprobe < 1 || p.nreg < 1)
        throw std::runtime_error("adc_scan: bad parameters");
    const size_t lds = (size_t)p.tq * p.M * kPqKsub * sizeof(float);
    if (lds > 128 * 1024) throw std::runtime_error("adc_scan: lookup tables exceed LDS");
    static const bool attr = [] {
        const void* fs[] = {
            (const void*)adc_scan_kernel<kPassSample, 8>, (const void*)adc_scan_kernel<kPassSample, 16>,
            (const void*)adc_scan_kernel<kPassSample, 32>, (const void*)adc_scan_kernel<kPassSample, 64>,
            (const void*)adc_scan_kernel<kPassSample, 0>, (const void*)adc_scan_kernel<kPassFull, 8>,
            (const void*)adc_scan_kernel<kPassFull, 16>, (const void*)adc_scan_kernel<kPassFull, 32>,
            (const void*)adc_scan_kernel<kPassFull, 64>, (const void*)adc_scan_kernel<kPassFull, 0>};
        for (const void* f : fs)
            if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024) != hipSuccess)
                throw std::runtime_error("adc_scan: cannot raise the dynamic LDS limit");
        return true;
    }();
    (void)attr;
    void* tok;
    prof_begin(pass == kPassSample ? kFamIvfBound : kFamIvfScan, s, &tok);
    if (pass == kPassSample) launch_adc_p<kPassSample>(p, grid, lds, s);
    else launch_adc_p<kPassFull>(p, grid, lds, s);
    prof_end(tok, s);
    check(hipGetLastError(), "adc_scan");
}

void launch_rerank_keys(const float* q, int nq, int dim, const float* full, const int* shortIds, int kRun, int metric,
                        uint2* cand, int* cnt, hipStream_t s) {
    if (nq <= 0 || kRun <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    count_zero_kernel<<<(nq + 255) / 256, 256, 0, s>>>(cnt, nq);
    const int64_t pairs = (int64_t)nq * kRun;
    if ((pairs + 63) / 64 > 0x7FFFFFFF) throw std::runtime_error("rerank_keys: too many pairs");
    if (dim % 4 == 0)   // float4 rows (the store is 256-byte aligned)
        rerank_rows_kernel<<<(unsigned)((pairs + 63) / 64), 64, 0, s>>>(q, nq, dim, full, shortIds, kRun, metric,
                                                                        cand, cnt);
    else
        rerank_keys_kernel<<<(unsigned)((pairs + 255) / 256), 256, 0, s>>>(q, nq, dim, full, shortIds, kRun, metric,
                                                                           cand, cnt);
    prof_end(tok, s);
    check(hipGetLastError(), "rerank_keys");
}

void launch_rerank_ids(const int* shortIds, int kRun, const int* sel, int nq, int k, int* ids, hipStream_t s) {
    if (nq <= 0 || k <= 0) return;
    rerank_ids_kernel<<<grid_of((int64_t)nq * k, 256), 256, 0, s>>>(shortIds, kRun, sel, nq, k, ids);
    check(hipGetLastError(), "rerank_ids");
}

}  // namespace mflat_amd
