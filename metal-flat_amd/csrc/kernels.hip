// SPDX-License-Identifier: Apache-2.0
// kernels.hip -- hand-written gfx950 kernels for exact flat search.
//
//   scan_filter  fused distance + threshold filter. An fp32 MFMA GEMM tile
//                (v_mfma_f32_32x32x2_f32) of kBM database rows x kBN queries,
//                whose epilogue turns dots into ranking keys and keeps only
//                candidates at or below the query's lexicographic (key, id)
//                bound. The nq x nb distance matrix never reaches HBM: only the
//                few surviving candidates are written. Replaces the reference's
//                MPS GEMM + per-tile merge pair (src/GemmDistance.mm:15-60,
//                src/FlatIndex.mm:63-107,375-402).
//   select       per-query exact top-k of the surviving candidates: radix select
//                on the 64-bit (key, id) composite, then the k winners ordered in
//                LDS (rank placement up to 256 of them, else a bitonic sort). It
//                is the cross-tile merge.
//   row norms / normalisation / packing helpers.
#include "kernels.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <type_traits>
#include <utility>
#include <stdexcept>
#include <string>

namespace mflat_amd {

typedef float fx4 __attribute__((ext_vector_type(4)));
typedef float fx16 __attribute__((ext_vector_type(16)));
typedef _Float16 hx8 __attribute__((ext_vector_type(8)));
typedef __bf16 bx8 __attribute__((ext_vector_type(8)));

// fp16 / bf16 MFMA on 16-byte operand pieces (8 values per lane), fp32 accumulate.
template <int S> __device__ __forceinline__ fx16 mfma32x32x16(fx4 a, fx4 b, fx16 c) {
    if constexpr (S == kF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(hx8, a), __builtin_bit_cast(hx8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bx8, a), __builtin_bit_cast(bx8, b), c, 0, 0, 0);
}
template <int S> __device__ __forceinline__ fx4 mfma16x16x32(fx4 a, fx4 b, fx4 c) {
    if constexpr (S == kF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(hx8, a), __builtin_bit_cast(hx8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bx8, a), __builtin_bit_cast(bx8, b), c, 0, 0, 0);
}

constexpr int kQGroup = 16;      // query blocks co-scheduled per XCD (see scan_filter)
constexpr int kLds = kBK + 4;   // LDS row stride in floats: 16-byte reads of 16
                                // consecutive rows land in distinct banks

// Order-preserving map of a float key to uint32 (ascending float order ==
// ascending unsigned order); NaN never reaches here (the filter rejects it).
__device__ __forceinline__ uint32_t key_to_ord(uint32_t bits) {
    return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}
__device__ __forceinline__ float ord_to_key(uint32_t o) {
    const uint32_t bits = (o & 0x80000000u) ? (o ^ 0x80000000u) : ~o;
    return __uint_as_float(bits);
}
__device__ __forceinline__ uint64_t composite(uint2 c) {
    return ((uint64_t)key_to_ord(c.x) << 32) | (uint64_t)c.y;
}

// First row of split s of a full-database pass: the splits share the kBM-row
// tiles as evenly as possible (tile counts differ by at most one), so a plan
// may take any split count; split nsplit starts at the padded row count.
__device__ __forceinline__ int64_t split_row(const ScanParams& p, int s) {
    const int64_t tiles = (p.nrows + kBM - 1) / kBM;
    return tiles * s / p.nsplit * kBM;
}

static void check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        throw std::runtime_error(std::string(what) + " launch failed: " + hipGetErrorString(e));
}

// ---------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------

// dst[r][c] = src[r*dim + c] for r < n, c < dim; zero elsewhere (r < n_pad, c < dpad)
__global__ void pack_rows_kernel(const float* __restrict__ src, int64_t n, int dim,
                                 float* __restrict__ dst, int64_t n_pad, int dpad) {
    const int64_t total = n_pad * dpad;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / dpad;
        const int c = (int)(i - r * dpad);
        dst[i] = (r < n && c < dim) ? src[r * dim + c] : 0.0f;
    }
}

// fp32 -> storage element bits, round to nearest even. fp16 by the hardware
// conversion (IEEE overflow to inf, subnormals kept); bf16 by rounding the
// upper half of the fp32 pattern (NaN -> the canonical quiet NaN 0x7fc0).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
template <int S> __device__ __forceinline__ uint16_t to_bits(float x) {
    return S == kF16 ? f32_to_f16_bits(x) : f32_to_bf16_bits(x);
}
template <int S> __device__ __forceinline__ float from_bits(uint16_t b) {
    return S == kF16 ? (float)__builtin_bit_cast(_Float16, b) : __uint_as_float((uint32_t)b << 16);
}
// element c of a 16-byte piece (4 fp32 or 8 fp16/bf16 values) as fp32
template <int S> __device__ __forceinline__ float piece_elem(const fx4& v, int c) {
    if constexpr (S == kF32) {
        return v[c];
    } else {
        const uint32_t w = __float_as_uint(v[c >> 1]);
        return from_bits<S>((uint16_t)((c & 1) ? (w >> 16) : (w & 0xffffu)));
    }
}
template <int S> constexpr int piece_elems() { return S == kF32 ? 4 : 8; }

// ||row||^2 with a sequential double sum of the stored values, cast to float:
// the accumulation the reference's rowSqNorms uses (src/Distance.h:40-47), so
// fp32 norms match it bit for bit. One thread per row of a row-major array.
template <int S>
__global__ void row_norms_kernel(const void* __restrict__ v, int64_t n, int dpad, float* __restrict__ out) {
    const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (r >= n) return;
    constexpr int PE = piece_elems<S>();
    const fx4* row = (const fx4*)v + r * (dpad / PE);
    double s = 0.0;
    for (int u = 0; u < dpad / PE; ++u) {
        const fx4 x = row[u];
#pragma unroll
        for (int c = 0; c < PE; ++c) {
            const float e = piece_elem<S>(x, c);
            s += (double)e * e;
        }
    }
    out[r] = (float)s;
}

// One search batch's queries in one launch, a wave per row (rows < n_pad):
// the caller's fp32 row (dim values) -> the zero-padded row of dpad elements
// in the storage type; Cosine first scales it by float(1 / sqrt(s)), s the
// sequential double sum of its squares (zero rows unchanged: the reference's
// normalizeRows, src/Distance.h:50-60); qn = float of the sequential double
// sum of the stored values' squares (rowSqNorms, src/Distance.h:40-47); the
// row's bound set to "no bound" (+inf, -1) when tau_key is given. Rows
// n .. n_pad are zero.
// The row goes in chunks of 64 pieces (16 bytes of output each, one a lane,
// coalesced); each chunk's values are staged in LDS, where lane 0 adds their
// squares in column order, so both sums keep the sequential order.
template <int S>
__global__ void __launch_bounds__(256) prep_queries_kernel(const float* __restrict__ src, int64_t n, int dim,
                                                           int64_t n_pad, int dpad, int cosine,
                                                           void* __restrict__ out, float* __restrict__ qn,
                                                           float* __restrict__ tau_key, int* __restrict__ tau_id) {
    constexpr int PE = piece_elems<S>();
    __shared__ float sRow[4][64 * PE];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t r = blockIdx.x * (int64_t)4 + wave;
    if (r >= n_pad) return;
    fx4* dst = (fx4*)out + r * (dpad / PE);
    const bool live = r < n;
    const float* row = src + r * dim;
    float* st = sRow[wave];
    const int npc = dpad / PE;

    // lane 0 adds the squares of the chunk staged in st (cols values)
    auto addChunk = [&](double acc, int cols) {
        __builtin_amdgcn_wave_barrier();
        if (lane == 0)
            for (int c = 0; c < cols; ++c) acc += (double)st[c] * st[c];
        __builtin_amdgcn_wave_barrier();
        return acc;
    };

    float inv = 1.0f;
    if (live && cosine) {
        double s = 0.0;
        for (int u0 = 0; u0 < npc; u0 += 64) {
            const int c0 = (u0 + lane) * PE;
#pragma unroll
            for (int e = 0; e < PE; ++e) st[lane * PE + e] = c0 + e < dim ? row[c0 + e] : 0.0f;
            const int cols = min(64 * PE, dim - u0 * PE);
            if (cols > 0) s = addChunk(s, cols);
        }
        if (lane == 0 && s > 0.0) inv = (float)(1.0 / sqrt(s));
        inv = __shfl(inv, 0);
    }
    double nrm = 0.0;
    for (int u0 = 0; u0 < npc; u0 += 64) {
        const int u = u0 + lane;
        float v[PE];
#pragma unroll
        for (int e = 0; e < PE; ++e) {
            const int c = u * PE + e;
            float x = (live && u < npc && c < dim) ? row[c] : 0.0f;
            if (cosine) x *= inv;
            if constexpr (S != kF32) x = from_bits<S>(to_bits<S>(x));
            v[e] = x;
            st[lane * PE + e] = x;
        }
        if (u < npc) {
            fx4 piece;
            if constexpr (S == kF32) {
                piece = fx4{v[0], v[1], v[2], v[3]};
            } else {
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    piece[w] = __uint_as_float((uint32_t)to_bits<S>(v[2 * w]) | ((uint32_t)to_bits<S>(v[2 * w + 1]) << 16));
            }
            dst[u] = piece;
        }
        const int cols = min(64 * PE, dim - u0 * PE);
        if (live && cols > 0) nrm = addChunk(nrm, cols);
    }
    if (lane == 0) {
        qn[r] = (float)nrm;
        if (tau_key && live) {
            tau_key[r] = INFINITY;
            tau_id[r] = -1;
        }
    }
}

// In-place L2 normalisation of fp32 row-major rows (reference
// src/Distance.h:50-60): double sum, inv = float(1 / sqrt(s)), x *= inv, zero
// rows unchanged.
__global__ void normalize_rows_kernel(float* __restrict__ v, int64_t n, int dpad) {
    const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (r >= n) return;
    float* row = v + r * dpad;
    double s = 0.0;
    for (int c = 0; c < dpad; ++c) s += (double)row[c] * row[c];
    if (s > 0.0) {
        const float inv = (float)(1.0 / sqrt(s));
        for (int c = 0; c < dpad; ++c) row[c] *= inv;
    }
}

// The same rule's scale factor for rows about to be stored: inv[r] =
// float(1 / sqrt(s)), or 1 for a zero row (x * 1 == x leaves it unchanged).
__global__ void row_inv_norms_kernel(const float* __restrict__ src, int64_t n, int dim,
                                     float* __restrict__ inv) {
    const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (r >= n) return;
    const float* row = src + r * dim;
    double s = 0.0;
    for (int c = 0; c < dim; ++c) s += (double)row[c] * row[c];
    inv[r] = s > 0.0 ? (float)(1.0 / sqrt(s)) : 1.0f;
}

// fp32 -> storage type, elementwise (count multiple of 8 for fp16/bf16).
template <int S>
__global__ void round_rows_kernel(const float* __restrict__ src, int64_t count, uint16_t* __restrict__ dst) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < count;
         i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = to_bits<S>(src[i]);
}

// Database (chunked layout) helpers; see blk_off / blk_off_h. One thread per
// 16-byte piece: 4 fp32 or 8 fp16/bf16 consecutive columns of one row.
template <int S>
__device__ __forceinline__ int64_t piece_off(int64_t row, int col, int dpad) {
    return S == kF32 ? blk_off(row, col, dpad) : blk_off_h(row, col, dpad);
}

template <int S>
__global__ void store_rows_blk_kernel(const float* __restrict__ src, int64_t n, int dim,
                                      const float* __restrict__ inv, void* __restrict__ X, int64_t row0,
                                      int dpad) {
    constexpr int PE = piece_elems<S>();
    const int pn = dpad / PE;
    const int64_t total = n * pn;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / pn;
        const int c = (int)(i - r * pn) * PE;
        const float sc = inv ? inv[r] : 1.0f;
        float v[PE];
#pragma unroll
        for (int j = 0; j < PE; ++j) v[j] = c + j < dim ? (inv ? src[r * dim + c + j] * sc : src[r * dim + c + j]) : 0.0f;
        fx4 w;
        if constexpr (S == kF32) {
            w = fx4{v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                w[j] = __uint_as_float((uint32_t)to_bits<S>(v[2 * j]) | ((uint32_t)to_bits<S>(v[2 * j + 1]) << 16));
        }
        *((fx4*)X + piece_off<S>(row0 + r, c, dpad) / PE) = w;
    }
}

// Sequential double sum over the row in column order (reference rowSqNorms).
template <int S>
__global__ void row_norms_blk_kernel(const void* __restrict__ X, int64_t row0, int64_t n, int dpad,
                                     float* __restrict__ out) {
    const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (r >= n) return;
    constexpr int PE = piece_elems<S>();
    double s = 0.0;
    for (int c = 0; c < dpad; c += PE) {
        const fx4 x = *((const fx4*)X + piece_off<S>(row0 + r, c, dpad) / PE);
#pragma unroll
        for (int j = 0; j < PE; ++j) {
            const float e = piece_elem<S>(x, j);
            s += (double)e * e;
        }
    }
    out[r] = (float)s;
}

// dst row r (chunked) = X row idx[r] (chunked), r < n
template <int S>
__global__ void gather_rows_blk_kernel(const void* __restrict__ X, const int* __restrict__ idx, int n,
                                       int dpad, void* __restrict__ dst) {
    constexpr int PE = piece_elems<S>();
    const int pn = dpad / PE;
    const int64_t total = (int64_t)n * pn;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / pn;
        const int c = (int)(i - r * pn) * PE;
        *((fx4*)dst + piece_off<S>(r, c, dpad) / PE) = *((const fx4*)X + piece_off<S>(idx[r], c, dpad) / PE);
    }
}

// row-major rows of `pieces` 16-byte pieces
__global__ void gather_rows_kernel(const fx4* __restrict__ src, const int* __restrict__ idx,
                                   int n, int pieces, fx4* __restrict__ dst, int64_t n_pad) {
    const int64_t total = n_pad * pieces;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / pieces;
        const int c = (int)(i - r * pieces);
        dst[i] = r < n ? src[(int64_t)idx[r] * pieces + c] : fx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
}

__global__ void gather_f32_kernel(const float* __restrict__ src, const int* __restrict__ idx,
                                  int n, float* __restrict__ dst) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[idx[i]];
}

// tau_out[i] = source sel[i] (0, 1 or 2) at row idx[i]
__global__ void gather_tau_kernel(TauSources src, const int* __restrict__ idx,
                                  const int* __restrict__ sel, int n, float* __restrict__ ko,
                                  int* __restrict__ io) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int q = idx[i];
    const int w = sel[i];
    ko[i] = src.key[w][q];
    io[i] = src.id[w][q];
}

// ---------------------------------------------------------------------------
// device-built retry work lists (flat search)
// ---------------------------------------------------------------------------

// The plan of a retry round (RetryLists), run by one block of NT threads.
// 1. The failing queries (status nonzero), listed in ascending order: a block
//    prefix count over NT x 4 queries per step, four status loads in flight.
// 2. For the first rmax of them, in parallel: bound, ladder step and pooled
//    capacity (LDS scratch w: two 64-bit words per entry).
// 3. Thread 0 walks those capacities in LDS assigning pool offsets while they
//    fit (a query too large for this pool before any fits is left for a
//    later, larger pool).
// 4. In parallel: the scheduled queries' lists, rows of Q and norms (rows
//    past them up to the end of their query block zeroed).
// sW: NT / 64 ints of LDS; w: 2 * rmax 64-bit words of LDS.
template <int NT>
__device__ void retry_plan_block(const RetryPlanArgs& a, int* sW, int* sBase, int* sN, uint64_t* w) {
    const RetryLists& rl = a.lists;
    const RetryLadder& lad = a.ladder;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    constexpr int NW = NT / 64;
    if (tid == 0) *sBase = 0;
    __syncthreads();
    for (int q0 = 0; q0 < a.mb; q0 += NT * 4) {
        int st[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int q = q0 + u * NT + tid;
            st[u] = q < a.mb ? a.status[q] : 0;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int q = q0 + u * NT + tid;
            if (a.first && q < a.mb) rl.lvl[q] = 0;
            const bool f = st[u] != 0;
            const unsigned long long bal = __ballot(f);
            if (lane == 0) sW[wave] = __popcll(bal);
            __syncthreads();
            int base = *sBase;
            for (int v = 0; v < wave; ++v) base += sW[v];
            if (f) rl.fail[base + __popcll(bal & ((1ull << lane) - 1ull))] = q;
            __syncthreads();
            if (tid == 0) {
                int t = *sBase;
                for (int v = 0; v < NW; ++v) t += sW[v];
                *sBase = t;
            }
            __syncthreads();
        }
    }
    const int nfail = *sBase;
    const int nc = nfail < a.rmax ? nfail : a.rmax;
    for (int i = tid; i < nc; i += NT) {
        const int q = rl.fail[i];
        const int stq = a.status[q];
        float bk = INFINITY;   // "no bound": every row with a finite key
        int bi = -1;
        int need = a.all_rows;
        int step = a.first ? 0 : rl.lvl[q];
        if (stq & 1) {
            bk = a.tau_k_key[q];
            bi = a.tau_k_id[q];
            need = a.total[q] > 1 ? a.total[q] : 1;
        } else if (step == 0 && lad.j2_key) {
            bk = lad.j2_key[q];
            bi = lad.j2_id[q];
            need = lad.cap_j2;
            step = 1;
        } else if (step <= 1 && lad.g_key) {
            bk = lad.g_key[q];
            bi = lad.g_id[q];
            need = lad.cap_g;
            step = 2;
        } else {
            step = 3;
        }
        w[2 * i] = ((uint64_t)(uint32_t)step << 32) | (uint32_t)need;
        w[2 * i + 1] = ((uint64_t)__float_as_uint(bk) << 32) | (uint32_t)bi;
    }
    __syncthreads();
    if (tid == 0) {
        int64_t off = 0;
        int n = 0;
        for (int i = 0; i < nc; ++i) {
            const int need = (int)(uint32_t)w[2 * i];
            if (off + need > a.pool_entries) {
                if (n == 0 && off == 0) {   // too large for this pool: a later round's larger pool
                    w[2 * i] = ~0ull;
                    continue;
                }
                for (int j = i; j < nc; ++j) w[2 * j] = ~0ull;
                break;
            }
            w[2 * i] = (w[2 * i] & 0xFF00000000ull) | ((uint64_t)n << 40) | (uint32_t)need;
            rl.qoff[n] = off;
            off += need;
            ++n;
        }
        rl.counters[0] = nfail;
        rl.counters[1] = n;
        rl.counters[2] = 0;
        *sN = n;
    }
    __syncthreads();
    for (int i = tid; i < nc; i += NT) {
        const uint64_t w0 = w[2 * i];
        if (w0 == ~0ull) continue;
        const int pos = (int)(w0 >> 40);
        const int q = rl.fail[i];
        rl.lvl[q] = (unsigned char)((w0 >> 32) & 0xFF);
        rl.idx[pos] = q;
        rl.tk[pos] = __uint_as_float((uint32_t)(w[2 * i + 1] >> 32));
        rl.ti[pos] = (int)(uint32_t)w[2 * i + 1];
        rl.qcap[pos] = (int)(uint32_t)w0;
        rl.qcnt[(int64_t)pos * kPoolCntStride] = 0;
    }
    __syncthreads();
    // gather: the scheduled queries' rows, then zeros to the end of the last
    // live query block (its masked rows)
    const int n = *sN;
    const int rowP = a.row_bytes / 16;
    int fill = (n + kBN - 1) / kBN * kBN;
    if (fill > a.rows_pad) fill = a.rows_pad;
    const fx4* src = (const fx4*)a.Q;
    fx4* dst = (fx4*)a.dst_q;
    for (int64_t i = tid; i < (int64_t)fill * rowP; i += NT) {
        const int r = (int)(i / rowP);
        const int c = (int)(i - (int64_t)r * rowP);
        dst[i] = r < n ? src[(int64_t)rl.idx[r] * rowP + c] : fx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    for (int r = tid; r < fill; r += NT) a.dst_qn[r] = r < n ? a.qn[rl.idx[r]] : 0.0f;
}

__global__ void __launch_bounds__(1024) retry_plan_kernel(RetryPlanArgs a) {
    __shared__ int sW[16];
    __shared__ int sBase, sN;
    __shared__ uint64_t w[2 * kRetryPlanMax];
    retry_plan_block<1024>(a, sW, &sBase, &sN, w);
}

// "No bound": (+inf, -1) admits every finite key and rejects +inf and NaN,
// matching the reference, which never inserts a score of -inf or NaN.
__global__ void fill_tau_none_kernel(float* __restrict__ key, int* __restrict__ id, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) { key[i] = INFINITY; id[i] = -1; }
}

__global__ void tau_min_kernel(float* __restrict__ ka, int* __restrict__ ia, const float* __restrict__ kb,
                               const int* __restrict__ ib, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float k = kb[i];
    const int id = ib[i];
    if (k < ka[i] || (k == ka[i] && id < ia[i])) { ka[i] = k; ia[i] = id; }
}

__global__ void fill_empty_kernel(int32_t* __restrict__ ids, float* __restrict__ vals,
                                  int64_t count, float empty) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < count;
         i += (int64_t)gridDim.x * blockDim.x) {
        if (ids) ids[i] = -1;
        if (vals) vals[i] = empty;
    }
}

// max over the finite-or-+inf norms (NaN skipped) -> *out as float bits.
// Norms are >= 0, so their bit patterns order like their values.
__global__ void max_norm_kernel(const float* __restrict__ xn, int64_t n, unsigned* __restrict__ out) {
    __shared__ float sm[256];
    float m = 0.0f;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float v = xn[i];
        if (v > m) m = v;          // false for NaN
    }
    sm[threadIdx.x] = m;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if ((int)threadIdx.x < off && sm[threadIdx.x + off] > sm[threadIdx.x])
            sm[threadIdx.x] = sm[threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) atomicMax(out, __float_as_uint(sm[0]));
}

// ---------------------------------------------------------------------------
// filter epilogue shared by the MFMA scan kernels
// ---------------------------------------------------------------------------
//
// One group of a lane's 32 x 32 accumulators: rows r0 .. r0 + 3 (register
// g4*4 + i of each block, row norms xn4) against the lane's query slots b0 ..
// b0 + NS - 1 (acc[b0 + b], per-query state tk/ti/qn/ft/qv). Rows at or above
// rowLim are padding; row r reports id r * idStride + idb[slot]. 4 NS fast
// tests without branches, then one wave-level branch: a group rarely holds a
// survivor in any of the 64 lanes. Only survivors take the exact
// lexicographic test; they go to emit(slot, key, id), or, for k = 1, replace
// the slot's running best.
// LQ: the survivor-only state (bound key and id, query norm) is read from the
// workgroup's LDS tables lq (entry bn * 32 + lq.r32 for slot bn) instead of
// the register arrays tk / ti / qn, which the caller then leaves dead: in
// kernels at the register limit this keeps survivor handling free of scratch
// reloads, whose wait for vector memory also waits for every prefetch load in
// flight.
// MAXT: the group test compares each slot's largest accumulator with its
// bound (larger = nearer), 2 operations a row pair instead of 2 a value; the
// slow path then tests every value. It needs accumulators ordered like the
// key: IP (the dot) or PRE.
// PRE (L2): the accumulators hold dot - ||x||^2 / 2 (the MFMA chain started
// from -||x||^2 / 2 instead of 0), so xn4 is unused, ft holds -ft / 2 (the
// bound on dot - ||x||^2 / 2) and key = fma(-2, acc, ||q||^2).
struct QTab {
    const float* tk;
    const int* ti;
    const float* qn;
    int r32;
};
template <int METRIC, int PASS, int NB, int NS, bool LQ = false, bool MAXT = false, bool PRE = false, class Emit>
__device__ __forceinline__ void filter_group(const fx16 (&acc)[NB], int g4, int b0, const fx4& xn4, int64_t r0,
                                             int64_t rowLim, int idStride, const int (&idb)[NB],
                                             const ScanParams& p, float (&tk)[NB], int (&ti)[NB],
                                             const float (&qn)[NB], float (&ft)[NB], const bool (&qv)[NB],
                                             const QTab& lq, Emit&& emit) {
    static_assert(!MAXT || METRIC != 0 || PRE, "MAXT needs accumulators ordered like the key");
    static_assert(!PRE || METRIC == 0, "PRE is an L2 form");
    bool f[4][NS];
    bool any = false;
    if constexpr (MAXT) {
        // fmaxf drops a NaN value (never a survivor); the slow path's tests
        // below reject it on their own
#pragma unroll
        for (int b = 0; b < NS; ++b) {
            const fx16& a = acc[b0 + b];
            const float m = fmaxf(fmaxf(a[g4 * 4 + 0], a[g4 * 4 + 1]), fmaxf(a[g4 * 4 + 2], a[g4 * 4 + 3]));
            any |= m >= ft[b0 + b];
        }
        if (!any) return;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int b = 0; b < NS; ++b) f[i][b] = acc[b0 + b][g4 * 4 + i] >= ft[b0 + b];
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int b = 0; b < NS; ++b) {
                const float dot = acc[b0 + b][g4 * 4 + i];
                f[i][b] = METRIC == 0 ? fmaf(-2.0f, dot, xn4[i]) <= ft[b0 + b] : dot >= ft[b0 + b];
                any |= f[i][b];
            }
        if (!any) return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t row = r0 + i;
        const bool rv = row < rowLim;
        const int idr = (int)(row * idStride);
#pragma unroll
        for (int b = 0; b < NS; ++b) {
            const int bn = b0 + b;
            if (!f[i][b]) continue;
            const int id = idr + idb[bn];
            const float dot = acc[bn][g4 * 4 + i];
            float key;
            if (METRIC == 0) {
                const float qnb = LQ ? lq.qn[bn * 32 + lq.r32] : qn[bn];
                const float t = PRE ? fmaf(-2.0f, dot, qnb) : fmaf(-2.0f, dot, qnb + xn4[i]);
                key = (t < 0.0f ? 0.0f : t) + 0.0f;
            } else {
                key = -dot + 0.0f;
            }
            if (PASS == kPassArgmin && !LQ) {
                // k = 1: keep the lexicographically smallest (key, id)
                if (rv && qv[bn] && (key < tk[bn] || (key == tk[bn] && id < ti[bn]))) {
                    tk[bn] = key;
                    ti[bn] = id;
                    ft[bn] = METRIC == 0 ? (key - qn[bn]) + 0x1p-20f * (key + 2.0f * qn[bn] + 2.0f * p.xnorm_max)
                                         : -key;
                    if (PRE) ft[bn] *= -0.5f;
                }
                continue;
            }
            const float tkb = LQ ? lq.tk[bn * 32 + lq.r32] : tk[bn];
            const int tib = LQ ? lq.ti[bn * 32 + lq.r32] : ti[bn];
            if (rv && qv[bn] && (key < tkb || (key == tkb && id <= tib))) emit(bn, key, id);
        }
    }
}

// ---------------------------------------------------------------------------
// scan_filter: MFMA distance tile + threshold filter
// ---------------------------------------------------------------------------
//
// Workgroup: 256 threads = 4 waves in a 2 x 2 arrangement; each wave owns a
// 64-row x 64-query quarter of the 128 x 128 tile as 2 x 2 blocks of
// v_mfma_f32_32x32x2_f32 (fp32 storage) or v_mfma_f32_32x32x16_{f16,bf16}.
// The operand roles: A = database rows (M), B = queries (N), so accumulator
// register r of lane l holds
//     row   = 8*(r/4) + 4*(l/32) + (r%4),   query = l%32
// i.e. every lane sees 16 rows of ONE query per block, which keeps the
// per-query threshold in a register during the epilogue.
//
// The K dimension is consumed in chunks of 128 bytes per row (32 fp32 or 64
// fp16/bf16 columns) staged through LDS, double buffered; one barrier per
// chunk. Every LDS operand read is a single ds_read_b128 of 16 bytes at byte
// 16 h + 32 g of the row (lane half h, group g = 0..3), on both operands:
//   fp32: MFMA step j of group g pairs columns (8g + j, 8g + 4 + j);
//   fp16/bf16: group g is one MFMA over columns 16g .. 16g + 15, lane half h
//   supplying 8h .. 8h + 7 of them.
// The same permutation on both operands leaves the dot unchanged. With fp16 /
// bf16 and dpad = 64 c + 32, the last chunk holds 32 real columns; the loaders
// fill its other half of LDS with zeros.
//
// A workgroup owns one query block and one split (a contiguous range of
// database rows) and walks the split's tiles in ascending row order. Linear
// workgroup ids are remapped so that each XCD (ids are dealt round-robin over
// the 8 XCDs) receives a contiguous run of (split, query block) pairs: the
// workgroups resident on one XCD then stream the same database rows through
// that XCD's L2.
// PASS only names the instantiation (0 = full database, 1 = row sample,
// 2 = retry of a few queries), so profiles separate the passes; the code is
// the same.
// IVF: a workgroup takes one IVF work item (a cell and up to 128 of the
// entries probing it) instead of a (query block, split): rows of that cell,
// queries gathered by entry, survivors into the entries' regions (spill as
// in scan_resident), ids = the row's scan position. The IVF index uses it
// where a 128-query tile does not fit scan_resident's LDS (large d).
template <int S, int METRIC, int PASS, bool IVF = false>
__global__ void __launch_bounds__(256, 2) scan_filter_kernel(ScanParams p) {
    constexpr int ES = S == kF32 ? 4 : 2;   // element bytes
    // fp16/bf16: the filter's group test through maxima (MAXT) and, for L2,
    // accumulators started from -||x||^2 / 2 (PRE); see filter_group
    constexpr bool MAXT = S != kF32;
    constexpr bool PRE = S != kF32 && METRIC == 0;
    __shared__ __attribute__((aligned(16))) float sX[2 * kBM * kLds];
    __shared__ __attribute__((aligned(16))) float sQ[2 * kBN * kLds];
    __shared__ __attribute__((aligned(16))) float sXn[2 * kBM];   // tile row norms, by tile parity
    __shared__ int sCnt[kBN];
    __shared__ unsigned long long sBest[kBN];   // argmin: per-query (ordered key, id)
    // Flat retry pass: survivors staged in LDS and written in one block of
    // slots per (workgroup, query), as in scan_resident (there: why); the
    // stage fits the LDS two workgroups per CU leave.
    constexpr bool STAGE = PASS == kPassRetry && !IVF;
    constexpr int kStage = 480;
    __shared__ uint2 sStage[STAGE ? kStage : 1];
    __shared__ uint32_t sStageTag[STAGE ? kStage : 1];
    __shared__ int sStageN;
    __shared__ int sEnt[IVF ? kBN : 1];   // IVF: the item's entries (-1: empty slot)
    __shared__ int sQi[IVF ? kBN : 1];    // ... their queries
    __shared__ int sReg[IVF ? kBN : 1];   // ... their candidate regions

    // Workgroup -> (query block, split). Hardware deals consecutive ids
    // round-robin over the 8 XCDs; v renumbers them so each XCD owns a
    // contiguous range. Within it, query blocks go in groups of kQGroup,
    // split-major inside a group: the ~64 workgroups resident on one XCD then
    // cover kQGroup query blocks (1 MB of Q tiles at d = 128, kept in its 4 MB
    // L2) times a few splits, and each database tile they stream is shared by
    // kQGroup workgroups.
    int qb = 0, split = 0;
    int4 wk = make_int4(0, 0, 0, 0);   // IVF work item: (cell, first entry, entries, 0)
    if constexpr (IVF) {
        if ((int)blockIdx.x >= *p.ivf_nwork) return;
        wk = p.ivf_work[blockIdx.x];
    } else {
        const int nwg = gridDim.x;
        const int bid = blockIdx.x;
        if (PASS == kPassRetry && p.nq_dev) {
            // A device-sized retry covers more query blocks than it usually
            // fills: block-major order dispatches the live blocks' splits
            // first, over every XCD, and the idle blocks trail.
            qb = bid / p.nsplit;
            split = bid - qb * p.nsplit;
        } else {
            const int full = (nwg / 8) * 8;
            const int v = bid < full ? (bid % 8) * (full / 8) + bid / 8 : bid;
            const int qgrp = p.qgroup > 0 ? p.qgroup : kQGroup;
            const int grpSize = p.nqb < qgrp ? p.nqb : qgrp;
            const int grp = v / (grpSize * p.nsplit);
            const int r = v - grp * grpSize * p.nsplit;
            const int inGrp = p.nqb - grp * grpSize < grpSize ? p.nqb - grp * grpSize : grpSize;
            split = r / inGrp;
            qb = grp * grpSize + (r - split * inGrp);
        }
    }
    // A retry whose work list the device built: query blocks beyond it are idle.
    const int nqv = (PASS == kPassRetry && p.nq_dev) ? *p.nq_dev : p.nq;
    if (!IVF && qb * kBN >= nqv) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave & 1;
    const int wn = wave >> 1;
    const int r32 = lane & 31;
    const int h = lane >> 5;

    if (tid == 0) sStageN = 0;
    if (tid < kBN) {
        sCnt[tid] = 0;
        sBest[tid] = ~0ull;
        if constexpr (IVF) {
            const int e = tid < wk.z ? p.ivf_ent[wk.y + tid] : -1;
            const int q = e >= 0 ? e / p.ivf_nprobe : -1;
            sEnt[tid] = e;
            sQi[tid] = q;
            sReg[tid] = e >= 0 ? q * p.ivf_nreg + (e - q * p.ivf_nprobe) : -1;
        }
    }
    if constexpr (IVF) __syncthreads();

    // Per-lane query state for the two query blocks this lane sees.
    // ft is the fast-reject bound, a NECESSARY condition for key <= tau:
    //   IP: key = -dot <= tau  <=>  dot >= -tau               (exact)
    //   L2: key <= tau  ==>  fma(-2, dot, ||x||^2) <= tau - ||q||^2 + M,
    //       M = 2^-20 (tau + 2||q||^2 + 2 max||x||^2). Both sides of the L2 key
    //       (||q||^2 + ||x||^2) - 2 q.x and ||x||^2 - 2 q.x round at most once
    //       per operation, so they differ from exact arithmetic by at most
    //       2^-24 (2||q||^2 + 3||x||^2) + 2^-23 tau; M covers that sixteen-fold
    //       together with the rounding of tau - ||q||^2 + M itself.
    // Only candidates passing the fast test take the exact lexicographic test.
    float tk[2], qn[2], ft[2];
    int ti[2];
    bool qv[2];
    int idb[2] = {0, 0};   // ids are row * id_stride (+ the cell's first scan position, IVF)
#pragma unroll
    for (int bn = 0; bn < 2; ++bn) {
        int q;
        if constexpr (IVF) {
            const int ql = wn * 64 + bn * 32 + r32;
            q = sQi[ql];
            qv[bn] = q >= 0;
            if (qv[bn]) idb[bn] = p.ivf_pos[sEnt[ql]];
        } else {
            q = qb * kBN + wn * 64 + bn * 32 + r32;
            qv[bn] = q < nqv;
        }
        if (PASS == kPassArgmin) {   // running best of this lane, from "no bound"
            tk[bn] = INFINITY;
            ti[bn] = -1;
        } else {
            tk[bn] = qv[bn] ? p.tau_key[q] : 0.0f;
            ti[bn] = qv[bn] ? p.tau_id[q] : -1;
        }
        qn[bn] = (METRIC == 0 && qv[bn]) ? p.qnorm[q] : 0.0f;
        if (METRIC == 0) {
            const float m = 0x1p-20f * (tk[bn] + 2.0f * qn[bn] + 2.0f * p.xnorm_max);
            ft[bn] = qv[bn] ? (tk[bn] - qn[bn]) + m : -INFINITY;
            if (PRE) ft[bn] *= -0.5f;
        } else {
            ft[bn] = qv[bn] ? -tk[bn] : INFINITY;
        }
    }

    // Rows [rowBeg, rowBeg + kBM ntiles); filter rows count from rowOrg (IVF:
    // the cell's first row), rows at or above rowLim are padding.
    int64_t rowBeg, rowOrg, rowLim;
    int ntiles;
    if constexpr (IVF) {
        rowBeg = p.ivf_cell_pad[wk.x];
        rowOrg = 0;
        rowLim = p.ivf_cell_size[wk.x];
        if (p.ivf_row_cap > 0 && rowLim > p.ivf_row_cap) rowLim = p.ivf_row_cap;   // a cell's first rows only
        ntiles = (int)((rowLim + kBM - 1) / kBM);
    } else {
        rowBeg = split_row(p, split);
        const int64_t rowEnd = split_row(p, split + 1);
        ntiles = rowEnd > rowBeg ? (int)((rowEnd - rowBeg) / kBM) : 0;
        rowOrg = rowBeg;
        rowLim = p.nrows;
    }
    const int nk = S == kF32 ? p.dpad / kBK : (p.dpad + 63) / 64;
    const bool halfTail = S != kF32 && (p.dpad & 32) != 0;   // last chunk: 32 columns
    const int total = ntiles * nk;

    // global -> register staging: 4 pieces of 16 bytes per thread per operand
    const int ldRow = tid >> 3;         // + 32*i
    const int ldCol = (tid & 7) * 4;    // in floats = 16-byte pieces
    const char* Xb = (const char*)p.X + rowBeg * p.dpad * ES;
    const char* Qb = (const char*)p.Q + (int64_t)qb * kBN * p.dpad * ES;
    // IVF: this thread's four query rows (ldRow + 32 i), gathered by entry
    const char* qrow[IVF ? 4 : 1] = {};
    if constexpr (IVF) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = sQi[ldRow + 32 * i];
            qrow[i] = q >= 0 ? (const char*)p.Q + (int64_t)q * p.dpad * ES : nullptr;
        }
    }
    fx4 rx[4], rq[4], rn;
    // The first chunk of every tile also brings the tile's 128 row norms
    // (threads 0..31, one float4 each) into sXn[tile & 1]; the epilogue of
    // that tile reads them from LDS instead of waiting on global memory.
    // Database chunks are linear 4 KB pieces (one per 32-row block, chunked
    // layout): thread t takes 16-byte piece t of each, i.e. row 32 i + xRow,
    // LDS float column xCol (fp32: columns 8 ((t >> 4) & 3) + 4 ((t >> 6) & 1)
    // .. +3; fp16/bf16: sub-chunk t >> 7, columns 32 (t >> 7) + 8 ((t >> 4) & 3)
    // .. +7). A 32-column fp16/bf16 tail chunk has only sub-chunk 0: threads
    // t >= 128 load nothing and stage zeros, as do the query loaders of its
    // second half.
    const int xRow = S == kF32 ? 16 * (tid >> 7) + (tid & 15) : 16 * ((tid >> 6) & 1) + (tid & 15);
    const int xCol = S == kF32 ? 8 * ((tid >> 4) & 3) + 4 * ((tid >> 6) & 1)
                               : 16 * (tid >> 7) + 4 * ((tid >> 4) & 3);
    auto gload = [&](int tile, int kc) {
        const char* xs = Xb + ((int64_t)tile * kBM) * p.dpad * ES + kc * 4096 + tid * 16;
        const int qo = kc * 128 + ldCol * 4;
        const char* qs = Qb + qo;
        const bool zx = S != kF32 && halfTail && kc == nk - 1 && tid >= 128;
        const bool zq = S != kF32 && halfTail && kc == nk - 1 && (tid & 7) >= 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            rx[i] = fx4{0.0f, 0.0f, 0.0f, 0.0f};
            rq[i] = fx4{0.0f, 0.0f, 0.0f, 0.0f};
            if (!zx) rx[i] = *(const fx4*)(xs + (int64_t)i * 32 * p.dpad * ES);
            if constexpr (IVF) {
                if (!zq && qrow[i]) rq[i] = *(const fx4*)(qrow[i] + qo);
            } else {
                if (!zq) rq[i] = *(const fx4*)(qs + (int64_t)(ldRow + 32 * i) * p.dpad * ES);
            }
        }
        if (METRIC == 0 && kc == 0 && tid < kBM / 4)
            rn = *(const fx4*)(p.xnorm + rowBeg + (int64_t)tile * kBM + tid * 4);
    };
    auto lstore = [&](int tile, int kc, int buf) {
        float* dx = sX + buf * (kBM * kLds);
        float* dq = sQ + buf * (kBN * kLds);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            *(fx4*)(dx + (32 * i + xRow) * kLds + xCol) = rx[i];
            *(fx4*)(dq + (ldRow + 32 * i) * kLds + ldCol) = rq[i];
        }
        if (METRIC == 0 && kc == 0 && tid < kBM / 4)
            *(fx4*)(sXn + (tile & 1) * kBM + tid * 4) = PRE ? rn * -0.5f : rn;
    };

    fx16 acc[2][2];

    if (total > 0) {
        gload(0, 0);
        lstore(0, 0, 0);
    }
    __syncthreads();

    const int aOff = (wm * 64 + r32) * kLds + h * 4;
    const int bOff = (wn * 64 + r32) * kLds + h * 4;

    int tile = 0, kc = 0;   // position of chunk `it`, advanced without division
    for (int it = 0; it < total; ++it) {
        const int buf = it & 1;
        const bool lastK = kc == nk - 1;
        const int ntile = lastK ? tile + 1 : tile;
        const int nkc = lastK ? 0 : kc + 1;
        if (it + 1 < total) gload(ntile, nkc);

        const float* sx = sX + buf * (kBM * kLds);
        const float* sq = sQ + buf * (kBN * kLds);
        // the epilogue's row norms, read before the last chunk's MFMAs
        fx4 xnr[2][4];
        if (METRIC == 0 && !PRE && kc == nk - 1) {
#pragma unroll
            for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4)
                    xnr[bm][g4] = *(const fx4*)(sXn + (tile & 1) * kBM + wm * 64 + bm * 32 + g4 * 8 + h * 4);
        }
        // A tile's first chunk starts every accumulator from an inline zero C
        // operand, so no accumulator is ever cleared with moves.
        auto mma = [&](auto zeroTag) {
            constexpr bool ZERO = decltype(zeroTag)::value;
            const fx16 z = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f,
                            0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                fx4 a0 = *(const fx4*)(sx + aOff + g * 8);
                fx4 a1 = *(const fx4*)(sx + aOff + 32 * kLds + g * 8);
                fx4 b0 = *(const fx4*)(sq + bOff + g * 8);
                fx4 b1 = *(const fx4*)(sq + bOff + 32 * kLds + g * 8);
                if constexpr (PRE) {
                    // a tile's first MFMAs start from acc[bm][0] (set below to
                    // the rows' -||x||^2 / 2), which is overwritten last
                    const bool zc = ZERO && g == 0;
                    acc[0][1] = mfma32x32x16<S>(a0, b1, zc ? acc[0][0] : acc[0][1]);
                    acc[0][0] = mfma32x32x16<S>(a0, b0, acc[0][0]);
                    acc[1][1] = mfma32x32x16<S>(a1, b1, zc ? acc[1][0] : acc[1][1]);
                    acc[1][0] = mfma32x32x16<S>(a1, b0, acc[1][0]);
                    continue;
                } else if constexpr (S != kF32) {
                    const bool zc = ZERO && g == 0;
                    acc[0][0] = mfma32x32x16<S>(a0, b0, zc ? z : acc[0][0]);
                    acc[0][1] = mfma32x32x16<S>(a0, b1, zc ? z : acc[0][1]);
                    acc[1][0] = mfma32x32x16<S>(a1, b0, zc ? z : acc[1][0]);
                    acc[1][1] = mfma32x32x16<S>(a1, b1, zc ? z : acc[1][1]);
                    continue;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (ZERO && g == 0 && j == 0) {
                        acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[j], b0[j], z, 0, 0, 0);
                        acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[j], b1[j], z, 0, 0, 0);
                        acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[j], b0[j], z, 0, 0, 0);
                        acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[j], b1[j], z, 0, 0, 0);
                    } else {
                        acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[j], b0[j], acc[0][0], 0, 0, 0);
                        acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[j], b1[j], acc[0][1], 0, 0, 0);
                        acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[j], b0[j], acc[1][0], 0, 0, 0);
                        acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[j], b1[j], acc[1][1], 0, 0, 0);
                    }
                }
            }
        };
        if (PRE && kc == 0) {
            // the tile's -||x||^2 / 2 (sXn, staged with its first chunk) for
            // the rows of this lane's accumulator registers: row wm * 64 +
            // bm * 32 + 8 g4 + 4 h + i at register 4 g4 + i
#pragma unroll
            for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const fx4 v = *(const fx4*)(sXn + (tile & 1) * kBM + wm * 64 + bm * 32 + g4 * 8 + h * 4);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[bm][0][g4 * 4 + i] = v[i];
                }
        }
        if (kc == 0)
            mma(std::true_type{});
        else
            mma(std::false_type{});

        if (kc == nk - 1) {
            // epilogue: keys, threshold test, append survivors
            const int64_t tileRow0 = rowOrg + (int64_t)tile * kBM;
#pragma unroll
            for (int bm = 0; bm < 2; ++bm) {
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int rl = wm * 64 + bm * 32 + g4 * 8 + h * 4;
                    const int64_t r0 = tileRow0 + rl;
                    fx4 xn4 = {0.0f, 0.0f, 0.0f, 0.0f};
                    if (METRIC == 0 && !PRE) xn4 = xnr[bm][g4];
                    filter_group<METRIC, PASS, 2, 2, false, MAXT, PRE>(acc[bm], g4, 0, xn4, r0, rowLim,
                                                                       IVF ? 1 : p.id_stride, idb,
                                                  p, tk, ti, qn, ft, qv, QTab{nullptr, nullptr, nullptr, 0},
                                                  [&](int bn, float key, int id) {
                        const int ql = wn * 64 + bn * 32 + r32;
                        const uint2 v = make_uint2(__float_as_uint(key), (unsigned)id);
                        if constexpr (STAGE) {
                            if (p.qcnt) {
                                const int e = atomicAdd(&sStageN, 1);
                                if (e < kStage) {
                                    sStage[e] = v;
                                    sStageTag[e] = ((uint32_t)atomicAdd(&sCnt[ql], 1) << 8) | (uint32_t)ql;
                                } else {   // a global slot of its own
                                    const int q = qb * kBN + ql;
                                    const int gs = atomicAdd(&p.qcnt[(int64_t)q * kPoolCntStride], 1);
                                    if (gs < p.qcap[q]) p.cand[p.qoff[q] + gs] = v;
                                }
                                return;
                            }
                        }
                        const int slot = atomicAdd(&sCnt[ql], 1);
                        if constexpr (IVF) {
                            if (slot < p.cap) {
                                p.cand[(int64_t)sReg[ql] * p.cap + slot] = v;
                            } else if (p.ivf_spill) {   // the query's spill region (global count)
                                const int64_t sr = (int64_t)sQi[ql] * p.ivf_nreg + p.ivf_nprobe;
                                const int sp = atomicAdd(&p.cnt[sr], 1);
                                if (sp < p.cap) p.cand[sr * p.cap + sp] = v;
                            }
                        } else if (PASS == kPassRetry && p.qcnt) {   // pooled region of the query
                            const int q = qb * kBN + ql;
                            const int gs = atomicAdd(&p.qcnt[(int64_t)q * kPoolCntStride], 1);
                            if (gs < p.qcap[q]) p.cand[p.qoff[q] + gs] = v;
                        } else if (slot < p.cap) {
                            const int64_t q = (int64_t)qb * kBN + ql;
                            p.cand[(q * p.nsplit + split) * p.cap + slot] = v;
                        }
                    });
                }
            }
        }

        if (it + 1 < total) lstore(ntile, nkc, buf ^ 1);
        __syncthreads();
        tile = ntile;
        kc = nkc;
    }

    if (PASS == kPassArgmin) {
        // the 4 lanes that saw each query -> LDS -> one global atomic per query
#pragma unroll
        for (int bn = 0; bn < 2; ++bn)
            if (ti[bn] >= 0)
                atomicMin(&sBest[wn * 64 + bn * 32 + r32],
                          ((unsigned long long)key_to_ord(__float_as_uint(tk[bn])) << 32) | (unsigned)ti[bn]);
        __syncthreads();
        if (tid < kBN) {
            const int q = qb * kBN + tid;
            if (q < p.nq && sBest[tid] != ~0ull) atomicMin(&p.best[q], sBest[tid]);
        }
        return;
    }
    __syncthreads();
    if constexpr (STAGE) {
        if (p.qcnt) {
            int* sBase = reinterpret_cast<int*>(sBest);
            if (tid < kBN) {
                const int q = qb * kBN + tid;
                sBase[tid] = sCnt[tid] > 0 ? atomicAdd(&p.qcnt[(int64_t)q * kPoolCntStride], sCnt[tid]) : 0;
            }
            __syncthreads();
            const int n = sStageN < kStage ? sStageN : kStage;
            for (int e = tid; e < n; e += 256) {
                const uint32_t tag = sStageTag[e];
                const int ql = (int)(tag & 255u);
                const int q = qb * kBN + ql;
                const int gs = sBase[ql] + (int)(tag >> 8);
                if (gs < p.qcap[q]) p.cand[p.qoff[q] + gs] = sStage[e];
            }
            return;
        }
    }
    if (tid < kBN) {
        if constexpr (IVF) {
            if (sReg[tid] >= 0) p.cnt[sReg[tid]] = p.ivf_spill && sCnt[tid] > p.cap ? p.cap : sCnt[tid];
        } else {
            const int q = qb * kBN + tid;
            if (q < nqv && !(PASS == kPassRetry && p.qcnt)) p.cnt[(int64_t)q * p.nsplit + split] = sCnt[tid];
        }
    }
}

// ---------------------------------------------------------------------------
// scan_wide: fp16/bf16 tiles of 256 rows x 256 queries (large d)
// ---------------------------------------------------------------------------
//
// For fp16/bf16 storage at a d whose 128-query tile does not fit
// scan_resident's LDS, and batches of more than 128 queries. scan_filter's
// 128 x 128 tile feeds each 32-cycle 16-bit MFMA one 16-byte LDS read a lane
// (2 x 2 blocks a wave) and re-reads a query or database chunk from beyond L2
// for every tile: operand staging and its latency bound it, not the matrix
// cores. Here a workgroup (512 threads, one per CU; two waves a SIMD as
// there) owns 256 rows x 256 queries and each of its 8 waves 64 rows x 128
// queries as 2 x 4 blocks of 32 x 32, so an operand fragment read from LDS
// feeds 2.7 MFMAs on average (2 there) and every staged byte twice the work.
//
// Staging: 32-column stages, copied from global memory straight into LDS
// (global_load_lds_dwordx4: no staging registers, no LDS write
// instructions), four stages in LDS and three in flight while one is
// consumed. A stage holds, for each of the 8 database row blocks and 8 query
// blocks of 32, one 2 KB unit in the chunked layout of blk_off_h: piece
// ((r / 16) * 4 + c / 8) * 16 + r % 16 for row r and column c of the unit,
// which is the database's own order in HBM (a unit is copied verbatim) and
// the order a 32 x 16 MFMA fragment reads in runs of 16 pieces (no bank
// conflicts). Query rows are row-major in HBM; each lane copies the piece of
// that order. One barrier a stage, preceded by a wait for this wave's copies
// of the stage (vector-memory counter, in order) but none of the later ones;
// __syncthreads' fence would wait for all of them. The next copy is issued
// after the stage's first 16-column step (fragment reads first: 3% faster
// than issuing it right after the barrier).
//
// The MFMA sequence per (query, row) pair is scan_filter's, so the keys are
// too: columns in ascending 16-column steps, the L2 accumulators starting
// from -||x||^2 / 2 (PRE), and for dpad = 64 c + 32 two more steps over
// zero operands at the end of each row block, the zero half of scan_filter's
// last 64-column chunk. A search that starts on this kernel runs its sample
// and full passes on it and its retry window (usually under 128 queries) on
// scan_filter: the keys agree, so every bound meets keys computed the same way.
// Database rows come in 128-row tiles (the split layout); a 256-row step
// whose second half lies past the split's last tile copies the split's first
// tile for it and reports none of its rows; query rows at or past nq copy the
// block's first query and are masked (no bound admits them).
constexpr int kWT = 256;                        // rows and queries of a wide tile
constexpr int kWideThreads = 512;               // 8 waves of 64 rows x 128 queries
constexpr int kWideStages = 4;                  // 32-column LDS stages
constexpr int kWideStageBytes = 2 * kWT * 64;   // both operands, 64 bytes a row

// 16 bytes a lane from global memory straight into LDS: lane l's piece lands
// at lds + 16 l (the LDS address is the wave's, the same for every lane). In
// asm, so the compiler does not see an LDS write in flight: it would wait for
// every copy (vmcnt(0)) before any LDS atomic of the epilogue; the kernel
// waits for its copies itself (wide_sync). M0 holds the LDS address; the nop
// is the M0-write-to-use wait state.
__device__ __forceinline__ void lds_copy16(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(lds) : "memory", "m0");
}
// LDS address of a shared-memory object, as a wave-uniform (scalar) value
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p);
}

// Wait until at most N of this wave's vector-memory operations are still
// outstanding and its LDS operations are done, then the workgroup barrier.
template <int N>
__device__ __forceinline__ void wide_sync() {
    static_assert(N >= 0 && N < 16, "the low vmcnt field");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0070 | N);   // vmcnt(N) expcnt(7) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int S, int METRIC, int PASS>
__global__ void __launch_bounds__(512, 1) scan_wide_kernel(ScanParams p) {
    static_assert(S != kF32, "the wide tile is the fp16/bf16 kernel");
    static_assert(PASS != kPassArgmin, "k = 1 runs scan_filter");
    constexpr int ES = 2;
    constexpr bool PRE = METRIC == 0;
    __shared__ __attribute__((aligned(16))) char sOp[kWideStages * kWideStageBytes];
    __shared__ __attribute__((aligned(16))) float sXn[2 * kWT];   // PRE: ||x||^2 of the step, by step parity
    __shared__ int sCnt[kWT];
    // survivor-only query state (bound key and id, query norm) in LDS, not
    // registers: filter_group's LQ tables
    __shared__ float sLTk[kWT];
    __shared__ int sLTi[kWT];
    __shared__ float sLQn[kWT];

    const int nqb = (p.nq + kWT - 1) / kWT;
    int qb, split;
    {
        const int nwg = gridDim.x;
        const int bid = blockIdx.x;
        if (PASS == kPassRetry && p.nq_dev) {   // block-major: the live blocks first
            qb = bid / p.nsplit;
            split = bid - qb * p.nsplit;
        } else {   // scan_filter's XCD grouping
            const int full = (nwg / 8) * 8;
            const int v = bid < full ? (bid % 8) * (full / 8) + bid / 8 : bid;
            const int qgrp = p.qgroup > 0 ? p.qgroup : kQGroup;
            const int grpSize = nqb < qgrp ? nqb : qgrp;
            const int grp = v / (grpSize * p.nsplit);
            const int r = v - grp * grpSize * p.nsplit;
            const int inGrp = nqb - grp * grpSize < grpSize ? nqb - grp * grpSize : grpSize;
            split = r / inGrp;
            qb = grp * grpSize + (r - split * inGrp);
        }
    }
    const int nqv = (PASS == kPassRetry && p.nq_dev) ? *p.nq_dev : p.nq;
    if (qb * kWT >= nqv) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave & 3;    // rows wm * 64 ..
    const int wn = wave >> 2;   // queries wn * 128 ..
    const int r32 = lane & 31;
    const int h = lane >> 5;
    if (tid < kWT) {
        sCnt[tid] = 0;
        const int q = qb * kWT + tid;
        const bool v = q < nqv;
        sLTk[tid] = v ? p.tau_key[q] : 0.0f;
        sLTi[tid] = v ? p.tau_id[q] : -1;
        sLQn[tid] = (METRIC == 0 && v) ? p.qnorm[q] : 0.0f;
    }

    // the lane's four query slots (bn: queries wn * 128 + bn * 32 + r32)
    float tk[4], qn[4], ft[4];
    int ti[4];
    bool qv[4];
    const int idb[4] = {0, 0, 0, 0};
#pragma unroll
    for (int bn = 0; bn < 4; ++bn) {
        const int q = qb * kWT + wn * 128 + bn * 32 + r32;
        qv[bn] = q < nqv;
        tk[bn] = qv[bn] ? p.tau_key[q] : 0.0f;
        ti[bn] = qv[bn] ? p.tau_id[q] : -1;
        qn[bn] = (METRIC == 0 && qv[bn]) ? p.qnorm[q] : 0.0f;
        if (METRIC == 0) {
            const float m = 0x1p-20f * (tk[bn] + 2.0f * qn[bn] + 2.0f * p.xnorm_max);
            ft[bn] = qv[bn] ? -0.5f * ((tk[bn] - qn[bn]) + m) : INFINITY;
        } else {
            ft[bn] = qv[bn] ? -tk[bn] : INFINITY;
        }
    }

    const int64_t rowBeg = split_row(p, split);
    const int64_t rowEnd = split_row(p, split + 1);
    const int tiles = rowEnd > rowBeg ? (int)((rowEnd - rowBeg) / kBM) : 0;   // 128-row tiles
    const int nsteps = (tiles + 1) / 2;
    const int64_t rowLim = rowEnd < p.nrows ? rowEnd : p.nrows;
    const int nk = p.dpad / 32;              // 32-column units of a row
    const bool halfTail = (nk & 1) != 0;     // dpad = 64 c + 32
    const int total = nsteps * nk;

    // Copies of a stage (step t, unit u): wave w brings database row block w
    // of the step (two 1 KB halves of its 2 KB unit) and query block w (rows
    // 32 w + 16 r + lane % 16, the lane's 16 bytes at column 8 (lane / 16)
    // of the unit), plus, at u = 0, wave 0 the step's 256 row norms.
    // (addresses: the lane's piece of block w of step 0, of the split's first
    // tile, and of its two query rows; LDS addresses scalar)
    const int64_t xBlk = (int64_t)32 * p.dpad * ES;
    const int64_t xStep = 8 * xBlk;
    const char* xw = (const char*)p.X + rowBeg * p.dpad * ES + wave * xBlk + lane * 16;
    const char* xr = (const char*)p.X + rowBeg * p.dpad * ES + (wave & 3) * xBlk + lane * 16;
    const char* qsrc[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int row = qb * kWT + wave * 32 + r * 16 + (lane & 15);
        qsrc[r] = (const char*)p.Q + (int64_t)(row < p.nq ? row : qb * kWT) * p.dpad * ES + (lane >> 4) * 16;
    }
    const int waveS = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t dOp = lds_addr(sOp) + waveS * 2048;
    const uint32_t dXn = lds_addr(sXn);
    auto copyStage = [&](int t, int u, int buf) {
        const uint32_t dst = dOp + buf * kWideStageBytes;
        const char* xs = (2 * t + (waveS >> 2) < tiles ? xw + t * xStep : xr) + u * 2048;
        lds_copy16(xs, dst);
        lds_copy16(xs + 1024, dst + 1024);
        lds_copy16(qsrc[0] + u * 64, dst + kWideStageBytes / 2);
        lds_copy16(qsrc[1] + u * 64, dst + kWideStageBytes / 2 + 1024);
        if (PRE && u == 0 && waveS == 0) {
            const bool nv = 2 * t + (lane >= 32 ? 1 : 0) < tiles;
            lds_copy16(p.xnorm + rowBeg + (nv ? (int64_t)t * kWT + lane * 4 : (int64_t)(lane & 31) * 4),
                       dXn + (t & 1) * kWT * 4);
        }
    };

    // fragment of 32 rows (or queries) x 16 columns, step g of the stage:
    // unit piece ((r32 / 16) * 4 + 2 g + h) * 16 + r32 % 16
    const int laneOff = (r32 >> 4) * 1024 + h * 256 + (r32 & 15) * 16;
    const int aOff = wm * 2 * 2048 + laneOff;                          // + bm * 2048
    const int bOff = kWideStageBytes / 2 + wn * 4 * 2048 + laneOff;    // + bn * 2048

    fx16 acc[2][4];
    if (total > 0) copyStage(0, 0, 0);
    if (total > 1) copyStage(1 / nk, 1 % nk, 1);
    if (total > 2) copyStage(2 / nk, 2 % nk, 2);
    int ct = 3 / nk, cu = 3 % nk;   // the next stage to copy
    // Unit loop inside the step loop, the epilogue after it: the
    // accumulators' only loop-carried path is MFMA to MFMA, so they stay in
    // the accumulator registers.
    int it = 0;   // stage counter over the whole split: LDS buffer it % 4
    for (int t = 0; t < nsteps; ++t) {
        for (int u = 0; u < nk; ++u, ++it) {
            // stage it is here once this wave's copies of it are (later
            // stages' copies may stay in flight) and every wave's are: the
            // barrier; after it, every wave is done with stage it - 1, whose
            // buffer the copy of stage it + 3 takes (issued below)
            const int after = total - 1 - it;
            if (after >= 2)
                wide_sync<8>();
            else if (after == 1)
                wide_sync<4>();
            else
                wide_sync<0>();
            const char* st = sOp + (it & 3) * kWideStageBytes;
            if (PRE && u == 0) {
                // acc[bm][0] = -||x||^2 / 2 of the lane's rows (register 4 g4 + i:
                // row wm * 64 + bm * 32 + 8 g4 + 4 h + i), the C operand of the
                // step's first MFMAs
#pragma unroll
                for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                    for (int g4 = 0; g4 < 4; ++g4) {
                        const fx4 v = *(const fx4*)(sXn + (t & 1) * kWT + wm * 64 + bm * 32 + g4 * 8 + h * 4);
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[bm][0][g4 * 4 + i] = v[i] * -0.5f;
                    }
            }
            auto mma = [&](auto zeroTag) {
                constexpr bool ZERO = decltype(zeroTag)::value;
                const fx16 z = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f,
                                0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int g = 0; g < 2; ++g) {
                    fx4 a[2], b[4];
#pragma unroll
                    for (int j = 0; j < 2; ++j) a[j] = *(const fx4*)(st + aOff + j * 2048 + g * 512);
#pragma unroll
                    for (int j = 0; j < 4; ++j) b[j] = *(const fx4*)(st + bOff + j * 2048 + g * 512);
                    const bool zc = ZERO && g == 0;
#pragma unroll
                    for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                        for (int bn = 3; bn >= 0; --bn)
                            acc[bm][bn] = mfma32x32x16<S>(a[bm], b[bn], zc ? (PRE ? acc[bm][0] : z) : acc[bm][bn]);
                    // the copy of stage it + 3 (into stage it - 1's buffer, free
                    // since the barrier) after the first step's MFMAs: the
                    // fragment reads go first
                    if (g == 0 && it + 3 < total) {
                        copyStage(ct, cu, (it + 3) & 3);
                        if (++cu == nk) {
                            cu = 0;
                            ++ct;
                        }
                    }
                }
            };
            if (u == 0)
                mma(std::true_type{});
            else
                mma(std::false_type{});
            if (halfTail && u == nk - 1) {   // scan_filter's zero half-chunk: acc + 0
                const fx4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int g = 0; g < 2; ++g)
#pragma unroll
                    for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                        for (int bn = 3; bn >= 0; --bn) acc[bm][bn] = mfma32x32x16<S>(z4, z4, acc[bm][bn]);
            }
        }
        // the step's epilogue: keys, bound test, survivors
        const int64_t row0 = rowBeg + (int64_t)t * kWT;
#pragma unroll
        for (int bm = 0; bm < 2; ++bm) {
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int64_t r0 = row0 + wm * 64 + bm * 32 + g4 * 8 + h * 4;
                const fx4 xn4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int bp = 0; bp < 2; ++bp) {
                    // one group at a time: nothing of the next is
                    // hoisted into this one's register budget
                    __builtin_amdgcn_sched_barrier(0);
                    filter_group<METRIC, PASS, 4, 2, true, true, PRE>(
                        acc[bm], g4, 2 * bp, xn4, r0, rowLim, p.id_stride, idb, p, tk, ti, qn, ft, qv,
                        QTab{sLTk + wn * 128, sLTi + wn * 128, sLQn + wn * 128, r32}, [&](int bn, float key, int id) {
                            const int ql = wn * 128 + bn * 32 + r32;
                            const int q = qb * kWT + ql;
                            const uint2 v = make_uint2(__float_as_uint(key), (unsigned)id);
                            if (PASS == kPassRetry && p.qcnt) {   // pooled region of the query
                                const int gs = atomicAdd(&p.qcnt[(int64_t)q * kPoolCntStride], 1);
                                if (gs < p.qcap[q]) p.cand[p.qoff[q] + gs] = v;
                                return;
                            }
                            const int slot = atomicAdd(&sCnt[ql], 1);
                            if (slot < p.cap) p.cand[((int64_t)q * p.nsplit + split) * p.cap + slot] = v;
                        });
                }
            }
        }
    }
    __syncthreads();   // every epilogue's slot counts
    if (!(PASS == kPassRetry && p.qcnt) && tid < kWT) {
        const int q = qb * kWT + tid;
        if (q < nqv) p.cnt[(int64_t)q * p.nsplit + split] = sCnt[tid];
    }
}

// ---------------------------------------------------------------------------
// scan_resident: query tile resident in LDS, database streamed per wave
// ---------------------------------------------------------------------------
//
// For batches of more than 64 queries whose 128-query tile fits in LDS (fp32
// dpad <= 128, fp16/bf16 dpad <= 256). A workgroup owns one query block and
// one split, as in scan_filter, but stages only the queries, once: they stay
// in LDS for the workgroup's lifetime as the MFMA B operand. Each wave then
// walks 64-row slices of the split on its own (slices w, w + 4, ...), loading
// its A operand straight from the chunked database layout into registers, so
// the main loop has no barriers and no LDS writes. A wave computes 64 rows x
// 128 queries per slice as 2 x 4 blocks of 32 x 32 (v_mfma_f32_32x32x2_f32 or
// v_mfma_f32_32x32x16_{f16,bf16}); lane l holds rows 8*(r/4) + 4*(l/32) +
// (r%4) of query l%32 of each block, as in scan_filter, whose filter epilogue
// this kernel shares.
// Operand pieces (16 bytes, lane half h = l/32, row r32 = l%32):
//   fp32, 8-column group g of a chunk: columns 8g + 4h .. +3 (MFMA step j
//         pairs columns 8g + j and 8g + 4 + j), chunk piece
//         ((r32/16)*2 + h)*64 + g*16 + r32%16 of blk_off's order;
//   fp16/bf16, 16-column step s: columns 16s + 8h .. +7, chunk piece
//         ((r32/16)*4 + 2s + h)*16 + r32%16 of blk_off_h's order.
// G > 0 (fp16/bf16, dpad = 32 G <= 128): a whole slice is buffered in
// registers and each chunk slot is refilled with the next slice's chunk as
// soon as its MFMAs are issued (about one slice of prefetch: the fp16 MFMAs
// consume a chunk in ~512 cycles, far less than a memory round trip). G == 0: one chunk
// of prefetch (fp32, whose chunk takes ~8k cycles of MFMA, and larger dpad).
// Prefetches are issued unconditionally (the last slice re-reads itself) so
// every wait on them is a static count. Database loads are ordinary (cached):
// the workgroups of up to kQGroup query blocks resident on one XCD read the
// same split at about the same time and share it through that XCD's L2 (a
// non-temporal hint here cost 7% at d = 128 fp32 and 16% with fp16 storage).
// IVF: the fine scan of an inverted-file index. A workgroup owns one work item
// (a cell and up to kBN of the (query, probe rank) entries that probe it): its
// query tile is gathered from the entries' query rows, its rows are the cell's
// (padded to kBM in the database), filter ids are cell-relative rows plus the
// entry's scan position, and survivors go to the entry's region
// (query * ivf_nreg + rank). Work items are in decreasing cell size, so the
// largest run first.
template <int S, int METRIC, int PASS, int G, bool IVF, int NB>
__global__ void __launch_bounds__(256, 2) scan_resident_kernel(ScanParams p) {
    constexpr int TQ = 32 * NB;                    // queries per tile (NB blocks of 32)
    constexpr int ES = S == kF32 ? 4 : 2;
    constexpr int NK = S == kF32 ? 4 : 2;          // operand pieces per row block per chunk
    constexpr int KSTEP = S == kF32 ? 256 : 512;   // byte step between a lane's pieces in a chunk
    constexpr int CB = 32 * 32 * ES;               // bytes per 32 x 32 chunk
    // fp16/bf16: the filter's group test through maxima (MAXT) and, for L2,
    // accumulators started from -||x||^2 / 2 (PRE); see filter_group
    constexpr bool MAXT = S != kF32;
    constexpr bool PRE = S != kF32 && METRIC == 0;
    extern __shared__ __attribute__((aligned(16))) float sQr[];   // [TQ][dpad + 16 / ES] elements
    __shared__ __attribute__((aligned(16))) float sXn[4 * 64];    // per wave: its slice's row norms
    __shared__ int sCnt[TQ];
    __shared__ unsigned long long sBest[TQ];
    // Per-wave survivor ring (fp32 full pass): (key, id, query) staged in LDS
    // and written to the candidate regions half a ring at a time, so the next
    // slices' prefetch waits rarely wait on survivor stores (1.4% at C2). The
    // fp16/bf16 instantiations hold a whole slice of operands in registers
    // and lose more to the extra register pressure.
    constexpr bool RING = S == kF32 && PASS == kPassFull;
    __shared__ uint32_t sRingKey[RING ? 4 * kRing : 1];
    __shared__ int sRingId[RING ? 4 * kRing : 1];
    __shared__ int sRingQ[RING ? 4 * kRing : 1];
    __shared__ int sRingN[4];
    // Flat retry pass (pooled regions, one global slot counter per query):
    // survivors staged in LDS with a slot among the workgroup's own for their
    // query (sCnt); at the end one global atomic per query reserves the
    // workgroup's block of slots (in sBest's storage) and the staged entries
    // are written there (one atomic per survivor on counters shared by every
    // workgroup: C2 fp16's retry pass 250 -> 193 us); beyond kStage a
    // survivor takes a slot of its own. (Entry: key bits and id; tag: slot
    // << 8 | query slot.)
    constexpr bool STAGE = PASS == kPassRetry && !IVF;
    constexpr int kStage = 768;   // 9 KB, the ring's LDS in the other passes
    __shared__ uint2 sStage[STAGE ? kStage : 1];
    __shared__ uint32_t sStageTag[STAGE ? kStage : 1];
    __shared__ int sStageN;
    // fp16/bf16 (a whole slice of operands in registers): survivor-only query
    // state in LDS (filter_group's LQ), not registers
    constexpr bool LQ = S != kF32 && PASS != kPassArgmin;
    __shared__ float sLTk[LQ ? TQ : 1];
    __shared__ int sLTi[LQ ? TQ : 1];
    __shared__ float sLQn[LQ ? TQ : 1];
    __shared__ int sEnt[IVF ? TQ : 1];   // IVF: the tile's entries (-1: empty slot)
    __shared__ int sQi[IVF ? TQ : 1];    // ... their queries
    __shared__ int sReg[IVF ? TQ : 1];   // ... their candidate regions

    int qb = 0, split = 0;
    int4 wk = make_int4(0, 0, 0, 0);   // IVF work item: (cell, first entry, entries, 0)
    if constexpr (IVF) {
        if ((int)blockIdx.x >= *p.ivf_nwork) return;
        wk = p.ivf_work[blockIdx.x];
    } else {
        // Workgroup -> (query block, split): the XCD grouping of scan_filter.
        const int nwg = gridDim.x;
        const int bid = blockIdx.x;
        if (PASS == kPassRetry && p.nq_dev) {
            // A device-sized retry covers more query blocks than it usually
            // fills: block-major order dispatches the live blocks' splits
            // first, over every XCD, and the idle blocks trail.
            qb = bid / p.nsplit;
            split = bid - qb * p.nsplit;
        } else {
            const int full = (nwg / 8) * 8;
            const int v = bid < full ? (bid % 8) * (full / 8) + bid / 8 : bid;
            const int qgrp = p.qgroup > 0 ? p.qgroup : kQGroup;
            const int grpSize = p.nqb < qgrp ? p.nqb : qgrp;
            const int grp = v / (grpSize * p.nsplit);
            const int r = v - grp * grpSize * p.nsplit;
            const int inGrp = p.nqb - grp * grpSize < grpSize ? p.nqb - grp * grpSize : grpSize;
            split = r / inGrp;
            qb = grp * grpSize + (r - split * inGrp);
        }
    }
    // A retry whose work list the device built: query blocks beyond it are idle.
    const int nqv = (PASS == kPassRetry && p.nq_dev) ? *p.nq_dev : p.nq;
    if (!IVF && qb * TQ >= nqv) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r32 = lane & 31;
    const int h = lane >> 5;
    const int ldqB = (p.dpad + 16 / ES) * ES;   // LDS query row stride (bytes): 16 B of padding

    if constexpr (IVF) {
        if (tid < TQ) {
            const int e = tid < wk.z ? p.ivf_ent[wk.y + tid] : -1;
            const int q = e >= 0 ? e / p.ivf_nprobe : -1;
            sEnt[tid] = e;
            sQi[tid] = q;
            sReg[tid] = e >= 0 ? q * p.ivf_nreg + (e - q * p.ivf_nprobe) : -1;
        }
        __syncthreads();
    }
    {
        const int rowP = p.dpad * ES / 16;
        const fx4* qg = (const fx4*)p.Q + (int64_t)qb * TQ * rowP;
        // eight 16-byte pieces per thread in flight (a work item of the IVF
        // scan is short enough for serial load latencies here to show)
        const int npc = TQ * rowP;
        for (int i0 = tid; i0 < npc; i0 += 8 * 256) {
            fx4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = i0 + u * 256;
                v[u] = fx4{0.0f, 0.0f, 0.0f, 0.0f};
                if (i < npc) {
                    const int row = i / rowP;
                    const int c = i - row * rowP;
                    if constexpr (IVF) {
                        const int q = sQi[row];
                        if (q >= 0) v[u] = ((const fx4*)p.Q)[(int64_t)q * rowP + c];
                    } else {
                        v[u] = qg[(int64_t)row * rowP + c];
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = i0 + u * 256;
                if (i < npc) {
                    const int row = i / rowP;
                    *(fx4*)((char*)sQr + row * ldqB + (i - row * rowP) * 16) = v[u];
                }
            }
        }
    }
    if (tid < TQ) {
        sCnt[tid] = 0;
        sBest[tid] = ~0ull;
    }
    if (tid < 4) sRingN[tid] = 0;
    if (tid == 0) sStageN = 0;

    // Per-lane query state for its NB query blocks; bounds as in scan_filter.
    float tk[NB], qn[NB], ft[NB];
    int ti[NB];
    bool qv[NB];
    int idb[NB] = {};   // IVF: scan position of the cell's first row, per slot
#pragma unroll
    for (int bn = 0; bn < NB; ++bn) {
        int q;
        if constexpr (IVF) {
            q = sQi[bn * 32 + r32];
            qv[bn] = q >= 0;
            if (qv[bn]) idb[bn] = p.ivf_pos[sEnt[bn * 32 + r32]];
        } else {
            q = qb * TQ + bn * 32 + r32;
            qv[bn] = q < nqv;
        }
        if (PASS == kPassArgmin) {
            tk[bn] = INFINITY;
            ti[bn] = -1;
        } else {
            tk[bn] = qv[bn] ? p.tau_key[q] : 0.0f;
            ti[bn] = qv[bn] ? p.tau_id[q] : -1;
        }
        qn[bn] = (METRIC == 0 && qv[bn]) ? p.qnorm[q] : 0.0f;
        if (METRIC == 0) {
            const float m = 0x1p-20f * (tk[bn] + 2.0f * qn[bn] + 2.0f * p.xnorm_max);
            ft[bn] = qv[bn] ? (tk[bn] - qn[bn]) + m : -INFINITY;
            if (PRE) ft[bn] *= -0.5f;
        } else {
            ft[bn] = qv[bn] ? -tk[bn] : INFINITY;
        }
    }
    if constexpr (LQ) {
        if (tid < TQ) {
            int q;
            bool v;
            if constexpr (IVF) {
                q = sQi[tid];
                v = q >= 0;
            } else {
                q = qb * TQ + tid;
                v = q < nqv;
            }
            sLTk[tid] = v ? p.tau_key[q] : 0.0f;
            sLTi[tid] = v ? p.tau_id[q] : -1;
            sLQn[tid] = (METRIC == 0 && v) ? p.qnorm[q] : 0.0f;
        }
    }
    const QTab lqt{sLTk, sLTi, sLQn, r32};
    __syncthreads();

    // Rows: [rowBeg, rowBeg + 64 nsl) of the database; filter rows count from
    // rowOrg (IVF: the cell's first row), rows at or above rowLim are padding.
    int64_t rowBeg, rowOrg, rowLim;
    int nsl;
    if constexpr (IVF) {
        rowBeg = p.ivf_cell_pad[wk.x];
        rowOrg = 0;
        rowLim = p.ivf_cell_size[wk.x];
        if (p.ivf_row_cap > 0 && rowLim > p.ivf_row_cap) rowLim = p.ivf_row_cap;   // a cell's first rows only
        nsl = (int)((rowLim + 63) / 64);
    } else {
        rowBeg = split_row(p, split);
        const int64_t rowEnd = split_row(p, split + 1);
        nsl = rowEnd > rowBeg ? (int)((rowEnd - rowBeg) / 64) : 0;
        rowOrg = rowBeg;
        rowLim = p.nrows;
    }
    const int idStride = IVF ? 1 : p.id_stride;
    auto region = [&](int ql) -> int64_t {
        if constexpr (IVF) return sReg[ql];
        return ((int64_t)qb * TQ + ql) * p.nsplit + split;
    };
    // Survivor of slot ql at its region's slot `slot`. IVF with a spill region
    // (region nprobe of each query, filled by global atomics on its count): the
    // survivors beyond a region's capacity go there, so one crowded cell does
    // not force a retry; the spill's count past cap still flags the overflow.
    auto store = [&](int ql, int slot, uint2 v) {
        if constexpr (PASS == kPassRetry && !IVF) {
            if (p.qcnt) {   // pooled region of the query (global slot counter)
                const int q = qb * TQ + ql;
                const int gs = atomicAdd(&p.qcnt[(int64_t)q * kPoolCntStride], 1);
                if (gs < p.qcap[q]) p.cand[p.qoff[q] + gs] = v;
                return;
            }
        }
        if (slot < p.cap) {
            p.cand[region(ql) * p.cap + slot] = v;
        } else if constexpr (IVF) {
            if (p.ivf_spill) {
                const int64_t sr = (int64_t)sQi[ql] * p.ivf_nreg + p.ivf_nprobe;
                const int sp = atomicAdd(&p.cnt[sr], 1);
                if (sp < p.cap) p.cand[sr * p.cap + sp] = v;
            }
        }
    };
    const int nchunk = p.dpad / 32;
    const int64_t blkB = (int64_t)32 * p.dpad * ES;
    const char* xw = (const char*)p.X + rowBeg * p.dpad * ES +
                     (S == kF32 ? ((r32 >> 4) * 2 + h) * 1024 : ((r32 >> 4) * 4 + h) * 256) + (r32 & 15) * 16;
    const char* qlds = (const char*)sQr + r32 * ldqB + h * 16;
    auto lda = [&](int sl, int bm, int t, int k) -> fx4 {
        return *(const fx4*)(xw + (int64_t)(2 * sl + bm) * blkB + t * CB + k * KSTEP);
    };
    auto ldb = [&](int bn, int t, int k) -> fx4 {
        return *(const fx4*)(qlds + bn * 32 * ldqB + t * 32 * ES + k * 32);
    };

    fx16 acc[2][NB];
    // One chunk of MFMAs from operand pieces a[bm][k]; a slice's first chunk
    // starts every accumulator from an inline zero.
    auto mma = [&](const fx4 (&a)[2][NK], int t, auto zeroTag) {
        constexpr bool ZERO = decltype(zeroTag)::value;
        const fx16 z = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f,
                        0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            fx4 b[NB];
#pragma unroll
            for (int bn = 0; bn < NB; ++bn) b[bn] = ldb(bn, t, k);
            if constexpr (S == kF32) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                        for (int bn = 0; bn < NB; ++bn)
                            acc[bm][bn] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                                a[bm][k][j], b[bn][j], (ZERO && k == 0 && j == 0) ? z : acc[bm][bn], 0, 0, 0);
            } else {
                // PRE: a slice's first MFMAs all start from acc[bm][0] (the
                // rows' -||x||^2 / 2, set by preInit), which is overwritten last
#pragma unroll
                for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                    for (int bn = NB - 1; bn >= 0; --bn)
                        acc[bm][bn] = mfma32x32x16<S>(a[bm][k], b[bn],
                                                      (ZERO && k == 0) ? (PRE ? acc[bm][0] : z) : acc[bm][bn]);
            }
        }
    };
    // PRE: acc[bm][0] = -||x||^2 / 2 of the rows this lane's accumulator
    // registers hold in block bm (register 4 g4 + i: row 32 bm + 8 g4 + 4 h + i
    // of the slice), staged through the wave's sXn entries.
    auto preInit = [&](float xnv) {
        if constexpr (PRE) {
            sXn[wave * 64 + lane] = -0.5f * xnv;
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const fx4 v = *(const fx4*)(sXn + wave * 64 + bm * 32 + g4 * 8 + h * 4);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[bm][0][g4 * 4 + i] = v[i];
                }
            __builtin_amdgcn_wave_barrier();
        }
    };

    // Filter epilogue of slice sl (rows rowBeg + 64 sl ..), whose row norms
    // this lane holds for row `lane` in xnv.
    auto epilogue = [&](int sl, float xnv) {
        if (METRIC == 0 && !PRE) {
            sXn[wave * 64 + lane] = xnv;
            __builtin_amdgcn_wave_barrier();
        }
#pragma unroll
        for (int bm = 0; bm < 2; ++bm) {
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int rl = bm * 32 + g4 * 8 + h * 4;
                const int64_t r0 = rowOrg + (int64_t)sl * 64 + rl;
                fx4 xn4 = {0.0f, 0.0f, 0.0f, 0.0f};
                if (METRIC == 0 && !PRE) xn4 = *(const fx4*)(sXn + wave * 64 + rl);
#pragma unroll
                for (int bp = 0; bp < (NB + 1) / 2; ++bp)
                    filter_group<METRIC, PASS, NB, NB == 1 ? 1 : 2, LQ, MAXT, PRE>(acc[bm], g4, 2 * bp, xn4, r0, rowLim,
                                                                         idStride, idb, p, tk, ti, qn, ft, qv, lqt,
                                                  [&](int bn, float key, int id) {
                        const int ql = bn * 32 + r32;
                        if constexpr (STAGE) {
                            if (p.qcnt) {
                                const uint2 v = make_uint2(__float_as_uint(key), (unsigned)id);
                                const int e = atomicAdd(&sStageN, 1);
                                if (e < kStage) {
                                    sStage[e] = v;
                                    sStageTag[e] = ((uint32_t)atomicAdd(&sCnt[ql], 1) << 8) | (uint32_t)ql;
                                } else {
                                    store(ql, 0, v);   // a global slot of its own
                                }
                                return;
                            }
                        }
                        const int pos = RING ? atomicAdd(&sRingN[wave], 1) : kRing;
                        if (pos < kRing) {
                            sRingKey[wave * kRing + pos] = __float_as_uint(key);
                            sRingId[wave * kRing + pos] = id;
                            sRingQ[wave * kRing + pos] = ql;
                        } else {   // ring full (or not used): store directly
                            store(ql, atomicAdd(&sCnt[ql], 1), make_uint2(__float_as_uint(key), (unsigned)id));
                        }
                    });
            }
        }
    };

    // fp16/bf16: a workgroup-uniform base and a 32-bit lane offset (one
    // address register, not a 64-bit pair held across the slice loop, which
    // the G = 4 instantiations would spill and reload in the loop)
    const float* xnw = p.xnorm + rowBeg;
    auto norm = [&](int sl) -> float {
        if constexpr (S == kF32) return METRIC == 0 ? p.xnorm[rowBeg + (int64_t)sl * 64 + lane] : 0.0f;
        return METRIC == 0 ? xnw[sl * 64 + lane] : 0.0f;
    };

    // Writes the wave's staged survivors to their candidate regions once at
    // least `atLeast` are staged (atLeast = 1: at the end).
    auto flush = [&](int atLeast) {
        if constexpr (RING) {
            __builtin_amdgcn_wave_barrier();
            const int n0 = sRingN[wave];
            const int n = n0 < kRing ? n0 : kRing;
            if (n < atLeast) return;
            for (int e = lane; e < n; e += 64) {
                const int ql = sRingQ[wave * kRing + e];
                store(ql, atomicAdd(&sCnt[ql], 1),
                      make_uint2(sRingKey[wave * kRing + e], (unsigned)sRingId[wave * kRing + e]));
            }
            __builtin_amdgcn_wave_barrier();
            if (lane == 0) sRingN[wave] = 0;
            __builtin_amdgcn_wave_barrier();
        }
    };

    if constexpr (G > 0) {
        fx4 buf[G][2][NK];
        float xnv = 0.0f;
        if (wave < nsl) {
            xnv = norm(wave);
#pragma unroll
            for (int t = 0; t < G; ++t)
#pragma unroll
                for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                    for (int k = 0; k < NK; ++k) buf[t][bm][k] = lda(wave, bm, t, k);
        }
        for (int sl = wave; sl < nsl; sl += 4) {
            const int nx = sl + 4 < nsl ? sl + 4 : sl;
            const float xnNext = norm(nx);
            preInit(xnv);
#pragma unroll
            for (int t = 0; t < G; ++t) {
                if (t == 0) mma(buf[t], t, std::true_type{});
                else mma(buf[t], t, std::false_type{});
#pragma unroll
                for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                    for (int k = 0; k < NK; ++k) buf[t][bm][k] = lda(nx, bm, t, k);
                // issue the refill here, not after the last chunk's MFMAs
                // (where the scheduler otherwise sinks it to reuse buf[t]'s
                // registers for the next chunk's query fragments)
                __builtin_amdgcn_sched_barrier(0);
            }
            epilogue(sl, xnv);
            flush(kRing / 2);
            xnv = xnNext;
        }
    } else {
        fx4 cur[2][NK];
        float xnv = 0.0f;
        if (wave < nsl) {
            xnv = norm(wave);
#pragma unroll
            for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                for (int k = 0; k < NK; ++k) cur[bm][k] = lda(wave, bm, 0, k);
        }
        for (int sl = wave; sl < nsl; sl += 4) {
            const int nxs = sl + 4 < nsl ? sl + 4 : sl;
            const float xnNext = norm(nxs);
            preInit(xnv);
            for (int t = 0; t < nchunk; ++t) {
                const bool lastT = t + 1 == nchunk;
                const int ns = lastT ? nxs : sl;
                const int ntc = lastT ? 0 : t + 1;
                fx4 nxt[2][NK];
#pragma unroll
                for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                    for (int k = 0; k < NK; ++k) nxt[bm][k] = lda(ns, bm, ntc, k);
                if (t == 0) mma(cur, t, std::true_type{});
                else mma(cur, t, std::false_type{});
#pragma unroll
                for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                    for (int k = 0; k < NK; ++k) cur[bm][k] = nxt[bm][k];
            }
            epilogue(sl, xnv);
            flush(kRing / 2);
            xnv = xnNext;
        }
    }

    flush(1);
    if (PASS == kPassArgmin) {
#pragma unroll
        for (int bn = 0; bn < NB; ++bn)
            if (ti[bn] >= 0)
                atomicMin(&sBest[bn * 32 + r32],
                          ((unsigned long long)key_to_ord(__float_as_uint(tk[bn])) << 32) | (unsigned)ti[bn]);
        __syncthreads();
        if (tid < TQ) {
            const int q = qb * TQ + tid;
            if (q < p.nq && sBest[tid] != ~0ull) atomicMin(&p.best[q], sBest[tid]);
        }
        return;
    }
    __syncthreads();
    if constexpr (STAGE) {
        if (p.qcnt) {
            int* sBase = reinterpret_cast<int*>(sBest);
            if (tid < TQ) {
                const int q = qb * TQ + tid;
                sBase[tid] = sCnt[tid] > 0 ? atomicAdd(&p.qcnt[(int64_t)q * kPoolCntStride], sCnt[tid]) : 0;
            }
            __syncthreads();
            const int n = sStageN < kStage ? sStageN : kStage;
            for (int e = tid; e < n; e += 256) {
                const uint32_t tag = sStageTag[e];
                const int ql = (int)(tag & 255u);
                const int q = qb * TQ + ql;
                const int gs = sBase[ql] + (int)(tag >> 8);
                if (gs < p.qcap[q]) p.cand[p.qoff[q] + gs] = sStage[e];
            }
            return;
        }
    }
    if constexpr (IVF) {
        if (tid < wk.z) p.cnt[sReg[tid]] = p.ivf_spill && sCnt[tid] > p.cap ? p.cap : sCnt[tid];
    } else if (tid < TQ) {
        const int q = qb * TQ + tid;
        if (q < nqv && !(PASS == kPassRetry && p.qcnt)) p.cnt[(int64_t)q * p.nsplit + split] = sCnt[tid];
    }
}

// ---------------------------------------------------------------------------
// scan_small: the same filter for small batches (nq <= 64), HBM-streaming
// ---------------------------------------------------------------------------
//
// With few queries every database byte is used by at most 64 queries, so the
// pass is bound by reading the database once from HBM, not by MFMA. The
// database rows go straight from global memory into the A operand of
// v_mfma_f32_16x16x4_f32 (fp32) or v_mfma_f32_16x16x32_{f16,bf16} (no LDS
// staging: each row is used by one wave only); the queries, NQB blocks of 16,
// sit in LDS as the B operand. Output layout: lane l holds query l%16 of the
// block and rows 4*(l/16) .. +3, so the epilogue keeps the per-query bound in
// a register as in scan_filter.
// K is consumed 32 columns (one chunk) at a time: lane quarter q = l/16 holds
// columns 32t + 8q .. +7 of its row -- fp32 as two float4 pieces e, MFMA j
// pairing column 32t + 8q + j across the quarters; fp16/bf16 as one 16-byte
// piece, one MFMA per chunk -- the same permutation on both operands.
// One workgroup per split.
// G > 0: dpad == 32 G, and a whole 32-row block is buffered in registers
// (the next block's step t is fetched as soon as step t of the current block is
// consumed), which keeps G pieces per lane in flight. G == 0: any dpad, one
// step of prefetch.
template <int S, int METRIC, int NQB, int PASS, int G, int KT>
__global__ void __launch_bounds__(256) scan_small_kernel(ScanParams p) {
    constexpr int ES = S == kF32 ? 4 : 2;
    constexpr int U = S == kF32 ? 2 : 1;      // 16-byte pieces per row half per chunk
    constexpr int PAD = 16 / ES;              // LDS row padding (elements)
    static_assert(KT == 0 || (NQB == 1 && PASS == kPassFull), "top-k mode: one block of 16 queries, full pass");
    extern __shared__ __attribute__((aligned(16))) float sQs[];   // [16*NQB][dpad + PAD] elements
    __shared__ int sCnt[16 * NQB];
    // Top-k mode (KT > 0): each wave's exact top-k (k = p.cap <= KT) of the
    // rows it scanned, per query, as ascending composites (ordered key << 32
    // | id); the list's k-th is the wave's bound for that query.
    __shared__ uint64_t sList[KT > 0 ? 4 * 16 * KT : 1];
    __shared__ int sLen[KT > 0 ? 4 * 16 : 1];
    // ... and the workgroup's best bound per query: the smallest k-th entry of
    // a full wave list (k rows at or below it exist, so no row above it is a
    // result); every wave filters with it once it beats the wave's own.
    __shared__ unsigned long long sBound[KT > 0 ? 16 : 1];
    __shared__ float sQn[KT > 0 ? 16 : 1];    // fused preparation: query norms ...
    __shared__ float sInv[KT > 0 ? 16 : 1];   // ... and Cosine scale factors

    const int split = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r16 = lane & 15;
    const int quarter = lane >> 4;
    const int ldqB = (p.dpad + PAD) * ES;     // LDS query row stride, bytes
    const int rowP = p.dpad * ES / 16;        // 16-byte pieces per query row
    // a retry whose work list the device built: nothing to do when it is empty
    const int nqv = (PASS == kPassRetry && p.nq_dev) ? *p.nq_dev : p.nq;
    if (nqv <= 0) return;
    constexpr bool kPoolable = PASS == kPassRetry;

    // Top-k mode with raw queries: prep_queries' rules, per workgroup: Cosine
    // rows scaled by float(1 / sqrt(s)) (s: sequential double sum of the
    // squares), values rounded to the storage type, L2 norms the sequential
    // double sum of the stored values' squares. The sums run on lanes 0..15,
    // one query each.
    const bool fused = KT > 0 && p.qraw != nullptr;
    if (fused) {
        constexpr int PE = S == kF32 ? 4 : 8;
        if (p.qcos) {
            if (tid < 16) {
                float inv = 1.0f;
                if (tid < p.nq) {
                    const float* row = p.qraw + (int64_t)tid * p.qdim;
                    double sum = 0.0;
                    for (int c = 0; c < p.qdim; ++c) sum += (double)row[c] * row[c];
                    if (sum > 0.0) inv = (float)(1.0 / sqrt(sum));
                }
                sInv[tid] = inv;
            }
            __syncthreads();
        }
        for (int i = tid; i < 16 * rowP; i += 256) {
            const int row = i / rowP;
            const int u = i - row * rowP;
            const bool live = row < p.nq;
            const float* src = p.qraw + (int64_t)(live ? row : 0) * p.qdim;
            float v[PE];
#pragma unroll
            for (int e = 0; e < PE; ++e) {
                const int c = u * PE + e;
                float x = live && c < p.qdim ? src[c] : 0.0f;
                if (p.qcos) x *= sInv[row];
                if constexpr (S != kF32) x = from_bits<S>(to_bits<S>(x));
                v[e] = x;
            }
            fx4 piece;
            if constexpr (S == kF32) {
                piece = fx4{v[0], v[1], v[2], v[3]};
            } else {
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    piece[w] = __uint_as_float((uint32_t)to_bits<S>(v[2 * w]) | ((uint32_t)to_bits<S>(v[2 * w + 1]) << 16));
            }
            *(fx4*)((char*)sQs + row * ldqB + u * 16) = piece;
        }
        if (METRIC == 0) {
            __syncthreads();
            if (tid < 16) {
                double nrm = 0.0;
                if (tid < p.nq) {
                    const char* rb = (const char*)sQs + tid * ldqB;
                    for (int c = 0; c < p.qdim; ++c) {
                        float x;
                        if constexpr (S == kF32) x = ((const float*)rb)[c];
                        else x = from_bits<S>(((const uint16_t*)rb)[c]);
                        nrm += (double)x * x;
                    }
                }
                sQn[tid] = (float)nrm;
            }
        }
        __syncthreads();
    } else {
        for (int i = tid; i < 16 * NQB * rowP; i += 256) {
            const int row = i / rowP;
            const int c = i - row * rowP;
            *(fx4*)((char*)sQs + row * ldqB + c * 16) = *((const fx4*)p.Q + (int64_t)row * rowP + c);
        }
    }
    if (tid < 16 * NQB) sCnt[tid] = 0;
    if (KT > 0 && tid < 4 * 16) sLen[tid] = 0;
    if (KT > 0 && tid < 16) sBound[tid] = ~0ull;

    float tk[NQB], qn[NQB], ft[NQB];
    int ti[NQB];
    bool qv[NQB];
#pragma unroll
    for (int bq = 0; bq < NQB; ++bq) {
        const int q = bq * 16 + r16;
        qv[bq] = q < nqv;
        // top-k mode starts from "no bound" (+inf, -1) in every wave
        tk[bq] = qv[bq] ? (KT > 0 ? INFINITY : p.tau_key[q]) : 0.0f;
        ti[bq] = qv[bq] ? (KT > 0 ? -1 : p.tau_id[q]) : -1;
        qn[bq] = (METRIC == 0 && qv[bq]) ? (fused ? sQn[q] : p.qnorm[q]) : 0.0f;
        if (METRIC == 0) {
            const float m = 0x1p-20f * (tk[bq] + 2.0f * qn[bq] + 2.0f * p.xnorm_max);
            ft[bq] = qv[bq] ? (tk[bq] - qn[bq]) + m : -INFINITY;
        } else {
            ft[bq] = qv[bq] ? -tk[bq] : INFINITY;
        }
    }
    __syncthreads();

    const int64_t rowBeg = split_row(p, split);
    const int64_t rowEnd = split_row(p, split + 1);
    // Each wave takes 32-row blocks (two 16-row MFMA sets) round-robin. In the
    // chunked layout, the operand piece e of row half hh for chunk t is one
    // linear 1 KB load per wave: lane l reads piece l of sub-chunk (hh, e),
    // i.e. row 16 hh + (l & 15), columns 32 t + 8 (l >> 4) (+ 4 e for fp32).
    // Rows are read exactly once: non-temporal loads keep them from displacing
    // the query tile and the candidate lines in the caches.
    const int nblk = rowEnd > rowBeg ? (int)((rowEnd - rowBeg) / 32) : 0;
    const int g32 = p.dpad / 32;
    const int64_t blkStride = (int64_t)32 * p.dpad * ES;   // bytes
    const char* xw = (const char*)p.X + rowBeg * p.dpad * ES + lane * 16;
    const char* qrow8 = (const char*)sQs + r16 * ldqB + quarter * 8 * ES;
    auto ld = [&](int b, int t, int hh, int e) -> fx4 {
        return __builtin_nontemporal_load((const fx4*)(xw + b * blkStride + t * (U * 2048) + (hh * U + e) * 1024));
    };

    constexpr int GB = G > 0 ? G : 1;
    fx4 buf[2][GB][U];   // G > 0: the wave's whole current block [row half][step][e]
    fx4 cur[2][U];       // G == 0: the current step
    if (wave < nblk) {
        if constexpr (G > 0) {
#pragma unroll
            for (int t = 0; t < GB; ++t)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int e = 0; e < U; ++e) buf[hh][t][e] = ld(wave, t, hh, e);
        } else {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int e = 0; e < U; ++e) cur[hh][e] = ld(wave, 0, hh, e);
        }
    }
    // One 32-row block of the wave. NEXT: whether block b + 4 exists and is
    // prefetched. The last block of a wave is a separate instantiation, so
    // the prefetch of every other block is unconditional: with a branch
    // around it the compiler's wait for the row norms has to fit both paths
    // and waits for the prefetch as well.
    // Top-k mode: the block's candidates of this lane (rows r0 + i of both
    // row halves, query r16) go into the wave's list of query r16. The four
    // lane quarters holding the same query insert one after another, so each
    // list has one writer at a time; an insertion re-checks against the
    // list's current k-th. Afterwards every lane re-reads its query's bound.
    const int kk = p.cap;
    // Bound of query slot 0 from a composite (ordered key << 32 | id).
    auto setBound = [&](uint64_t x) {
        tk[0] = ord_to_key((uint32_t)(x >> 32));
        ti[0] = (int)(uint32_t)(x & 0xFFFFFFFFu);
        if (METRIC == 0) {
            const float m = 0x1p-20f * (tk[0] + 2.0f * qn[0] + 2.0f * p.xnorm_max);
            ft[0] = (tk[0] - qn[0]) + m;
        } else {
            ft[0] = -tk[0];
        }
    };
    auto topk_block = [&](const fx4 (&acc)[2][NQB], const fx4 (&xnh)[2], const int b) {
        if (qv[0]) {   // another wave's tighter bound
            const uint64_t sb = sBound[r16];
            if (sb < ((uint64_t)key_to_ord(__float_as_uint(tk[0])) << 32 | (uint32_t)ti[0])) setBound(sb);
        }
        uint64_t cc[2][4];
        bool has = false;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int64_t r0 = rowBeg + (int64_t)b * 32 + hh * 16 + quarter * 4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float dot = acc[hh][0][i];
                const bool f = METRIC == 0 ? fmaf(-2.0f, dot, xnh[hh][i]) <= ft[0] : dot >= ft[0];
                cc[hh][i] = ~0ull;
                if (f) {
                    const int64_t row = r0 + i;
                    float key;
                    if (METRIC == 0) {
                        const float tt = fmaf(-2.0f, dot, qn[0] + xnh[hh][i]);
                        key = (tt < 0.0f ? 0.0f : tt) + 0.0f;
                    } else {
                        key = -dot + 0.0f;
                    }
                    const int id = (int)(row * p.id_stride);
                    // +inf and NaN keys are never results ("no bound" rejects them)
                    if (row < p.nrows && qv[0] && key < INFINITY &&
                        (key < tk[0] || (key == tk[0] && id < ti[0]))) {
                        cc[hh][i] = ((uint64_t)key_to_ord(__float_as_uint(key)) << 32) | (uint32_t)id;
                        has = true;
                    }
                }
            }
        }
        if (!__any(has)) return;
        uint64_t* L = sList + (wave * 16 + r16) * KT;
        int* len = sLen + wave * 16 + r16;
        for (int qt = 0; qt < 4; ++qt) {
            if (quarter == qt && has) {
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint64_t c = cc[hh][i];
                        if (c == ~0ull) continue;
                        const int n = *len;
                        if (n == kk && c >= L[kk - 1]) continue;
                        int j = n == kk ? kk - 1 : n;
                        while (j > 0 && L[j - 1] > c) {
                            L[j] = L[j - 1];
                            --j;
                        }
                        L[j] = c;
                        if (n < kk) *len = n + 1;
                    }
            }
            __builtin_amdgcn_wave_barrier();
        }
        if (*len == kk && qv[0]) {
            const uint64_t x = L[kk - 1];
            const uint64_t sb = sBound[r16];
            if (x < sb) {
                if (quarter == 0) atomicMin(&sBound[r16], (unsigned long long)x);
                setBound(x);
            } else {
                setBound(sb);
            }
        }
    };

    auto block = [&](const int b, auto nextTag) {
        constexpr bool NEXT = decltype(nextTag)::value;
        // The block's row norms are loaded BEFORE the next block's prefetch:
        // vector-memory loads complete in order, so waiting for norms loaded
        // after the prefetch would wait for the whole prefetch too.
        fx4 xnh[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
        if (METRIC == 0) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
                xnh[hh] = *(const fx4*)(p.xnorm + rowBeg + (int64_t)b * 32 + hh * 16 + quarter * 4);
        }
        fx4 acc[2][NQB];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int bq = 0; bq < NQB; ++bq) acc[hh][bq] = fx4{0.0f, 0.0f, 0.0f, 0.0f};
        auto step = [&](const fx4 (&x)[2][U], int t) {
#pragma unroll
            for (int bq = 0; bq < NQB; ++bq) {
                const char* qp = qrow8 + bq * 16 * ldqB + t * 32 * ES;
                if constexpr (S == kF32) {
                    const fx4 bv0 = *(const fx4*)qp;
                    const fx4 bv1 = *(const fx4*)(qp + 16);
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float bj = j < 4 ? bv0[j & 3] : bv1[j & 3];
                        acc[0][bq] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[0][j >> 2][j & 3], bj, acc[0][bq], 0, 0, 0);
                        acc[1][bq] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[1][j >> 2][j & 3], bj, acc[1][bq], 0, 0, 0);
                    }
                } else {
                    const fx4 bv = *(const fx4*)qp;
                    acc[0][bq] = mfma16x16x32<S>(x[0][0], bv, acc[0][bq]);
                    acc[1][bq] = mfma16x16x32<S>(x[1][0], bv, acc[1][bq]);
                }
            }
        };
        if constexpr (G > 0) {
#pragma unroll
            for (int t = 0; t < GB; ++t) {
                fx4 x[2][U];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int e = 0; e < U; ++e) x[hh][e] = buf[hh][t][e];
                if constexpr (NEXT) {
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                        for (int e = 0; e < U; ++e) buf[hh][t][e] = ld(b + 4, t, hh, e);
                }
                // Keeps the prefetch of step t issued before step t's MFMAs
                // (left alone, the scheduler sinks all of it to the block end).
                __builtin_amdgcn_sched_barrier(0);
                step(x, t);
            }
        } else {
            for (int t = 0; t < g32; ++t) {
                const bool lastT = t + 1 == g32;
                const int nbk = lastT ? b + 4 : b;
                const int nt = lastT ? 0 : t + 1;
                fx4 nx[2][U];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int e = 0; e < U; ++e) nx[hh][e] = cur[hh][e];
                if (NEXT || !lastT) {
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                        for (int e = 0; e < U; ++e) nx[hh][e] = ld(nbk, nt, hh, e);
                }
                __builtin_amdgcn_sched_barrier(0);
                step(cur, t);
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int e = 0; e < U; ++e) cur[hh][e] = nx[hh][e];
            }
        }

        if constexpr (KT > 0) {
            topk_block(acc, xnh, b);
            return;
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int64_t r0 = rowBeg + (int64_t)b * 32 + hh * 16 + quarter * 4;
            const fx4 xn4 = xnh[hh];
#pragma unroll
            for (int bq = 0; bq < NQB; ++bq) {
                bool f[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    f[i] = METRIC == 0 ? fmaf(-2.0f, acc[hh][bq][i], xn4[i]) <= ft[bq]
                                       : acc[hh][bq][i] >= ft[bq];
                if (!(f[0] | f[1] | f[2] | f[3])) continue;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (!f[i]) continue;
                    const int64_t row = r0 + i;
                    const int id = (int)(row * p.id_stride);
                    const float dot = acc[hh][bq][i];
                    float key;
                    if (METRIC == 0) {
                        const float tt = fmaf(-2.0f, dot, qn[bq] + xn4[i]);
                        key = (tt < 0.0f ? 0.0f : tt) + 0.0f;
                    } else {
                        key = -dot + 0.0f;
                    }
                    const bool pass = row < p.nrows && qv[bq] &&
                                      (key < tk[bq] || (key == tk[bq] && id <= ti[bq]));
                    if (pass && kPoolable && p.qcnt) {   // pooled region of the query
                        const int ql = bq * 16 + r16;
                        const int gs = atomicAdd(&p.qcnt[ql * kPoolCntStride], 1);
                        if (gs < p.qcap[ql]) p.cand[p.qoff[ql] + gs] = make_uint2(__float_as_uint(key), (unsigned)id);
                    } else if (pass) {
                        const int ql = bq * 16 + r16;
                        const int slot = atomicAdd(&sCnt[ql], 1);
                        if (slot < p.cap)
                            p.cand[((int64_t)ql * p.nsplit + split) * p.cap + slot] =
                                make_uint2(__float_as_uint(key), (unsigned)id);
                    }
                }
            }
        }
    };
    int b = wave;
    for (; b + 4 < nblk; b += 4) block(b, std::true_type{});
    if (b < nblk) block(b, std::false_type{});

    __syncthreads();
    if constexpr (KT > 0) {
        // the split's top-k of query tid: a merge of its four waves' lists
        if (tid < 16 && tid < nqv) {
            int h[4] = {0, 0, 0, 0};
            int n[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) n[w] = sLen[w * 16 + tid];
            uint2* out = p.cand + ((int64_t)tid * p.nsplit + split) * p.cap;
            int o = 0;
            for (; o < kk; ++o) {
                uint64_t best = ~0ull;
                int bw = -1;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    if (h[w] < n[w]) {
                        const uint64_t x = sList[(w * 16 + tid) * KT + h[w]];
                        if (x < best) {
                            best = x;
                            bw = w;
                        }
                    }
                }
                if (bw < 0) break;
                ++h[bw];
                out[o] = make_uint2(__float_as_uint(ord_to_key((uint32_t)(best >> 32))),
                                    (unsigned)(best & 0xFFFFFFFFu));
            }
            p.cnt[(int64_t)tid * p.nsplit + split] = o;
        }
        return;
    }
    if (tid < 16 * NQB && tid < nqv && !(kPoolable && p.qcnt)) p.cnt[(int64_t)tid * p.nsplit + split] = sCnt[tid];
}

// ---------------------------------------------------------------------------
// select: exact per-query top-k of the candidate regions
// ---------------------------------------------------------------------------

// One workgroup (256 threads) per query. The (key, id) composites are distinct
// (an id appears at most once per query), so the k-th smallest composite T is
// unique and the winners are exactly the composites <= T.
// KT: winners (and k-th bucket members) the block can hold, k <= KT; a
// smaller KT (k <= 256) leaves LDS for more blocks per CU.
template <int NBUF, int KT>
__global__ void __launch_bounds__(256) select_kernel(SelectParams p) {
    __shared__ uint64_t sBuf[NBUF];
    __shared__ uint64_t sTop[KT];
    extern __shared__ int sOff[];   // nsplit + 1 entries (dynamic)
    __shared__ unsigned sHist[256];
    __shared__ unsigned sSel[3];
    __shared__ int sWave[4];
    __shared__ int sSeen[4];
    __shared__ uint64_t sT;
    __shared__ int sN;
    __shared__ unsigned sRange[2][4];

    const int q = blockIdx.x;
    if (p.nq_dev && q >= *p.nq_dev) return;   // a device-built work list shorter than the grid
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int ns = p.nsplit;
    const int64_t qbase = (int64_t)q * ns;
    // region capacity and start: per (query, split) of p.cap entries, or one
    // pooled region per query (nsplit == 1)
    const int capq = p.qcap ? p.qcap[q] : p.cap;
    auto regBase = [&](int sidx) -> int64_t { return p.qoff ? p.qoff[q] : (qbase + sidx) * p.cap; };

    // exclusive prefix of the stored (clamped) counts: sOff[s] .. sOff[s+1].
    // Thread t owns the contiguous splits [t per, (t + 1) per), so any split
    // count costs one block scan (two barriers).
    const int per = (ns + 255) / 256;
    const int s0 = tid * per;
    int local = 0;
    int seen = 0;   // unclamped
    bool ovfLocal = false;
    for (int i = 0; i < per; ++i) {
        const int sidx = s0 + i;
        if (sidx < ns) {
            const int n = p.cnt[p.qoff ? (int64_t)q * kPoolCntStride : qbase + sidx];
            ovfLocal |= n > capq;
            local += n < capq ? n : capq;
            seen += n;
        }
    }
    if (p.total) {
        for (int off = 32; off > 0; off >>= 1) seen += __shfl_xor(seen, off, 64);
    }
    int x = local;
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(x, off, 64);
        if (lane >= off) x += t;
    }
    if (lane == 63) sWave[wave] = x;
    if (lane == 0) sSeen[wave] = seen;
    __syncthreads();
    int run = x - local;
    for (int w = 0; w < wave; ++w) run += sWave[w];
    for (int i = 0; i < per; ++i) {
        const int sidx = s0 + i;
        if (sidx < ns) {
            const int n = p.cnt[p.qoff ? (int64_t)q * kPoolCntStride : qbase + sidx];
            run += n < capq ? n : capq;
            sOff[sidx + 1] = run;
        }
    }
    if (tid == 0) sOff[0] = 0;
    const bool ovf = __syncthreads_or(ovfLocal);
    const int c = sWave[0] + sWave[1] + sWave[2] + sWave[3];
    const bool inLds = c <= NBUF;

    // flat index -> candidate (binary search over the split offsets)
    auto fetch = [&](int e) -> uint64_t {
        int lo = 0, hi = ns;   // find s with sOff[s] <= e < sOff[s+1]
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (sOff[mid] <= e) lo = mid; else hi = mid;
        }
        return composite(p.cand[regBase(lo) + (e - sOff[lo])]);
    };
    if (inLds) {
        if (ns >= 256) {
            // many splits with few candidates each (small batches): thread t's
            // splits [s0, s0 + per) hold the flat elements [sOff[s0],
            // sOff[s0 + per]); a split cursor walks them (no offset search per
            // element), eight loads in flight
            if (s0 < ns) {
                const int E1 = sOff[min(s0 + per, ns)];
                int cur = s0;
                for (int e0 = sOff[s0]; e0 < E1; e0 += 8) {
                    uint64_t v[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int e = e0 + u;
                        if (e < E1) {
                            while (sOff[cur + 1] <= e) ++cur;
                            v[u] = composite(p.cand[regBase(cur) + (e - sOff[cur])]);
                        }
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        if (e0 + u < E1) sBuf[e0 + u] = v[u];
                }
            }
        } else {
            // eight offset searches and loads per thread in flight
            for (int e0 = tid; e0 < c; e0 += 8 * 256) {
                uint64_t v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = e0 + u * 256 < c ? fetch(e0 + u * 256) : 0ull;
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (e0 + u * 256 < c) sBuf[e0 + u * 256] = v[u];
            }
        }
    }
    __syncthreads();

    auto for_each = [&](auto&& f) {
        if (inLds) {
            for (int e = tid; e < c; e += 256) f(sBuf[e]);
        } else {
            // eight candidates per thread in flight (offset searches and loads)
            for (int e0 = tid; e0 < c; e0 += 8 * 256) {
                uint64_t v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = e0 + u * 256 < c ? fetch(e0 + u * 256) : 0ull;
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (e0 + u * 256 < c) f(v[u]);
            }
        }
    };

    const int k = p.k;
    // Bucket of the histogram sHist holding rank kr (1-based) of the counted
    // elements -> sSel = {bucket, rank within it, bucket size}.
    auto findBucket = [&](unsigned kr) {
        __syncthreads();
        if (tid < 64) {
            const unsigned h0 = sHist[4 * tid], h1 = sHist[4 * tid + 1];
            const unsigned h2 = sHist[4 * tid + 2], h3 = sHist[4 * tid + 3];
            const unsigned s4 = h0 + h1 + h2 + h3;
            unsigned incl = s4;
            for (int off = 1; off < 64; off <<= 1) {
                const unsigned t = __shfl_up(incl, off, 64);
                if (tid >= off) incl += t;
            }
            const unsigned excl = incl - s4;
            if (excl < kr && kr <= incl) {
                unsigned cum = excl;
                unsigned b = 4 * tid, hb = h0;
                if (cum + h0 < kr) {
                    cum += h0; b += 1; hb = h1;
                    if (cum + h1 < kr) {
                        cum += h1; b += 1; hb = h2;
                        if (cum + h2 < kr) { cum += h2; b += 1; hb = h3; }
                    }
                }
                sSel[0] = b;
                sSel[1] = kr - cum;
                sSel[2] = hb;
            }
        }
        __syncthreads();
    };
    // ascending bitonic sort of sTop[0, P), P a power of two
    auto sortTop = [&](int P) {
        for (int size = 2; size <= P; size <<= 1) {
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                for (int i = tid; i < (P >> 1); i += 256) {
                    const int lo = 2 * i - (i & (stride - 1));
                    const int hi = lo + stride;
                    const bool asc = (lo & size) == 0;
                    const uint64_t a = sTop[lo], b = sTop[hi];
                    if ((a > b) == asc) { sTop[lo] = b; sTop[hi] = a; }
                }
                __syncthreads();
            }
        }
    };

    // Rank of element i of sTop[0, n) in ascending (composite, position) order:
    // the elements before it. n <= 256 with one element per thread: a read pass
    // of broadcast LDS loads and no barriers inside, against the ~28 barrier
    // stages of a bitonic sort of 128. Composites of one query are distinct
    // (an id is stored at most once); the position tie-break keeps the ranks a
    // permutation regardless.
    auto rankOf = [&](int n, int i, uint64_t x) -> int {
        int r = 0;
#pragma unroll 4
        for (int jj = 0; jj < n; ++jj) {
            const uint64_t y = sTop[jj];
            r += (y < x || (y == x && jj < i)) ? 1 : 0;
        }
        return r;
    };

    uint64_t T = ~0ull;   // take everything when c <= k
    if (c > k) {
        bool found = false;
        // One histogram over the key ordinals' actual range [omin, omax] (keys
        // of one query usually span a narrow range, which would put most of
        // them in one bin of a fixed-digit radix pass): the k-th composite lies
        // in bucket b, whose members (composites order by key first) are the
        // only ones that need sorting.
        unsigned omin = ~0u, omax = 0u;
        for_each([&](uint64_t x) {
            const unsigned o = (unsigned)(x >> 32);
            omin = o < omin ? o : omin;
            omax = o > omax ? o : omax;
        });
        for (int off = 32; off > 0; off >>= 1) {
            const unsigned a = (unsigned)__shfl_xor((int)omin, off, 64);
            const unsigned b = (unsigned)__shfl_xor((int)omax, off, 64);
            omin = a < omin ? a : omin;
            omax = b > omax ? b : omax;
        }
        if (lane == 0) { sRange[0][wave] = omin; sRange[1][wave] = omax; }
        __syncthreads();
        omin = sRange[0][0]; omax = sRange[1][0];
        for (int w = 1; w < 4; ++w) {
            omin = sRange[0][w] < omin ? sRange[0][w] : omin;
            omax = sRange[1][w] > omax ? sRange[1][w] : omax;
        }
        if (omax > omin) {
            const int bits = 32 - __clz((int)(omax - omin));   // bits of the largest offset
            const int sh = bits > 8 ? bits - 8 : 0;
            sHist[tid] = 0;
            __syncthreads();
            for_each([&](uint64_t x) { atomicAdd(&sHist[((unsigned)(x >> 32) - omin) >> sh], 1u); });
            findBucket((unsigned)k);
            const unsigned b = sSel[0], kr = sSel[1], hb = sSel[2];
            if (hb <= (unsigned)KT) {
                if (tid == 0) sN = 0;
                __syncthreads();
                for_each([&](uint64_t x) {
                    if ((((unsigned)(x >> 32) - omin) >> sh) == b) sTop[atomicAdd(&sN, 1)] = x;
                });
                __syncthreads();
                if (hb <= 256u) {
                    // the bucket member of rank kr - 1 is T
                    if (tid < (int)hb) {
                        const uint64_t x = sTop[tid];
                        if (rankOf((int)hb, tid, x) == (int)kr - 1) sT = x;
                    }
                    __syncthreads();
                    T = sT;
                } else {
                    int P = 1;
                    while (P < (int)hb) P <<= 1;
                    for (int i = (int)hb + tid; i < P; i += 256) sTop[i] = ~0ull;
                    __syncthreads();
                    sortTop(P);
                    T = sTop[kr - 1];
                }
                found = true;
                __syncthreads();
            }
        }
        // Fallback (all keys equal, or an overfull bucket): radix select on
        // 8-bit digits of the composite.
        uint64_t prefix = 0, mask = 0;
        unsigned kr = (unsigned)k;
        for (int shift = 56; shift >= 0 && !found; shift -= 8) {
            sHist[tid] = 0;
            __syncthreads();
            for_each([&](uint64_t x) {
                if ((x & mask) == prefix) atomicAdd(&sHist[(unsigned)(x >> shift) & 255u], 1u);
            });
            findBucket(kr);
            const unsigned b = sSel[0];
            kr = sSel[1];
            const unsigned hb = sSel[2];
            prefix |= (uint64_t)b << shift;
            mask |= (uint64_t)0xFFu << shift;
            __syncthreads();
            if (hb == 1u) {
                for_each([&](uint64_t x) {
                    if ((x & mask) == prefix) sT = x;
                });
                __syncthreads();
                T = sT;
                found = true;
            }
        }
        if (!found) T = prefix;
    }

    if (tid == 0) sN = 0;
    __syncthreads();
    for_each([&](uint64_t x) {
        if (x <= T) {
            const int pos = atomicAdd(&sN, 1);
            if (pos < KT) sTop[pos] = x;
        }
    });
    __syncthreads();
    const int nsel = sN < KT ? sN : KT;
    if (nsel <= 256) {
        // every thread reads before any writes: one barrier between
        uint64_t x = 0;
        int r = 0;
        if (tid < nsel) {
            x = sTop[tid];
            r = rankOf(nsel, tid, x);
        }
        __syncthreads();
        if (tid < nsel) sTop[r] = x;
        __syncthreads();
    } else {
        int P = 1;
        while (P < nsel) P <<= 1;
        for (int i = nsel + tid; i < P; i += 256) sTop[i] = ~0ull;
        __syncthreads();
        sortTop(P);
    }

    const int orow = p.qmap ? p.qmap[q] : q;
    if (p.out_ids || p.out_vals) {
        for (int i = tid; i < k; i += 256) {
            int32_t id = -1;
            float val = p.metric == 0 ? INFINITY : -INFINITY;
            if (i < nsel) {
                const uint64_t x = sTop[i];
                id = (int32_t)(uint32_t)(x & 0xFFFFFFFFu);
                const float key = ord_to_key((uint32_t)(x >> 32));
                val = p.metric == 0 ? key : -key;
            }
            if (p.out_ids) p.out_ids[(int64_t)orow * p.out_stride + i] = id;
            if (p.out_vals) p.out_vals[(int64_t)orow * p.out_stride + i] = val;
        }
    }
    if (tid == 0) {
        if (p.tau_j_key) {
            if (nsel >= p.j) {
                const uint64_t x = sTop[p.j - 1];
                p.tau_j_key[orow] = ord_to_key((uint32_t)(x >> 32));
                p.tau_j_id[orow] = (int)(uint32_t)(x & 0xFFFFFFFFu);
            } else {
                p.tau_j_key[orow] = INFINITY;
                p.tau_j_id[orow] = -1;
            }
        }
        if (p.tau_j2_key) {
            if (nsel >= p.j2) {
                const uint64_t x = sTop[p.j2 - 1];
                p.tau_j2_key[orow] = ord_to_key((uint32_t)(x >> 32));
                p.tau_j2_id[orow] = (int)(uint32_t)(x & 0xFFFFFFFFu);
            } else {
                p.tau_j2_key[orow] = INFINITY;
                p.tau_j2_id[orow] = -1;
            }
        }
        if (p.tau_k_key) {
            if (nsel >= k) {
                const uint64_t x = sTop[k - 1];
                p.tau_k_key[orow] = ord_to_key((uint32_t)(x >> 32));
                p.tau_k_id[orow] = (int)(uint32_t)(x & 0xFFFFFFFFu);
            } else {
                p.tau_k_key[orow] = INFINITY;
                p.tau_k_id[orow] = -1;
            }
        }
        const int st = (ovf ? 1 : 0) | (c < k ? 2 : 0);
        if (p.status) p.status[orow] = st;
        if (p.fail_count && st) atomicAdd(p.fail_count, 1);
        if (p.total) p.total[orow] = sSeen[0] + sSeen[1] + sSeen[2] + sSeen[3];
    }
}

// k = 1 results: packed (ordered key, id) -> id, reported value; all-ones = empty.
__global__ void argmin_finalize_kernel(const unsigned long long* __restrict__ best, int nq, int metric,
                                       int32_t* __restrict__ ids, float* __restrict__ vals) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= nq) return;
    const unsigned long long x = best[q];
    int32_t id = -1;
    float val = metric == 0 ? INFINITY : -INFINITY;
    if (x != ~0ull) {
        id = (int32_t)(uint32_t)(x & 0xFFFFFFFFull);
        const float key = ord_to_key((uint32_t)(x >> 32));
        val = metric == 0 ? key : -key;
    }
    if (ids) ids[q] = id;
    if (vals) vals[q] = val;
}

__global__ void fill_u64_kernel(unsigned long long* __restrict__ p, int64_t n, unsigned long long v) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

static int grid_for(int64_t work, int block) {
    int64_t g = (work + block - 1) / block;
    if (g > 65536) g = 65536;
    if (g < 1) g = 1;
    return (int)g;
}

void launch_pack_rows(const float* src, int64_t n, int dim, float* dst, int64_t n_pad, int dpad,
                      hipStream_t s) {
    if (n_pad <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    pack_rows_kernel<<<grid_for(n_pad * dpad, 256), 256, 0, s>>>(src, n, dim, dst, n_pad, dpad);
    prof_end(tok, s);
    check_launch("pack_rows");
}

void launch_prep_queries(const float* src, int64_t n, int dim, int64_t n_pad, int dpad, int storage, bool cosine,
                         void* out, float* qn, float* tau_key, int* tau_id, hipStream_t s) {
    if (n_pad <= 0) return;
    if (dpad % 8 != 0) throw std::runtime_error("prep_queries: dpad must be a multiple of 8");
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    const int g = (int)((n_pad + 3) / 4);   // a wave per row
    if (storage == kF32)
        prep_queries_kernel<kF32><<<g, 256, 0, s>>>(src, n, dim, n_pad, dpad, cosine ? 1 : 0, out, qn, tau_key, tau_id);
    else if (storage == kF16)
        prep_queries_kernel<kF16><<<g, 256, 0, s>>>(src, n, dim, n_pad, dpad, cosine ? 1 : 0, out, qn, tau_key, tau_id);
    else if (storage == kBF16)
        prep_queries_kernel<kBF16><<<g, 256, 0, s>>>(src, n, dim, n_pad, dpad, cosine ? 1 : 0, out, qn, tau_key, tau_id);
    else
        throw std::runtime_error("prep_queries: unknown storage type");
    prof_end(tok, s);
    check_launch("prep_queries");
}

void launch_normalize_rows(float* v, int64_t n, int dpad, hipStream_t s) {
    if (n <= 0) return;
    void* tok;
    prof_begin(kFamNorms, s, &tok);
    normalize_rows_kernel<<<(int)((n + 255) / 256), 256, 0, s>>>(v, n, dpad);
    prof_end(tok, s);
    check_launch("normalize_rows");
}

static void check_storage(int storage) {
    if (storage != kF32 && storage != kF16 && storage != kBF16)
        throw std::runtime_error("unknown storage type");
}

void launch_round_rows(const float* src, int64_t count, int storage, void* dst, hipStream_t s) {
    if (count <= 0) return;
    check_storage(storage);
    if (storage == kF32) throw std::runtime_error("round_rows: fp32 needs no rounding");
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    if (storage == kF16)
        round_rows_kernel<kF16><<<grid_for(count, 256), 256, 0, s>>>(src, count, (uint16_t*)dst);
    else
        round_rows_kernel<kBF16><<<grid_for(count, 256), 256, 0, s>>>(src, count, (uint16_t*)dst);
    prof_end(tok, s);
    check_launch("round_rows");
}

void launch_row_norms(const void* v, int64_t n, int dpad, int storage, float* out, hipStream_t s) {
    if (n <= 0) return;
    check_storage(storage);
    void* tok;
    prof_begin(kFamNorms, s, &tok);
    const int g = (int)((n + 255) / 256);
    if (storage == kF32) row_norms_kernel<kF32><<<g, 256, 0, s>>>(v, n, dpad, out);
    else if (storage == kF16) row_norms_kernel<kF16><<<g, 256, 0, s>>>(v, n, dpad, out);
    else row_norms_kernel<kBF16><<<g, 256, 0, s>>>(v, n, dpad, out);
    prof_end(tok, s);
    check_launch("row_norms");
}

void launch_row_inv_norms(const float* src, int64_t n, int dim, float* inv, hipStream_t s) {
    if (n <= 0) return;
    void* tok;
    prof_begin(kFamNorms, s, &tok);
    row_inv_norms_kernel<<<(int)((n + 255) / 256), 256, 0, s>>>(src, n, dim, inv);
    prof_end(tok, s);
    check_launch("row_inv_norms");
}

void launch_store_rows_blk(const float* src, int64_t n, int dim, const float* inv, void* X, int64_t row0,
                           int dpad, int storage, hipStream_t s) {
    if (n <= 0) return;
    check_storage(storage);
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    const int g = grid_for(n * dpad / 4, 256);
    if (storage == kF32) store_rows_blk_kernel<kF32><<<g, 256, 0, s>>>(src, n, dim, inv, X, row0, dpad);
    else if (storage == kF16) store_rows_blk_kernel<kF16><<<g, 256, 0, s>>>(src, n, dim, inv, X, row0, dpad);
    else store_rows_blk_kernel<kBF16><<<g, 256, 0, s>>>(src, n, dim, inv, X, row0, dpad);
    prof_end(tok, s);
    check_launch("store_rows_blk");
}

void launch_row_norms_blk(const void* X, int64_t row0, int64_t n, int dpad, int storage, float* out,
                          hipStream_t s) {
    if (n <= 0) return;
    check_storage(storage);
    void* tok;
    prof_begin(kFamNorms, s, &tok);
    const int g = (int)((n + 255) / 256);
    if (storage == kF32) row_norms_blk_kernel<kF32><<<g, 256, 0, s>>>(X, row0, n, dpad, out);
    else if (storage == kF16) row_norms_blk_kernel<kF16><<<g, 256, 0, s>>>(X, row0, n, dpad, out);
    else row_norms_blk_kernel<kBF16><<<g, 256, 0, s>>>(X, row0, n, dpad, out);
    prof_end(tok, s);
    check_launch("row_norms_blk");
}

void launch_gather_rows_blk(const void* X, const int* idx, int n, int dpad, int storage, void* dst,
                            hipStream_t s) {
    if (n <= 0) return;
    check_storage(storage);
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    const int g = grid_for((int64_t)n * dpad / 4, 256);
    if (storage == kF32) gather_rows_blk_kernel<kF32><<<g, 256, 0, s>>>(X, idx, n, dpad, dst);
    else if (storage == kF16) gather_rows_blk_kernel<kF16><<<g, 256, 0, s>>>(X, idx, n, dpad, dst);
    else gather_rows_blk_kernel<kBF16><<<g, 256, 0, s>>>(X, idx, n, dpad, dst);
    prof_end(tok, s);
    check_launch("gather_rows_blk");
}

void launch_gather_rows(const void* src, const int* idx, int n, int row_bytes, void* dst,
                        int64_t n_pad, hipStream_t s) {
    if (n_pad <= 0) return;
    if (row_bytes % 16 != 0) throw std::runtime_error("gather_rows: row size not a multiple of 16 bytes");
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    const int pieces = row_bytes / 16;
    gather_rows_kernel<<<grid_for(n_pad * pieces, 256), 256, 0, s>>>((const fx4*)src, idx, n, pieces,
                                                                      (fx4*)dst, n_pad);
    prof_end(tok, s);
    check_launch("gather_rows");
}

void launch_gather_f32(const float* src, const int* idx, int n, float* dst, hipStream_t s) {
    if (n <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    gather_f32_kernel<<<(n + 255) / 256, 256, 0, s>>>(src, idx, n, dst);
    prof_end(tok, s);
    check_launch("gather_f32");
}

void launch_gather_tau(const TauSources& src, const int* idx, const int* sel, int n, float* ko,
                       int* io, hipStream_t s) {
    if (n <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    gather_tau_kernel<<<(n + 255) / 256, 256, 0, s>>>(src, idx, sel, n, ko, io);
    prof_end(tok, s);
    check_launch("gather_tau");
}

void launch_retry_plan(const RetryPlanArgs& a, hipStream_t s) {
    if (a.mb <= 0 || a.rmax <= 0 || a.rmax > kRetryPlanMax || a.rows_pad < a.rmax || a.row_bytes % 16 != 0)
        throw std::runtime_error("retry_plan: bad sizes");
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    retry_plan_kernel<<<1, 1024, 0, s>>>(a);
    prof_end(tok, s);
    check_launch("retry_plan");
}

void launch_fill_tau_none(float* key, int* id, int n, hipStream_t s) {
    if (n <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    fill_tau_none_kernel<<<(n + 255) / 256, 256, 0, s>>>(key, id, n);
    prof_end(tok, s);
    check_launch("fill_tau_none");
}

void launch_tau_min(float* key_a, int* id_a, const float* key_b, const int* id_b, int n, hipStream_t s) {
    if (n <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    tau_min_kernel<<<(n + 255) / 256, 256, 0, s>>>(key_a, id_a, key_b, id_b, n);
    prof_end(tok, s);
    check_launch("tau_min");
}

void launch_fill_empty(int32_t* ids, float* vals, int64_t count, float empty, hipStream_t s) {
    if (count <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    fill_empty_kernel<<<grid_for(count, 256), 256, 0, s>>>(ids, vals, count, empty);
    prof_end(tok, s);
    check_launch("fill_empty");
}

void launch_max_norm(const float* xn, int64_t n, unsigned* out, hipStream_t s) {
    if (n <= 0) return;
    void* tok;
    prof_begin(kFamNorms, s, &tok);
    max_norm_kernel<<<grid_for(n, 256) < 1024 ? grid_for(n, 256) : 1024, 256, 0, s>>>(xn, n, out);
    prof_end(tok, s);
    check_launch("max_norm");
}

template <int S, int M, int NQB, int G>
static void launch_small_g(const ScanParams& p, int pass, int g, size_t lds, hipStream_t s) {
    if (pass == kPassSample) scan_small_kernel<S, M, NQB, kPassSample, G, 0><<<g, 256, lds, s>>>(p);
    else if (pass == kPassRetry) scan_small_kernel<S, M, NQB, kPassRetry, G, 0><<<g, 256, lds, s>>>(p);
    else scan_small_kernel<S, M, NQB, kPassFull, G, 0><<<g, 256, lds, s>>>(p);
}
template <int S, int M, int G>
static const void* topk_fn() {
    return (const void*)scan_small_kernel<S, M, 1, kPassFull, G, kStreamTopK>;
}
template <int S, int M>
static const void* topk_fn_d(int dpad) {
    return dpad == 96 ? topk_fn<S, M, 3>() : dpad == 128 ? topk_fn<S, M, 4>() : topk_fn<S, M, 0>();
}
static const void* topk_kernel(int dpad, int storage, int metric) {
    if (storage == kF32) return metric == 0 ? topk_fn_d<kF32, 0>(dpad) : topk_fn_d<kF32, 1>(dpad);
    if (storage == kF16) return metric == 0 ? topk_fn_d<kF16, 0>(dpad) : topk_fn_d<kF16, 1>(dpad);
    return metric == 0 ? topk_fn_d<kBF16, 0>(dpad) : topk_fn_d<kBF16, 1>(dpad);
}
template <int S, int M, int NQB>
static void launch_small(const ScanParams& p, int pass, int g, size_t lds, hipStream_t s) {
    if (p.dpad == 96) launch_small_g<S, M, NQB, 3>(p, pass, g, lds, s);
    else if (p.dpad == 128) launch_small_g<S, M, NQB, 4>(p, pass, g, lds, s);
    else launch_small_g<S, M, NQB, 0>(p, pass, g, lds, s);
}
template <int S, int M>
static void launch_small_m(const ScanParams& p, int pass, int nqb16, size_t lds, hipStream_t s) {
    if (nqb16 == 1) launch_small<S, M, 1>(p, pass, p.nsplit, lds, s);
    else if (nqb16 == 2) launch_small<S, M, 2>(p, pass, p.nsplit, lds, s);
    else launch_small<S, M, 4>(p, pass, p.nsplit, lds, s);
}
template <int S>
static void launch_small_s(const ScanParams& p, int metric, int pass, int nqb16, size_t lds, hipStream_t s) {
    if (metric == 0) launch_small_m<S, 0>(p, pass, nqb16, lds, s);
    else launch_small_m<S, 1>(p, pass, nqb16, lds, s);
}
// Raises a kernel's dynamic-LDS limit to kResidentMaxLdsNarrow (needed above
// the default per-launch limit; the launch's own size sets the occupancy);
// throws if the runtime refuses.
static void allow_resident_lds(const void* f) {
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kResidentMaxLdsNarrow) != hipSuccess)
        throw std::runtime_error("scan_resident: cannot raise the dynamic LDS limit");
}
template <int S, int M, int P, int G, bool IVF = false, int NB = 4>
static void launch_resident_p(const ScanParams& p, int g, size_t lds, hipStream_t s) {
    static const bool ok = (allow_resident_lds((const void*)scan_resident_kernel<S, M, P, G, IVF, NB>), true);
    (void)ok;
    scan_resident_kernel<S, M, P, G, IVF, NB><<<g, 256, lds, s>>>(p);
}
static size_t resident_lds_bytes(int dpad, int storage, int tileQueries);
// The row-sample pass runs 32-query tiles (NB = 1): it stores every row it
// reads, so the survivor stores, not the MFMA work, set its time, and 4x the
// workgroups spread them; the per-pair MFMA sequence is the same as the
// 128-query tiles', so its keys are bit-identical to the other passes'.
template <int S, int M, int G>
static void launch_resident_g(const ScanParams& p, int pass, int g, size_t lds, hipStream_t s) {
    if (pass == kPassSample) {
        ScanParams q = p;
        q.nqb = (p.nq + 31) / 32;
        launch_resident_p<S, M, kPassSample, G, false, 1>(q, q.nqb * p.nsplit, resident_lds_bytes(p.dpad, S, 32), s);
    }
    else if (pass == kPassRetry) launch_resident_p<S, M, kPassRetry, G>(p, g, lds, s);
    else launch_resident_p<S, M, kPassFull, G>(p, g, lds, s);
}
// k = 1 keeps a running best per lane instead of stores; it always takes the
// one-chunk-prefetch loop.
template <int S, int M>
static void launch_resident(const ScanParams& p, int pass, int g, size_t lds, hipStream_t s) {
    if (pass == kPassArgmin) return launch_resident_p<S, M, kPassArgmin, 0>(p, g, lds, s);
    if constexpr (S != kF32) {
        if (p.dpad == 96) return launch_resident_g<S, M, 3>(p, pass, g, lds, s);
        if (p.dpad == 128) return launch_resident_g<S, M, 4>(p, pass, g, lds, s);
    }
    launch_resident_g<S, M, 0>(p, pass, g, lds, s);
}
template <int S>
static void launch_resident_s(const ScanParams& p, int metric, int pass, int g, size_t lds, hipStream_t s) {
    if (metric == 0) launch_resident<S, 0>(p, pass, g, lds, s);
    else launch_resident<S, 1>(p, pass, g, lds, s);
}
// IVF fine scan: kPassSample (no bound, the bound pass) or kPassFull, with
// the G variants of the flat scan (the same key function for a given dpad);
// tiles of 128 (NB = 4) or 32 (NB = 1) queries, bit-identical keys.
template <int S, int M, int G, int NB>
static void launch_ivf_g(const ScanParams& p, int pass, int g, size_t lds, hipStream_t s) {
    if (pass == kPassSample) launch_resident_p<S, M, kPassSample, G, true, NB>(p, g, lds, s);
    else launch_resident_p<S, M, kPassFull, G, true, NB>(p, g, lds, s);
}
template <int S, int M, int NB>
static void launch_ivf(const ScanParams& p, int pass, int g, size_t lds, hipStream_t s) {
    if constexpr (S != kF32) {
        if (p.dpad == 96) return launch_ivf_g<S, M, 3, NB>(p, pass, g, lds, s);
        if (p.dpad == 128) return launch_ivf_g<S, M, 4, NB>(p, pass, g, lds, s);
    }
    launch_ivf_g<S, M, 0, NB>(p, pass, g, lds, s);
}
template <int S>
static void launch_ivf_s(const ScanParams& p, int metric, int pass, int nb, int g, size_t lds, hipStream_t s) {
    if (nb == 4) {
        if (metric == 0) launch_ivf<S, 0, 4>(p, pass, g, lds, s);
        else launch_ivf<S, 1, 4>(p, pass, g, lds, s);
    } else {
        if (metric == 0) launch_ivf<S, 0, 1>(p, pass, g, lds, s);
        else launch_ivf<S, 1, 1>(p, pass, g, lds, s);
    }
}

static size_t resident_lds_bytes(int dpad, int storage, int tileQueries) {
    const int es = elem_bytes(storage);
    return (size_t)tileQueries * (dpad + 16 / es) * es;
}

bool resident_scan_fits(int dpad, int storage) {
    return resident_lds_bytes(dpad, storage, kBN) <= kResidentMaxLds;
}

bool ivf_narrow_fits(int dpad, int storage) {
    return resident_lds_bytes(dpad, storage, 32) <= kResidentMaxLdsNarrow;
}

template <int S, int M>
static void launch_tiled(const ScanParams& p, int pass, int g, hipStream_t s) {
    if (pass == kPassSample) scan_filter_kernel<S, M, kPassSample><<<g, 256, 0, s>>>(p);
    else if (pass == kPassRetry) scan_filter_kernel<S, M, kPassRetry><<<g, 256, 0, s>>>(p);
    else if (pass == kPassArgmin) scan_filter_kernel<S, M, kPassArgmin><<<g, 256, 0, s>>>(p);
    else scan_filter_kernel<S, M, kPassFull><<<g, 256, 0, s>>>(p);
}
template <int S, int M>
static void launch_tiled_ivf(const ScanParams& p, int pass, int g, hipStream_t s) {
    if (pass == kPassSample) scan_filter_kernel<S, M, kPassSample, true><<<g, 256, 0, s>>>(p);
    else scan_filter_kernel<S, M, kPassFull, true><<<g, 256, 0, s>>>(p);
}
template <int S>
static void launch_tiled_ivf_s(const ScanParams& p, int metric, int pass, int g, hipStream_t s) {
    if (metric == 0) launch_tiled_ivf<S, 0>(p, pass, g, s);
    else launch_tiled_ivf<S, 1>(p, pass, g, s);
}
template <int S>
static void launch_tiled_s(const ScanParams& p, int metric, int pass, int g, hipStream_t s) {
    if (metric == 0) launch_tiled<S, 0>(p, pass, g, s);
    else launch_tiled<S, 1>(p, pass, g, s);
}

static size_t small_lds_bytes(int nq, int dpad, int storage) {
    const int nqb16 = nq <= 16 ? 1 : nq <= 32 ? 2 : 4;
    const int es = elem_bytes(storage);
    return (size_t)16 * nqb16 * (dpad + 16 / es) * es;
}

bool small_scan_fits(int nq, int dpad, int storage) {
    return nq >= 1 && nq <= kSmallMaxQ && small_lds_bytes(nq, dpad, storage) <= kSmallMaxLds;
}

int topk_concurrency(int dpad, int storage, int metric) {
    const void* f = topk_kernel(dpad, storage, metric);
    const size_t lds = small_lds_bytes(1, dpad, storage);
    int dev = 0, cus = 0, per = 0;
    if (!f || hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, f, 256, lds) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return per > 0 && cus > 0 ? per * cus : 0;
}

void launch_scan_topk(const ScanParams& p, int metric, int storage, hipStream_t s) {
    if (p.nsplit <= 0) return;
    if (p.nq < 1 || p.nq > kStreamMaxQ || p.cap < 1 || p.cap > kStreamTopK || p.rows_per_split % kBM != 0 ||
        p.dpad % kBK != 0 || !small_scan_fits(p.nq, p.dpad, storage) ||
        (p.qraw ? (p.qdim < 1 || p.qdim > p.dpad) : p.Q == nullptr))
        throw std::runtime_error("scan_topk: bad parameters");
    const void* f = topk_kernel(p.dpad, storage, metric);
    const size_t lds = small_lds_bytes(1, p.dpad, storage);
    void* tok;
    prof_begin(kFamScan, s, &tok);
    void* args[] = {(void*)&p};
    const hipError_t e = hipLaunchKernel(f, dim3(p.nsplit), dim3(256), args, lds, s);
    prof_end(tok, s);
    if (e != hipSuccess) throw std::runtime_error(std::string("scan_topk launch: ") + hipGetErrorString(e));
    check_launch("scan_topk");
}

// The function launch_scan_filter starts for a batch too large for scan_small,
// and its dynamic LDS (for the occupancy query).
template <int S, int M>
static const void* resident_fn(int pass, int dpad) {
    auto f = [](const void* k) {
        allow_resident_lds(k);
        return k;
    };
    if (pass == kPassArgmin) {
        static const void* a = f((const void*)scan_resident_kernel<S, M, kPassArgmin, 0, false, 4>);
        return a;
    }
    const int G = S != kF32 && dpad == 96 ? 3 : S != kF32 && dpad == 128 ? 4 : 0;
#define MFLAT_RES_FN(P, GG)                                                                 \
    if (pass == P && G == GG) {                                                             \
        static const void* k = f((const void*)scan_resident_kernel<S, M, P, GG, false, 4>); \
        return k;                                                                           \
    }
#define MFLAT_RES_FN1(GG)                                                                              \
    if (pass == kPassSample && G == GG) {                                                              \
        static const void* k = f((const void*)scan_resident_kernel<S, M, kPassSample, GG, false, 1>); \
        return k;                                                                                      \
    }
    MFLAT_RES_FN1(0) MFLAT_RES_FN(kPassRetry, 0) MFLAT_RES_FN(kPassFull, 0)
    if constexpr (S != kF32) {
        MFLAT_RES_FN1(3) MFLAT_RES_FN(kPassRetry, 3) MFLAT_RES_FN(kPassFull, 3)
        MFLAT_RES_FN1(4) MFLAT_RES_FN(kPassRetry, 4) MFLAT_RES_FN(kPassFull, 4)
    }
#undef MFLAT_RES_FN
#undef MFLAT_RES_FN1
    return nullptr;
}
template <int S, int M>
static const void* tiled_fn(int pass) {
    if (pass == kPassSample) return (const void*)scan_filter_kernel<S, M, kPassSample>;
    if (pass == kPassRetry) return (const void*)scan_filter_kernel<S, M, kPassRetry>;
    if (pass == kPassArgmin) return (const void*)scan_filter_kernel<S, M, kPassArgmin>;
    return (const void*)scan_filter_kernel<S, M, kPassFull>;
}
template <int S, int M>
static const void* wide_fn(int pass) {
    if (pass == kPassSample) return (const void*)scan_wide_kernel<S, M, kPassSample>;
    if (pass == kPassRetry) return (const void*)scan_wide_kernel<S, M, kPassRetry>;
    return (const void*)scan_wide_kernel<S, M, kPassFull>;
}
template <int S>
static const void* wide_fn_s(int metric, int pass) {
    return metric == 0 ? wide_fn<S, 0>(pass) : wide_fn<S, 1>(pass);
}

bool wide_scan_applies(int nq, int dpad, int storage) {
    return storage != kF32 && nq > kBN && !resident_scan_fits(dpad, storage);
}

template <int S>
static const void* scan_fn(int dpad, int metric, int pass, size_t& lds) {
    if (resident_scan_fits(dpad, S)) {
        lds = resident_lds_bytes(dpad, S, pass == kPassSample ? 32 : kBN);   // the sample pass: 32-query tiles
        return metric == 0 ? resident_fn<S, 0>(pass, dpad) : resident_fn<S, 1>(pass, dpad);
    }
    lds = 0;
    return metric == 0 ? tiled_fn<S, 0>(pass) : tiled_fn<S, 1>(pass);
}

int scan_concurrency(int dpad, int storage, int metric, int pass, bool wide) {
    size_t lds = 0;
    const void* f = (wide && storage != kF32 && pass != kPassArgmin && !resident_scan_fits(dpad, storage))
                        ? (storage == kF16 ? wide_fn_s<kF16>(metric, pass) : wide_fn_s<kBF16>(metric, pass))
                    : storage == kF32 ? scan_fn<kF32>(dpad, metric, pass, lds)
                    : storage == kF16 ? scan_fn<kF16>(dpad, metric, pass, lds)
                                      : scan_fn<kBF16>(dpad, metric, pass, lds);
    const int threads = (wide && storage != kF32 && pass != kPassArgmin && !resident_scan_fits(dpad, storage))
                            ? kWideThreads : 256;
    int dev = 0, cus = 0, per = 0;
    if (!f || hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, f, threads, lds) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return per > 0 && cus > 0 ? per * cus : 0;
}

void launch_scan_filter(const ScanParams& p, int metric, int pass, int storage, hipStream_t s, bool allowSmall) {
    if (storage != kF32 && storage != kF16 && storage != kBF16)
        throw std::runtime_error("scan_filter: unknown storage type");
    if (allowSmall && pass != kPassArgmin && small_scan_fits(p.nq, p.dpad, storage)) {
        if (p.nsplit <= 0) return;
        if (p.rows_per_split % kBM != 0 || p.cap < 1 || p.dpad % kBK != 0)
            throw std::runtime_error("scan_small: bad tiling parameters");
        const int nqb16 = p.nq <= 16 ? 1 : p.nq <= 32 ? 2 : 4;
        const size_t lds = small_lds_bytes(p.nq, p.dpad, storage);
        void* tok;
        prof_begin(pass == kPassSample ? kFamScanSample : pass == kPassRetry ? kFamScanRetry : kFamScan, s, &tok);
        if (storage == kF32) launch_small_s<kF32>(p, metric, pass, nqb16, lds, s);
        else if (storage == kF16) launch_small_s<kF16>(p, metric, pass, nqb16, lds, s);
        else launch_small_s<kBF16>(p, metric, pass, nqb16, lds, s);
        prof_end(tok, s);
        check_launch("scan_small");
        return;
    }
    const int64_t grid = (int64_t)p.nqb * p.nsplit;
    if (grid <= 0) return;
    if (grid > 0x7FFFFFFF) throw std::runtime_error("scan_filter grid too large");
    if (p.dpad % kBK != 0 || p.rows_per_split % kBM != 0 || p.cap < 1)
        throw std::runtime_error("scan_filter: bad tiling parameters");
    void* tok;
    prof_begin(pass == kPassSample ? kFamScanSample : pass == kPassRetry ? kFamScanRetry
               : pass == kPassArgmin ? kFamArgmin : kFamScan, s, &tok);
    const int g = (int)grid;
    if (resident_scan_fits(p.dpad, storage)) {
        const size_t lds = resident_lds_bytes(p.dpad, storage, kBN);
        if (storage == kF32) launch_resident_s<kF32>(p, metric, pass, g, lds, s);
        else if (storage == kF16) launch_resident_s<kF16>(p, metric, pass, g, lds, s);
        else launch_resident_s<kBF16>(p, metric, pass, g, lds, s);
        prof_end(tok, s);
        check_launch("scan_resident");
        return;
    }
    // fp16/bf16 batches the caller put on the wide tile: 256-query blocks
    if (p.wide && storage != kF32 && pass != kPassArgmin) {
        const int nqb2 = (p.nq + kWT - 1) / kWT;
        const int64_t gw = (int64_t)nqb2 * p.nsplit;
        if (gw > 0x7FFFFFFF) throw std::runtime_error("scan_wide grid too large");
        ScanParams pw = p;
        if (pw.qgroup <= 0) {
            const int64_t tileBytes = (int64_t)kWT * p.dpad * 2;
            pw.qgroup = (int)std::max<int64_t>(1, std::min<int64_t>(kQGroup, ((int64_t)5 << 19) / tileBytes));
        }
        const void* f = storage == kF16 ? wide_fn_s<kF16>(metric, pass) : wide_fn_s<kBF16>(metric, pass);
        void* args[] = {(void*)&pw};
        const hipError_t e = hipLaunchKernel(f, dim3((unsigned)gw), dim3(kWideThreads), args, 0, s);
        prof_end(tok, s);
        if (e != hipSuccess) throw std::runtime_error(std::string("scan_wide launch: ") + hipGetErrorString(e));
        return;
    }
    // LDS-tiled kernel: every database tile re-reads the group's query tiles
    // through L2, so the group is as many query blocks as ~2.5 MB of query
    // tiles (the XCD's L2 is 4 MB and also streams the database tiles).
    ScanParams pt = p;
    if (pt.qgroup <= 0) {
        const int64_t tileBytes = (int64_t)kBN * p.dpad * elem_bytes(storage);
        pt.qgroup = (int)std::max<int64_t>(1, std::min<int64_t>(kQGroup, ((int64_t)5 << 19) / tileBytes));
    }
    if (storage == kF32) launch_tiled_s<kF32>(pt, metric, pass, g, s);
    else if (storage == kF16) launch_tiled_s<kF16>(pt, metric, pass, g, s);
    else launch_tiled_s<kBF16>(pt, metric, pass, g, s);
    prof_end(tok, s);
    check_launch("scan_filter");
}

void launch_scan_ivf(const ScanParams& p, int metric, int pass, int storage, int tileQueries, int grid,
                     hipStream_t s) {
    if (storage != kF32 && storage != kF16 && storage != kBF16) throw std::runtime_error("scan_ivf: unknown storage type");
    if (grid <= 0) return;
    if (pass != kPassSample && pass != kPassFull) throw std::runtime_error("scan_ivf: bad pass");
    if (tileQueries != 128 && tileQueries != 32) throw std::runtime_error("scan_ivf: tiles hold 128 or 32 queries");
    // 128-query items whose tile does not fit scan_resident's LDS run the tiled kernel
    const bool tiled = tileQueries == 128 && !resident_scan_fits(p.dpad, storage);
    if (!(tileQueries == 128 || ivf_narrow_fits(p.dpad, storage)) || p.dpad % kBK != 0 || p.cap < 1 ||
        p.ivf_nprobe < 1 || p.ivf_nreg < 1)
        throw std::runtime_error("scan_ivf: bad parameters");
    void* tok;
    prof_begin(pass == kPassSample ? kFamIvfBound : kFamIvfScan, s, &tok);
    if (tiled) {
        if (storage == kF32) launch_tiled_ivf_s<kF32>(p, metric, pass, grid, s);
        else if (storage == kF16) launch_tiled_ivf_s<kF16>(p, metric, pass, grid, s);
        else launch_tiled_ivf_s<kBF16>(p, metric, pass, grid, s);
        prof_end(tok, s);
        check_launch("scan_ivf_tiled");
        return;
    }
    const size_t lds = resident_lds_bytes(p.dpad, storage, tileQueries);
    const int nb = tileQueries / 32;
    if (storage == kF32) launch_ivf_s<kF32>(p, metric, pass, nb, grid, lds, s);
    else if (storage == kF16) launch_ivf_s<kF16>(p, metric, pass, nb, grid, lds, s);
    else launch_ivf_s<kBF16>(p, metric, pass, nb, grid, lds, s);
    prof_end(tok, s);
    check_launch("scan_ivf");
}

void launch_argmin_finalize(const unsigned long long* best, int nq, int metric, int32_t* ids, float* vals,
                            hipStream_t s) {
    if (nq <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    argmin_finalize_kernel<<<(nq + 255) / 256, 256, 0, s>>>(best, nq, metric, ids, vals);
    prof_end(tok, s);
    check_launch("argmin_finalize");
}

void launch_fill_u64(unsigned long long* p, int64_t n, unsigned long long v, hipStream_t s) {
    if (n <= 0) return;
    void* tok;
    prof_begin(kFamPrep, s, &tok);
    fill_u64_kernel<<<grid_for(n, 256), 256, 0, s>>>(p, n, v);
    prof_end(tok, s);
    check_launch("fill_u64");
}

// A query's candidates are staged in LDS when they fit (else read from global
// memory on every pass): the small buffer runs ~2.5x more blocks per CU, for
// searches that expect few candidates per query. A batch of at most one block
// per CU loses nothing to the large buffer's occupancy (one block per CU): it
// keeps the ~j nb / R0 survivors of a small batch's full pass in LDS.
template <int KT>
static void launch_select_kt(const SelectParams& p, size_t dyn, hipStream_t s) {
    if (p.expect > 0 && p.expect <= kSelLdsSmall)
        select_kernel<kSelLdsSmall, KT><<<p.nq, 256, dyn, s>>>(p);
    else if (p.expect > 0 && p.expect <= kSelLdsMid)
        select_kernel<kSelLdsMid, KT><<<p.nq, 256, dyn, s>>>(p);
    else if (p.nq <= 256 && p.nsplit <= kSelLargeMaxSplit && !(p.expect > 0 && p.expect <= kSelLds))
        select_kernel<kSelLdsLarge, KT><<<p.nq, 256, dyn, s>>>(p);
    else
        select_kernel<kSelLds, KT><<<p.nq, 256, dyn, s>>>(p);
}

// ---------------------------------------------------------------------------
// merge_lists: exact top-k of the streaming scan's per-split lists
// ---------------------------------------------------------------------------
//
// One workgroup per query; region (q, s) holds cnt[q, s] <= cap <=
// kStreamTopK composites in ascending order (the streaming scan's per-split
// top-k). A k-way merge in two levels: lane s holds region s in registers;
// each wave takes k rounds of "smallest head of its 64 lanes" (composites are
// distinct: a row is in one split, so exactly one lane owns the minimum and
// shifts its list), leaving the wave's ascending top-k in LDS; wave 0 then
// merges the 16 wave lists the same way into the query's output.
constexpr int kMergeThreads = kMergeMaxSplit;   // a list per thread

// Minimum of x over the wave: DPP steps within each 16-lane row (swap
// neighbours, swap pairs, reverse 8, reverse 16), then the four rows' results
// read from lanes 0, 16, 32, 48.
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_min_step(uint64_t x) {
    const uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
    const uint32_t lo2 = (uint32_t)__builtin_amdgcn_update_dpp((int)lo, (int)lo, CTRL, 0xf, 0xf, false);
    const uint32_t hi2 = (uint32_t)__builtin_amdgcn_update_dpp((int)hi, (int)hi, CTRL, 0xf, 0xf, false);
    const uint64_t y = ((uint64_t)hi2 << 32) | lo2;
    return y < x ? y : x;
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t x) {
    x = dpp_min_step<0xB1>(x);    // quad_perm [1, 0, 3, 2]
    x = dpp_min_step<0x4E>(x);    // quad_perm [2, 3, 0, 1]
    x = dpp_min_step<0x141>(x);   // row_half_mirror
    x = dpp_min_step<0x140>(x);   // row_mirror
    uint64_t m = ~0ull;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint64_t y = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), 16 * r) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, 16 * r);
        m = y < m ? y : m;
    }
    return m;
}

// k rounds over the lanes' ascending lists, each lane holding its list's
// head (~0: empty): round r's smallest head goes to emit(r, m) and its lane
// replaces the head with pop(); stops early once every list is empty.
template <class Pop, class Emit>
__device__ __forceinline__ void wave_merge(uint64_t head, int k, Pop&& pop, Emit&& emit) {
    for (int r = 0; r < k; ++r) {
        const uint64_t m = wave_min_u64(head);
        if (m == ~0ull) return;
        if (head == m) head = pop();
        emit(r, m);
    }
}

// KT: entries a region holds at most (cap <= KT): 16 for k <= 16, else
// kStreamTopK. With KT = 16 a lane's entries past the head wait in LDS
// (entry e of lane t at sTail[(e - 1) * kMergeThreads + t]: 120 KB); with 32
// they stay in registers and a pop shifts them.
template <int KT>
__global__ void __launch_bounds__(kMergeThreads) merge_lists_kernel(SelectParams p) {
    constexpr int NW = kMergeThreads / 64;
    constexpr bool TAIL_LDS = KT <= 16;
    __shared__ uint64_t sTail[TAIL_LDS ? (KT - 1) * kMergeThreads : 1];
    __shared__ uint64_t sWave[NW][KT];

    const int q = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int k = p.k;

    uint64_t v[KT];
    int c;
    {
        // every lane loads from a valid address (lanes past the last region
        // re-read it, entries past cap re-read the last one) so that the
        // loads issue back to back, unpredicated; masks apply afterwards
        const int sidx = tid < p.nsplit ? tid : p.nsplit - 1;
        const uint2* reg = p.cand + ((int64_t)q * p.nsplit + sidx) * p.cap;
        c = p.cnt[(int64_t)q * p.nsplit + sidx];
        uint2 raw[KT];
#pragma unroll
        for (int e = 0; e < KT; ++e) raw[e] = reg[e < p.cap ? e : p.cap - 1];
        c = tid < p.nsplit ? (c < p.cap ? c : p.cap) : 0;
#pragma unroll
        for (int e = 0; e < KT; ++e) v[e] = e < c ? composite(raw[e]) : ~0ull;
    }
    if constexpr (TAIL_LDS) {
#pragma unroll
        for (int e = 1; e < KT; ++e) sTail[(e - 1) * kMergeThreads + tid] = v[e];
    }
    if (lane < KT) sWave[wave][lane] = ~0ull;
    __builtin_amdgcn_wave_barrier();
    int h = 0;
    auto pop1 = [&]() -> uint64_t {
        ++h;
        if constexpr (TAIL_LDS) {
            return h < c ? sTail[(h - 1) * kMergeThreads + tid] : ~0ull;
        } else {
#pragma unroll
            for (int e = 0; e + 1 < KT; ++e) v[e] = v[e + 1];
            v[KT - 1] = ~0ull;
            return v[0];
        }
    };
    wave_merge(v[0], k, pop1, [&](int r, uint64_t m) {
        if (lane == 0) sWave[wave][r] = m;
    });
    __syncthreads();
    if (wave != 0) return;

    // wave 0: lane l < NW merges wave l's ascending list
    int h2 = 0;
    const int src = lane < NW ? lane : 0;
    auto pop2 = [&]() -> uint64_t {
        ++h2;
        return h2 < KT ? sWave[src][h2] : ~0ull;
    };
    const uint64_t head2 = lane < NW ? sWave[src][0] : ~0ull;
    const int orow = p.qmap ? p.qmap[q] : q;
    int got = 0;
    wave_merge(head2, k, pop2, [&](int r, uint64_t m) {
        got = r + 1;
        if (lane == 0) {
            const float key = ord_to_key((uint32_t)(m >> 32));
            if (p.out_ids) p.out_ids[(int64_t)orow * p.out_stride + r] = (int32_t)(uint32_t)(m & 0xFFFFFFFFu);
            if (p.out_vals) p.out_vals[(int64_t)orow * p.out_stride + r] = p.metric == 0 ? key : -key;
        }
    });
    // fewer than k rows in the whole database: padding
    for (int i = got + lane; i < k; i += 64) {
        if (p.out_ids) p.out_ids[(int64_t)orow * p.out_stride + i] = -1;
        if (p.out_vals) p.out_vals[(int64_t)orow * p.out_stride + i] = p.metric == 0 ? INFINITY : -INFINITY;
    }
}

void launch_merge_lists(const SelectParams& p, hipStream_t s) {
    if (p.nq <= 0) return;
    if (p.k < 1 || p.k > p.cap || p.cap > kStreamTopK || p.nsplit < 1 || p.nsplit > kMergeThreads)
        throw std::runtime_error("merge_lists: bad k/cap/nsplit");
    void* tok;
    prof_begin(kFamSelect, s, &tok);
    if (p.cap <= 16) merge_lists_kernel<16><<<p.nq, kMergeThreads, 0, s>>>(p);
    else merge_lists_kernel<kStreamTopK><<<p.nq, kMergeThreads, 0, s>>>(p);
    prof_end(tok, s);
    check_launch("merge_lists");
}

void launch_select(const SelectParams& p, hipStream_t s) {
    if (p.nq <= 0) return;
    if (p.k < 1 || p.k > kTopMax || p.j < 1 || p.j > p.k || p.j2 < 1 || p.j2 > p.k)
        throw std::runtime_error("select: bad k/j");
    if (p.nsplit < 1 || p.nsplit > kMaxSplit) throw std::runtime_error("select: bad nsplit");
    // the split offsets (dynamic LDS) reach (kMaxSplit + 1) ints, above the
    // default dynamic-LDS limit of a launch
    static const bool attr = [] {
        const std::pair<const void*, int> fs[] = {
            {(const void*)select_kernel<kSelLds, kTopMax>, kMaxSplit},
            {(const void*)select_kernel<kSelLdsSmall, kTopMax>, kMaxSplit},
            {(const void*)select_kernel<kSelLdsMid, kTopMax>, kMaxSplit},
            {(const void*)select_kernel<kSelLdsLarge, kTopMax>, kSelLargeMaxSplit},
            {(const void*)select_kernel<kSelLds, kTopSmall>, kMaxSplit},
            {(const void*)select_kernel<kSelLdsSmall, kTopSmall>, kMaxSplit},
            {(const void*)select_kernel<kSelLdsMid, kTopSmall>, kMaxSplit},
            {(const void*)select_kernel<kSelLdsLarge, kTopSmall>, kSelLargeMaxSplit}};
        for (const auto& f : fs)
            if (hipFuncSetAttribute(f.first, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)((f.second + 1) * sizeof(int))) != hipSuccess)
                throw std::runtime_error("select: cannot raise the dynamic LDS limit");
        return true;
    }();
    (void)attr;
    void* tok;
    prof_begin(kFamSelect, s, &tok);
    const size_t dyn = (size_t)(p.nsplit + 1) * sizeof(int);
    // k <= 256: a 2 KB winner buffer instead of 8 KB (select_kernel<1024>:
    // ~12 KB of LDS a block, ~13 blocks per CU instead of 8)
    if (p.k <= kTopSmall) launch_select_kt<kTopSmall>(p, dyn, s);
    else launch_select_kt<kTopMax>(p, dyn, s);
    prof_end(tok, s);
    check_launch("select");
}

}  // namespace mflat_amd
