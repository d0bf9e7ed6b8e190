/* SPDX-License-Identifier: Apache-2.0
 *
 * flat_oracle.c -- TEST INFRASTRUCTURE ONLY. CPU restatement of the reference's
 * exact flat-search algorithm, used as the parity checker for the HIP library
 * and as the CPU baseline timed by bench.py. Nothing in the product library
 * (metal-flat_amd/) links, loads or calls this file.
 *
 * Every function follows a reference function line by line in semantics
 * (loop order, accumulation type, comparison strictness), written from scratch:
 *
 *   orc_dot              src/Distance.h:26-30   float accumulation, c ascending
 *   orc_sql2             src/Distance.h:33-37   float accumulation of (a-b)^2
 *   orc_row_sq_norms     src/Distance.h:40-47   double accumulation, cast to float
 *   orc_normalize_rows   src/Distance.h:50-60   double sum, inv = float(1/sqrt(s))
 *   orc_cpu_search       src/FlatIndex.mm:259-290 (cpuSearch) with score()
 *                        src/Distance.h:67-75: running top-k ascending, strict '>'
 *                        insertion, reversal to nearest-first, -1 / +-inf padding
 *   orc_flat_search      src/FlatIndex.mm:236-245 + 294-321: FlatIndex::add/search
 *                        semantics (Cosine normalises db rows and a query copy)
 *                        without the kMaxK clamp (k is generic in cpuSearch)
 *   orc_argmin_l2        src/CoarseQuantizer.mm:122-131 strict '<' argmin
 *                        (k = 1 assignment; must agree with orc_cpu_search k=1)
 *   orc_brute_lex        bench/bench.mm:52-64 cpuTopkL2: partial sort of
 *                        (dist, id) pairs -- an independent cross-check
 *   orc_kmeans_update    src/CoarseQuantizer.mm:44-66 (k-means update): per-cell
 *                        double sums over the points in ascending index order,
 *                        centroid = float(sum / count); an empty cell copies
 *                        the row its reseed entry names
 *   orc_ivf_search       src/IvfIndex.mm:518-560 (searchCpu, with the caller's
 *                        probed cells as its probedRows): per query, a running
 *                        top-k over the rows of its cells in probe order (rows
 *                        lo..hi of the cell-ordered payload), strict '>'
 *                        insertion, ids through reorderedIds, cells < 0 skipped
 *   orc_ivfpq_search     src/IvfPqIndex.mm:383-445 (searchCpu, residual mode) with
 *                        the tables of src/PqTrainer.h:84-116: lut = ||p||^2 -
 *                        2 q_m.p, T = 2 c_m.p, base = sqL2(q, c); dist = base +
 *                        sum_m (lut + T) in ascending m; strict '>' on -dist;
 *                        value = dist
 *   orc_pq_rerank        src/IvfPqIndex.mm:598-625: exact score over a shortlist,
 *                        strict '>' in shortlist order, -1 entries skipped
 *
 * Build with -ffp-contract=off so no multiply-add is fused: the sums are the
 * plain sequential fp32 sums the reference's C++ source spells out.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_L2 0
#define ORC_IP 1
#define ORC_COS 2

float orc_dot(const float* a, const float* b, int dim) {
    float acc = 0.0f;
    for (int c = 0; c < dim; ++c) acc += a[c] * b[c];
    return acc;
}

float orc_sql2(const float* a, const float* b, int dim) {
    float acc = 0.0f;
    for (int c = 0; c < dim; ++c) {
        float e = a[c] - b[c];
        acc += e * e;
    }
    return acc;
}

void orc_row_sq_norms(const float* v, int64_t n, int dim, float* out) {
    for (int64_t i = 0; i < n; ++i) {
        const float* row = v + i * dim;
        double s = 0.0;
        for (int c = 0; c < dim; ++c) s += (double)row[c] * row[c];
        out[i] = (float)s;
    }
}

void orc_normalize_rows(float* v, int64_t n, int dim) {
    for (int64_t i = 0; i < n; ++i) {
        float* row = v + i * dim;
        double s = 0.0;
        for (int c = 0; c < dim; ++c) s += (double)row[c] * row[c];
        if (s > 0.0) {
            const float inv = (float)(1.0 / sqrt(s));
            for (int c = 0; c < dim; ++c) row[c] *= inv;
        }
    }
}

/* Ranking score, larger = nearer: L2 -> -sqL2, IP/Cosine -> dot. */
static inline float orc_score(int metric, const float* q, const float* x, int dim) {
    return metric == ORC_L2 ? -orc_sql2(q, x, dim) : orc_dot(q, x, dim);
}
static inline float orc_score_to_value(int metric, float s) {
    return metric == ORC_L2 ? -s : s;
}

/* One query of cpuSearch. best_s/best_i: scratch of k entries. */
static void orc_search_one(const float* db, int64_t nb, int dim, int metric,
                           const float* q, int k, float* best_s, int32_t* best_i,
                           int32_t* out_ids, float* out_vals) {
    for (int i = 0; i < k; ++i) { best_s[i] = -INFINITY; best_i[i] = -1; }
    for (int64_t j = 0; j < nb; ++j) {
        const float s = orc_score(metric, q, db + j * dim, dim);
        if (s > best_s[0]) {
            int pos = 0;
            while (pos + 1 < k && s > best_s[pos + 1]) {
                best_s[pos] = best_s[pos + 1];
                best_i[pos] = best_i[pos + 1];
                ++pos;
            }
            best_s[pos] = s;
            best_i[pos] = (int32_t)j;
        }
    }
    for (int i = 0; i < k; ++i) {
        const int src = k - 1 - i;
        out_ids[i] = best_i[src];
        /* unfilled slots keep -inf -> value +inf (L2) / -inf (IP), which is
           emptyValue() of src/Distance.h:73-75 */
        out_vals[i] = orc_score_to_value(metric, best_s[src]);
    }
}

typedef struct {
    const float* db; int64_t nb; int dim; int metric;
    const float* q; int k; int32_t* ids; float* vals;
    int64_t lo, hi; int status;
} orc_job_t;

static void* orc_worker(void* arg) {
    orc_job_t* j = (orc_job_t*)arg;
    float* bs = (float*)malloc(sizeof(float) * (size_t)j->k);
    int32_t* bi = (int32_t*)malloc(sizeof(int32_t) * (size_t)j->k);
    if (!bs || !bi) { free(bs); free(bi); j->status = -1; return NULL; }
    for (int64_t qi = j->lo; qi < j->hi; ++qi)
        orc_search_one(j->db, j->nb, j->dim, j->metric, j->q + qi * j->dim, j->k, bs, bi,
                       j->ids + qi * j->k, j->vals + qi * j->k);
    free(bs); free(bi);
    j->status = 0;
    return NULL;
}

/* cpuSearch over already-prepared rows (metric: 0 L2, 1 IP; Cosine callers pass
   normalised rows with metric 1). threads <= 1 runs the reference's serial loop
   on the calling thread; more threads split the queries in contiguous chunks
   (as bench/bench.mm:134-156 does for its baseline). Returns 0 on success. */
int orc_cpu_search(const float* db, int64_t nb, int dim, int metric, const float* q,
                   int64_t m, int k, int32_t* out_ids, float* out_vals, int threads) {
    if (k < 1 || m < 0 || dim <= 0) return -2;
    const int sm = (metric == ORC_L2) ? ORC_L2 : ORC_IP;
    if (threads <= 1 || m < 2) {
        orc_job_t j = {db, nb, dim, sm, q, k, out_ids, out_vals, 0, m, 0};
        orc_worker(&j);
        return j.status;
    }
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    orc_job_t jobs[256];
    const int64_t chunk = (m + threads - 1) / threads;
    int started = 0, rc = 0;
    for (int t = 0; t < threads; ++t) {
        const int64_t lo = (int64_t)t * chunk;
        const int64_t hi = lo + chunk < m ? lo + chunk : m;
        if (lo >= hi) break;
        orc_job_t jj = {db, nb, dim, sm, q, k, out_ids, out_vals, lo, hi, 0};
        jobs[t] = jj;
        if (pthread_create(&tid[t], NULL, orc_worker, &jobs[t]) != 0) { rc = -1; break; }
        ++started;
    }
    for (int t = 0; t < started; ++t) {
        pthread_join(tid[t], NULL);
        if (jobs[t].status != 0) rc = -1;
    }
    return rc;
}

/* FlatIndex::add + FlatIndex::search semantics (unclamped k): Cosine stores
   normalised copies of the rows and normalises a copy of the queries, then
   ranks by the dot product. Returns 0 on success. */
int orc_flat_search(const float* db, int64_t nb, int dim, int metric, const float* q,
                    int64_t m, int k, int32_t* out_ids, float* out_vals, int threads) {
    if (metric != ORC_COS)
        return orc_cpu_search(db, nb, dim, metric, q, m, k, out_ids, out_vals, threads);
    float* dbn = (float*)malloc(sizeof(float) * (size_t)(nb > 0 ? nb : 1) * dim);
    float* qn = (float*)malloc(sizeof(float) * (size_t)(m > 0 ? m : 1) * dim);
    if (!dbn || !qn) { free(dbn); free(qn); return -1; }
    memcpy(dbn, db, sizeof(float) * (size_t)nb * dim);
    memcpy(qn, q, sizeof(float) * (size_t)m * dim);
    orc_normalize_rows(dbn, nb, dim);
    orc_normalize_rows(qn, m, dim);
    const int rc = orc_cpu_search(dbn, nb, dim, ORC_IP, qn, m, k, out_ids, out_vals, threads);
    free(dbn); free(qn);
    return rc;
}

/* Strict '<' argmin of the squared L2 distance (lowest index wins ties). */
void orc_argmin_l2(const float* pts, int64_t n, const float* cents, int64_t c, int dim,
                   int32_t* out_ids, float* out_d) {
    for (int64_t i = 0; i < n; ++i) {
        float best = INFINITY;
        int32_t bc = 0;
        for (int64_t j = 0; j < c; ++j) {
            const float d = orc_sql2(pts + i * dim, cents + j * dim, dim);
            if (d < best) { best = d; bc = (int32_t)j; }
        }
        out_ids[i] = bc;
        out_d[i] = best;
    }
}

/* Independent cross-check: full lexicographic (dist, id) sort per query, L2. */
typedef struct { float d; int32_t id; } orc_pair_t;
static int orc_pair_cmp(const void* a, const void* b) {
    const orc_pair_t* x = (const orc_pair_t*)a;
    const orc_pair_t* y = (const orc_pair_t*)b;
    if (x->d < y->d) return -1;
    if (x->d > y->d) return 1;
    return (x->id > y->id) - (x->id < y->id);
}
int orc_brute_lex(const float* db, int64_t nb, int dim, const float* q, int64_t m, int k,
                  int32_t* out_ids, float* out_vals) {
    orc_pair_t* all = (orc_pair_t*)malloc(sizeof(orc_pair_t) * (size_t)(nb > 0 ? nb : 1));
    if (!all) return -1;
    for (int64_t qi = 0; qi < m; ++qi) {
        for (int64_t j = 0; j < nb; ++j) {
            all[j].d = orc_sql2(q + qi * dim, db + j * dim, dim);
            all[j].id = (int32_t)j;
        }
        qsort(all, (size_t)nb, sizeof(orc_pair_t), orc_pair_cmp);
        for (int i = 0; i < k; ++i) {
            out_ids[qi * k + i] = i < nb ? all[i].id : -1;
            out_vals[qi * k + i] = i < nb ? all[i].d : INFINITY;
        }
    }
    free(all);
    return 0;
}

void orc_kmeans_update(const float* pts, int64_t n, int dim, const int32_t* assign, int nlist,
                       const int32_t* reseed, float* centroids) {
    double* sums = (double*)calloc((size_t)nlist * dim, sizeof(double));
    int64_t* counts = (int64_t*)calloc((size_t)nlist, sizeof(int64_t));
    if (!sums || !counts) { free(sums); free(counts); return; }
    for (int64_t i = 0; i < n; ++i) {
        const float* v = pts + i * dim;
        double* sc = sums + (int64_t)assign[i] * dim;
        for (int d = 0; d < dim; ++d) sc[d] += v[d];
        ++counts[assign[i]];
    }
    for (int c = 0; c < nlist; ++c) {
        float* ce = centroids + (int64_t)c * dim;
        if (counts[c] > 0) {
            for (int d = 0; d < dim; ++d) ce[d] = (float)(sums[(int64_t)c * dim + d] / (double)counts[c]);
        } else {
            memcpy(ce, pts + (int64_t)reseed[c] * dim, (size_t)dim * sizeof(float));
        }
    }
    free(sums);
    free(counts);
}

/* IVF fine scan (searchCpu): rdb = the rows in cell order (row j of cell c is
   payload row cellStart[c] + j, i.e. reorderedDb), rid = reorderedIds, probed =
   m x nprobe cells nearest first. metric 0 L2, otherwise dot (Cosine callers
   pass normalised rows and queries). threads as orc_cpu_search. */
typedef struct {
    const float* rdb; const int32_t* rid; const int32_t* cs; int dim; int metric;
    const float* q; const int32_t* probed; int nprobe; int k;
    int32_t* ids; float* vals; int64_t lo, hi; int status;
} orc_ivf_job_t;

static void* orc_ivf_worker(void* arg) {
    orc_ivf_job_t* j = (orc_ivf_job_t*)arg;
    float* bs = (float*)malloc(sizeof(float) * (size_t)j->k);
    int32_t* bi = (int32_t*)malloc(sizeof(int32_t) * (size_t)j->k);
    if (!bs || !bi) { free(bs); free(bi); j->status = -1; return NULL; }
    for (int64_t qi = j->lo; qi < j->hi; ++qi) {
        const float* q = j->q + qi * j->dim;
        for (int i = 0; i < j->k; ++i) { bs[i] = -INFINITY; bi[i] = -1; }
        for (int pp = 0; pp < j->nprobe; ++pp) {
            const int32_t c = j->probed[qi * j->nprobe + pp];
            if (c < 0) continue;
            for (int64_t r = j->cs[c]; r < j->cs[c + 1]; ++r) {
                const float s = orc_score(j->metric, q, j->rdb + r * j->dim, j->dim);
                if (s > bs[0]) {
                    int pos = 0;
                    while (pos + 1 < j->k && s > bs[pos + 1]) {
                        bs[pos] = bs[pos + 1];
                        bi[pos] = bi[pos + 1];
                        ++pos;
                    }
                    bs[pos] = s;
                    bi[pos] = j->rid[r];
                }
            }
        }
        for (int i = 0; i < j->k; ++i) {
            const int src = j->k - 1 - i;
            j->ids[qi * j->k + i] = bi[src];
            j->vals[qi * j->k + i] = orc_score_to_value(j->metric, bs[src]);
        }
    }
    free(bs); free(bi);
    j->status = 0;
    return NULL;
}

int orc_ivf_search(const float* rdb, const int32_t* rid, const int32_t* cell_start, int dim, int metric,
                   const float* q, int64_t m, const int32_t* probed, int nprobe, int k,
                   int32_t* out_ids, float* out_vals, int threads) {
    if (k < 1 || m < 0 || dim <= 0 || nprobe < 1) return -2;
    const int sm = (metric == ORC_L2) ? ORC_L2 : ORC_IP;
    if (threads <= 1 || m < 2) {
        orc_ivf_job_t j = {rdb, rid, cell_start, dim, sm, q, probed, nprobe, k, out_ids, out_vals, 0, m, 0};
        orc_ivf_worker(&j);
        return j.status;
    }
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    orc_ivf_job_t jobs[256];
    const int64_t chunk = (m + threads - 1) / threads;
    int started = 0, rc = 0;
    for (int t = 0; t < threads; ++t) {
        const int64_t lo = (int64_t)t * chunk;
        const int64_t hi = lo + chunk < m ? lo + chunk : m;
        if (lo >= hi) break;
        orc_ivf_job_t jj = {rdb, rid, cell_start, dim, sm, q, probed, nprobe, k, out_ids, out_vals, lo, hi, 0};
        jobs[t] = jj;
        if (pthread_create(&tid[t], NULL, orc_ivf_worker, &jobs[t]) != 0) { rc = -1; break; }
        ++started;
    }
    for (int t = 0; t < started; ++t) {
        pthread_join(tid[t], NULL);
        if (jobs[t].status != 0) rc = -1;
    }
    return rc;
}

/* IVF-PQ ADC search (residual). cent nlist x dim; cs/rid the CSR; codes n x M
   bytes in cell order; pqc M x 256 x dsub. q already normalised for Cosine. */
typedef struct {
    const float* cent; const int32_t* cs; const int32_t* rid; const uint8_t* codes; const float* pqc;
    const float* norms; const float* T; int M; int dsub; int dim;
    const float* q; const int32_t* probed; int nprobe; int k;
    int32_t* ids; float* vals; int64_t lo, hi; int status;
} orc_pq_job_t;

static void* orc_pq_worker(void* arg) {
    orc_pq_job_t* j = (orc_pq_job_t*)arg;
    const int M = j->M, K = 256;
    float* lut = (float*)malloc(sizeof(float) * (size_t)M * K);
    float* bs = (float*)malloc(sizeof(float) * (size_t)j->k);
    int32_t* bi = (int32_t*)malloc(sizeof(int32_t) * (size_t)j->k);
    if (!lut || !bs || !bi) { free(lut); free(bs); free(bi); j->status = -1; return NULL; }
    for (int64_t qi = j->lo; qi < j->hi; ++qi) {
        const float* q = j->q + qi * j->dim;
        for (int mm = 0; mm < M; ++mm)
            for (int c = 0; c < K; ++c)
                lut[mm * K + c] = j->norms[mm * K + c] -
                                  2.0f * orc_dot(q + mm * j->dsub, j->pqc + ((int64_t)mm * K + c) * j->dsub, j->dsub);
        for (int i = 0; i < j->k; ++i) { bs[i] = -INFINITY; bi[i] = -1; }
        for (int pp = 0; pp < j->nprobe; ++pp) {
            const int32_t c = j->probed[qi * j->nprobe + pp];
            if (c < 0) continue;
            const float base = orc_sql2(q, j->cent + (int64_t)c * j->dim, j->dim);
            const float* Tc = j->T + (int64_t)c * M * K;
            for (int64_t r = j->cs[c]; r < j->cs[c + 1]; ++r) {
                const uint8_t* code = j->codes + r * M;
                float dist = base;
                for (int mm = 0; mm < M; ++mm) dist += lut[mm * K + code[mm]] + Tc[mm * K + code[mm]];
                const float s = -dist;
                if (s > bs[0]) {
                    int pos = 0;
                    while (pos + 1 < j->k && s > bs[pos + 1]) {
                        bs[pos] = bs[pos + 1];
                        bi[pos] = bi[pos + 1];
                        ++pos;
                    }
                    bs[pos] = s;
                    bi[pos] = j->rid[r];
                }
            }
        }
        for (int i = 0; i < j->k; ++i) {
            const int src = j->k - 1 - i;
            j->ids[qi * j->k + i] = bi[src];
            j->vals[qi * j->k + i] = -bs[src];
        }
    }
    free(lut); free(bs); free(bi);
    j->status = 0;
    return NULL;
}

int orc_ivfpq_search(const float* cent, int nlist, const int32_t* cs, const int32_t* rid, const uint8_t* codes,
                     const float* pqc, int M, int dim, const float* q, int64_t m, const int32_t* probed, int nprobe,
                     int k, int32_t* out_ids, float* out_vals, int threads) {
    if (k < 1 || m < 0 || dim <= 0 || M <= 0 || dim % M != 0 || nprobe < 1) return -2;
    const int dsub = dim / M, K = 256;
    float* norms = (float*)malloc(sizeof(float) * (size_t)M * K);
    float* T = (float*)malloc(sizeof(float) * (size_t)nlist * M * K);
    if (!norms || !T) { free(norms); free(T); return -1; }
    for (int e = 0; e < M * K; ++e) norms[e] = orc_dot(pqc + (int64_t)e * dsub, pqc + (int64_t)e * dsub, dsub);
    for (int c = 0; c < nlist; ++c)
        for (int mm = 0; mm < M; ++mm)
            for (int jj = 0; jj < K; ++jj)
                T[((int64_t)c * M + mm) * K + jj] =
                    2.0f * orc_dot(cent + (int64_t)c * dim + mm * dsub, pqc + ((int64_t)mm * K + jj) * dsub, dsub);
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    orc_pq_job_t jobs[256];
    const int64_t chunk = (m + threads - 1) / threads;
    int started = 0, rc = 0;
    for (int t = 0; t < threads; ++t) {
        const int64_t lo = (int64_t)t * chunk;
        const int64_t hi = lo + chunk < m ? lo + chunk : m;
        if (lo >= hi) break;
        orc_pq_job_t jj = {cent, cs, rid, codes, pqc, norms, T, M, dsub, dim, q, probed, nprobe, k,
                           out_ids, out_vals, lo, hi, 0};
        jobs[t] = jj;
        if (threads == 1) { orc_pq_worker(&jobs[t]); started = -1; break; }
        if (pthread_create(&tid[t], NULL, orc_pq_worker, &jobs[t]) != 0) { rc = -1; break; }
        ++started;
    }
    if (started < 0) rc = jobs[0].status;
    for (int t = 0; t < started; ++t) {
        pthread_join(tid[t], NULL);
        if (jobs[t].status != 0) rc = -1;
    }
    free(norms); free(T);
    return rc;
}

/* Exact rerank of a shortlist (nq x kRun ids, -1 skipped): metric 0 L2 (score
   -sqL2), otherwise dot; k best by strict '>' in shortlist order; value =
   scoreToValue (sqL2 / dot; unfilled +inf / -inf). */
int orc_pq_rerank(const float* full, int dim, int metric, const float* q, int64_t m, const int32_t* shortIds,
                  int kRun, int k, int32_t* out_ids, float* out_vals) {
    float* bs = (float*)malloc(sizeof(float) * (size_t)k);
    int32_t* bi = (int32_t*)malloc(sizeof(int32_t) * (size_t)k);
    if (!bs || !bi) { free(bs); free(bi); return -1; }
    const int sm = metric == ORC_L2 ? ORC_L2 : ORC_IP;
    for (int64_t qi = 0; qi < m; ++qi) {
        for (int i = 0; i < k; ++i) { bs[i] = -INFINITY; bi[i] = -1; }
        for (int i = 0; i < kRun; ++i) {
            const int32_t id = shortIds[qi * kRun + i];
            if (id < 0) continue;
            const float s = orc_score(sm, q + qi * dim, full + (int64_t)id * dim, dim);
            if (s > bs[0]) {
                int pos = 0;
                while (pos + 1 < k && s > bs[pos + 1]) {
                    bs[pos] = bs[pos + 1];
                    bi[pos] = bi[pos + 1];
                    ++pos;
                }
                bs[pos] = s;
                bi[pos] = id;
            }
        }
        for (int i = 0; i < k; ++i) {
            const int src = k - 1 - i;
            out_ids[qi * k + i] = bi[src];
            out_vals[qi * k + i] = orc_score_to_value(sm, bs[src]);
        }
    }
    free(bs); free(bi);
    return 0;
}
