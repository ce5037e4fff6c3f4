/*
 * oracle.c -- CPU restatement of the MetalANNS exact-search hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker and the timed
 * CPU baseline.  Nothing in the shipped library links or calls it; only the
 * tests, the smoke check and the benchmark's CPU-baseline leg load it.
 *
 * Arithmetic follows the reference's Swift/C sources statement by statement
 * (citations are to files of the reference repository).  Where the reference
 * calls Apple Accelerate (vDSP / BLAS), whose summation order is not
 * published, this file uses the scalar left-to-right order of
 * Sources/MetalANNSC/dots.c:40-47 and says so at the call site; results at
 * those points are pinned by tolerance against the reference's tests, not
 * bit for bit.  Compiled with -ffp-contract=off so no multiply-add is fused,
 * which is how dots.c executes on x86-64.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_EXPORT __attribute__((visibility("default")))

enum { METRIC_COSINE = 0, METRIC_L2 = 1, METRIC_IP = 2, METRIC_HAMMING = 3 };

/* ------------------------------------------------------------------------ */
/* Dot kernels: Sources/MetalANNSC/dots.c, scalar branch (x86 build).        */
/* ------------------------------------------------------------------------ */

/* dots.c:40-47 */
ORC_EXPORT void orc_f32_dot_rows(const float *corpus, const float *query, int64_t rows,
                                 int64_t dim, float *out) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *row = corpus + r * dim;
        float acc = 0.0f;
        for (int64_t d = 0; d < dim; ++d) acc += row[d] * query[d];
        out[r] = acc;
    }
}

/* dots.c:50-88 (int32 accumulation, one conversion) */
ORC_EXPORT void orc_i8_dot_rows_f32(const int8_t *codes, const int8_t *qcodes, int64_t rows,
                                    int64_t dim, float *out) {
    for (int64_t r = 0; r < rows; ++r) {
        const int8_t *row = codes + r * dim;
        int32_t total = 0;
        for (int64_t d = 0; d < dim; ++d) total += (int32_t)row[d] * (int32_t)qcodes[d];
        out[r] = (float)total;
    }
}

/* dots.c:90-125 scalar branch */
ORC_EXPORT void orc_f32_dot_rows_gather(const float *corpus, const float *query,
                                        const uint32_t *idx, int64_t count, int64_t dim,
                                        float *out) {
    for (int64_t i = 0; i < count; ++i) {
        const float *row = corpus + (int64_t)idx[i] * dim;
        float acc = 0.0f;
        for (int64_t d = 0; d < dim; ++d) acc += row[d] * query[d];
        out[i] = acc;
    }
}

/* Squared row norms.  The reference uses vDSP_vsq + cblas_sgemv
 * (FlatGPUSearch.swift:484-501), whose order is unpublished; this is the
 * sequential order (parity at this point: tolerance only). */
ORC_EXPORT void orc_row_norms(const float *corpus, int64_t n, int64_t dim, float *out) {
    for (int64_t r = 0; r < n; ++r) {
        const float *row = corpus + r * dim;
        float acc = 0.0f;
        for (int64_t d = 0; d < dim; ++d) acc += row[d] * row[d];
        out[r] = acc;
    }
}

/* Query squared norm: FlatGPUSearch.swift:532-535 (sequential Swift loop). */
ORC_EXPORT float orc_query_norm(const float *q, int64_t dim) {
    float s = 0.0f;
    for (int64_t d = 0; d < dim; ++d) s += q[d] * q[d];
    return s;
}

/* Host distance formulas: ParallelFlatScan.swift:237-257,
 * BoundedExactScan.swift:346-363, IVFFlatSearch.swift:294-311. */
static inline float host_distance(float dot, float qn, float vn, int metric) {
    switch (metric) {
    case METRIC_IP:
        return -dot;
    case METRIC_L2: {
        float d = qn - 2.0f * dot + vn;
        return d > 0.0f ? d : 0.0f;
    }
    case METRIC_COSINE: {
        float denom = sqrtf(qn * vn);
        return denom < 1e-10f ? 1.0f : 1.0f - dot / denom;
    }
    default:
        return 3.4028234663852886e38f;
    }
}

ORC_EXPORT float orc_host_distance(float dot, float qn, float vn, int metric) {
    return host_distance(dot, qn, vn, metric);
}

/* ------------------------------------------------------------------------ */
/* Small parallel-for on pthreads (the reference uses concurrentPerform).     */
/* ------------------------------------------------------------------------ */

typedef void (*task_fn)(void *ctx, int64_t index);

typedef struct {
    task_fn fn;
    void *ctx;
    int64_t count;
    int64_t next;
    pthread_mutex_t lock;
} pool_state;

static void *pool_worker(void *arg) {
    pool_state *p = (pool_state *)arg;
    for (;;) {
        pthread_mutex_lock(&p->lock);
        int64_t i = p->next++;
        pthread_mutex_unlock(&p->lock);
        if (i >= p->count) break;
        p->fn(p->ctx, i);
    }
    return NULL;
}

static void parallel_for(int64_t count, int threads, task_fn fn, void *ctx) {
    if (threads <= 1 || count <= 1) {
        for (int64_t i = 0; i < count; ++i) fn(ctx, i);
        return;
    }
    if (threads > 256) threads = 256;
    if (threads > count) threads = (int)count;
    pool_state p = {fn, ctx, count, 0, PTHREAD_MUTEX_INITIALIZER};
    pthread_t tids[256];
    int started = 0;
    for (int t = 0; t < threads - 1; ++t)
        if (pthread_create(&tids[started], NULL, pool_worker, &p) == 0) ++started;
    pool_worker(&p);
    for (int t = 0; t < started; ++t) pthread_join(tids[t], NULL);
}

/* ------------------------------------------------------------------------ */
/* ParallelFlatScan (ParallelFlatScan.swift:84-314)                          */
/* ------------------------------------------------------------------------ */

typedef struct {
    float distance;
    uint32_t id;
} entry;

/* ParallelFlatScan.swift:84-88 */
ORC_EXPORT int64_t orc_slice_count(int64_t n, int64_t cores) {
    int64_t by_work = n / 2048;
    if (by_work < 1) by_work = 1;
    int64_t s = cores;
    if (s > 32) s = 32;
    if (s > by_work) s = by_work;
    return s < 1 ? 1 : s;
}

/* Bounded max-heap on distance only (ParallelFlatScan.swift:201-235). */
static void heap_append(entry *h, int64_t *count, int64_t cap, float dist, uint32_t id) {
    if (*count < cap) {
        int64_t pos = (*count)++;
        h[pos].distance = dist;
        h[pos].id = id;
        while (pos > 0) {
            int64_t parent = (pos - 1) / 2;
            if (h[pos].distance > h[parent].distance) {
                entry t = h[pos];
                h[pos] = h[parent];
                h[parent] = t;
                pos = parent;
            } else {
                break;
            }
        }
    } else if (dist < h[0].distance) {
        h[0].distance = dist;
        h[0].id = id;
        int64_t pos = 0, n = *count;
        for (;;) {
            int64_t l = 2 * pos + 1, r = l + 1, largest = pos;
            if (l < n && h[l].distance > h[largest].distance) largest = l;
            if (r < n && h[r].distance > h[largest].distance) largest = r;
            if (largest == pos) break;
            entry t = h[pos];
            h[pos] = h[largest];
            h[largest] = t;
            pos = largest;
        }
    }
}

/* ParallelFlatScan.swift:266-285 */
static void heap_sorted_ascending(entry *h, int64_t count) {
    while (count > 1) {
        entry t = h[0];
        h[0] = h[count - 1];
        h[count - 1] = t;
        --count;
        int64_t pos = 0;
        for (;;) {
            int64_t l = 2 * pos + 1, r = l + 1, largest = pos;
            if (l < count && h[l].distance > h[largest].distance) largest = l;
            if (r < count && h[r].distance > h[largest].distance) largest = r;
            if (largest == pos) break;
            entry u = h[pos];
            h[pos] = h[largest];
            h[largest] = u;
            pos = largest;
        }
    }
}

/* ParallelFlatScan.swift:188-263 for one slice: dots then bounded heap. */
static int64_t scan_slice(const float *corpus, const float *norms, const float *q, float qn,
                          int64_t start, int64_t rows, int64_t dim, int64_t topk, int metric,
                          float *dots, entry *out) {
    orc_f32_dot_rows(corpus + start * dim, q, rows, dim, dots);
    int64_t count = 0;
    for (int64_t r = 0; r < rows; ++r) {
        float vn = norms ? norms[start + r] : 0.0f;
        heap_append(out, &count, topk, host_distance(dots[r], qn, vn, metric),
                    (uint32_t)(start + r));
    }
    heap_sorted_ascending(out, count);
    return count;
}

/* ParallelFlatScan.swift:288-314: first list with the strictly smaller head wins. */
static int64_t merge_sorted(entry **lists, const int64_t *lens, int64_t nlists, int64_t limit,
                            entry *out) {
    int64_t cursors[64] = {0};
    int64_t merged = 0;
    while (merged < limit) {
        int64_t best = -1;
        float bestd = INFINITY;
        for (int64_t i = 0; i < nlists; ++i) {
            if (cursors[i] < lens[i] && lists[i][cursors[i]].distance < bestd) {
                bestd = lists[i][cursors[i]].distance;
                best = i;
            }
        }
        if (best < 0) break;
        out[merged++] = lists[best][cursors[best]++];
    }
    return merged;
}

typedef struct {
    const float *corpus, *norms, *q;
    float qn;
    int64_t n, dim, chunk, topk;
    int metric;
    float *dots;
    entry *results;
    int64_t *lens;
} slice_ctx;

static void slice_task(void *vctx, int64_t s) {
    slice_ctx *c = (slice_ctx *)vctx;
    int64_t start = s * c->chunk;
    int64_t end = start + c->chunk < c->n ? start + c->chunk : c->n;
    c->lens[s] = 0;
    if (start >= end) return;
    c->lens[s] = scan_slice(c->corpus, c->norms, c->q, c->qn, start, end - start, c->dim,
                            c->topk, c->metric, c->dots + s * c->chunk, c->results + s * c->topk);
}

/* FlatGPUSearch.hostSearch -> hostScan -> ParallelFlatScan.search
 * (FlatGPUSearch.swift:325-380, 523-571; ParallelFlatScan.swift:96-155).
 * k is capped at min(k, 256, n) (FlatGPUSearch.swift:337).  `cores` plays
 * activeProcessorCount; `threads` is how many OS threads run the slices.
 * Returns the number of results written. */
ORC_EXPORT int64_t orc_flat_search(const float *corpus, const float *norms, int64_t n,
                                   int64_t dim, const float *q, int64_t k, int metric,
                                   int64_t cores, int threads, float *out_dist,
                                   uint32_t *out_ids) {
    if (n <= 0 || k <= 0 || metric == METRIC_HAMMING) return 0;
    int64_t topk = k < 256 ? k : 256;
    if (topk > n) topk = n;
    float qn = (metric == METRIC_COSINE || metric == METRIC_L2) ? orc_query_norm(q, dim) : 0.0f;
    int64_t slices = orc_slice_count(n, cores);
    int64_t chunk = (n + slices - 1) / slices;
    float *dots = (float *)malloc(sizeof(float) * (size_t)(slices * chunk));
    entry *res = (entry *)malloc(sizeof(entry) * (size_t)(slices * topk));
    int64_t lens[64];
    slice_ctx c = {corpus, norms, q, qn, n, dim, chunk, topk, metric, dots, res, lens};
    parallel_for(slices, threads, slice_task, &c);
    entry *lists[64];
    for (int64_t s = 0; s < slices; ++s) lists[s] = res + s * topk;
    entry merged[256];
    int64_t m;
    if (slices == 1) {
        m = lens[0] < topk ? lens[0] : topk;
        memcpy(merged, res, sizeof(entry) * (size_t)m);
    } else {
        m = merge_sorted(lists, lens, slices, topk, merged);
    }
    for (int64_t i = 0; i < m; ++i) {
        out_dist[i] = merged[i].distance;
        out_ids[i] = merged[i].id;
    }
    free(dots);
    free(res);
    return m;
}

typedef struct {
    const float *corpus, *norms, *queries;
    int64_t n, dim, k, cores;
    int metric;
    float *out_dist;
    uint32_t *out_ids;
    int64_t *out_counts;
    int64_t stride;
} batch_ctx;

static void batch_task(void *vctx, int64_t i) {
    batch_ctx *c = (batch_ctx *)vctx;
    int64_t m = orc_flat_search(c->corpus, c->norms, c->n, c->dim, c->queries + i * c->dim, c->k,
                                c->metric, c->cores, 1, c->out_dist + i * c->stride,
                                c->out_ids + i * c->stride);
    if (c->out_counts) c->out_counts[i] = m;
}

/* Host batch path without a GPU context: one task per query across cores
 * (FlatGPUSearch.swift:754-779, 1024-1036).  Output stride = min(k, 256). */
ORC_EXPORT void orc_flat_search_batch(const float *corpus, const float *norms, int64_t n,
                                      int64_t dim, const float *queries, int64_t nq, int64_t k,
                                      int metric, int64_t cores, int threads, float *out_dist,
                                      uint32_t *out_ids, int64_t *out_counts) {
    int64_t stride = k < 256 ? k : 256;
    batch_ctx c = {corpus, norms, queries, n, dim, k, cores, metric, out_dist, out_ids,
                   out_counts, stride};
    parallel_for(nq, threads, batch_task, &c);
}

/* ------------------------------------------------------------------------ */
/* Int8 codes (Int8CodeCache.swift:64-99) and the bounded exact scan         */
/* (BoundedExactScan.swift:30-369).                                          */
/* ------------------------------------------------------------------------ */

/* Int8CodeCache.swift:64-99, all in Float. */
ORC_EXPORT void orc_int8_build(const float *corpus, int64_t n, int64_t dim, int8_t *codes,
                               float *u_out, float *w_out, float *normsq_out,
                               float *invsqrt_out) {
    for (int64_t r = 0; r < n; ++r) {
        const float *row = corpus + r * dim;
        float max_abs = 0.0f; /* vDSP_maxmgv: order-free */
        for (int64_t d = 0; d < dim; ++d) {
            float a = fabsf(row[d]);
            if (a > max_abs) max_abs = a;
        }
        float scale = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
        float inverse = 1.0f / scale;
        int32_t abs_sum = 0;
        float normsq = 0.0f;
        for (int64_t d = 0; d < dim; ++d) {
            float v = row[d];
            normsq += v * v;
            float scaled = v * inverse;
            int32_t rounded = (int32_t)(scaled >= 0.0f ? scaled + 0.5f : scaled - 0.5f);
            if (rounded > 127) rounded = 127;
            else if (rounded < -127) rounded = -127;
            codes[r * dim + d] = (int8_t)rounded;
            abs_sum += rounded < 0 ? -rounded : rounded;
        }
        float ebase = ((float)abs_sum / 2.0f + (float)dim / 4.0f) * (1.0f + 1e-6f) + 16.0f;
        u_out[r] = scale;
        w_out[r] = scale * ebase;
        normsq_out[r] = normsq;
        invsqrt_out[r] = normsq > 1e-20f ? 1.0f / sqrtf(normsq) : 0.0f;
    }
}

/* Query quantisation in Double (BoundedExactScan.swift:52-94). */
typedef struct {
    int8_t qcodes[8192];
    float qs_dot, qs_w, qs_qabs_half, cos_f_dot, cos_f_h, cos_f_w;
    double qn_d;
    float qn;
} int8_query;

ORC_EXPORT void orc_int8_quantize_query(const float *q, int64_t dim, float qn, int8_t *qcodes,
                                        float *coef /* [6] */) {
    float max_abs = 0.0f;
    for (int64_t d = 0; d < dim; ++d) {
        float a = fabsf(q[d]);
        if (a > max_abs) max_abs = a;
    }
    double qscale = max_abs > 0.0f ? (double)max_abs / 127.0 : 1.0;
    int64_t abs_sum = 0;
    for (int64_t d = 0; d < dim; ++d) {
        double scaled = (double)q[d] / qscale;
        int32_t rounded = (int32_t)(scaled >= 0 ? scaled + 0.5 : scaled - 0.5);
        if (rounded > 127) rounded = 127;
        else if (rounded < -127) rounded = -127;
        qcodes[d] = (int8_t)rounded;
        abs_sum += rounded < 0 ? -rounded : rounded;
    }
    float qs = (float)qscale;
    float qabs_half = (float)abs_sum / 2.0f;
    float inv = qn > 1e-20f ? 1.0f / sqrtf(qn) : 0.0f;
    coef[0] = qs;             /* qsDot == qsW */
    coef[1] = qs * qabs_half; /* qsQabsHalf */
    coef[2] = qs * inv;       /* cosFDot == cosFW */
    coef[3] = qs * qabs_half * inv; /* cosFH */
    coef[4] = qabs_half;
    coef[5] = qs;
}

/* Lower-bound key of one row (BoundedExactScan.swift:178-228). */
static inline float int8_key(int metric, const float *coef, double qn_d, float dot, float u,
                             float w, float vn, float invsqrt) {
    float qs = coef[0], qsqh = coef[1], cfd = coef[2], cfh = coef[3];
    switch (metric) {
    case METRIC_IP:
        return -(qs * u * dot + qsqh * u + qs * w);
    case METRIC_L2: {
        float two_qs_dot = 2.0f * qs, two_qsqh = 2.0f * qsqh, two_qs_w = 2.0f * qs;
        double key = qn_d + (double)vn - (double)(two_qs_dot * u * dot) -
                     (double)(two_qsqh * u) - (double)(two_qs_w * w);
        return (float)key;
    }
    case METRIC_COSINE: {
        float inner = cfd * u * dot + cfh * u + cfd * w;
        return 1.0f - inner * invsqrt;
    }
    default:
        return INFINITY;
    }
}

ORC_EXPORT float orc_int8_key(int metric, const float *coef, double qn_d, float dot, float u,
                              float w, float vn, float invsqrt) {
    return int8_key(metric, coef, qn_d, dot, u, w, vn, invsqrt);
}

typedef struct {
    float key;
    uint32_t id;
} kentry;

static void kheap_admit(kentry *h, int64_t *count, int64_t cap, float key, uint32_t id) {
    if (*count < cap) {
        int64_t pos = (*count)++;
        h[pos].key = key;
        h[pos].id = id;
        while (pos > 0) {
            int64_t parent = (pos - 1) / 2;
            if (h[pos].key > h[parent].key) {
                kentry t = h[pos];
                h[pos] = h[parent];
                h[parent] = t;
                pos = parent;
            } else {
                break;
            }
        }
    } else if (key < h[0].key) {
        h[0].key = key;
        h[0].id = id;
        int64_t pos = 0, n = *count;
        for (;;) {
            int64_t l = 2 * pos + 1, r = l + 1, largest = pos;
            if (l < n && h[l].key > h[largest].key) largest = l;
            if (r < n && h[r].key > h[largest].key) largest = r;
            if (largest == pos) break;
            kentry t = h[pos];
            h[pos] = h[largest];
            h[largest] = t;
            pos = largest;
        }
    }
}

static void kheap_sorted(kentry *h, int64_t count) {
    while (count > 1) {
        kentry t = h[0];
        h[0] = h[count - 1];
        h[count - 1] = t;
        --count;
        int64_t pos = 0;
        for (;;) {
            int64_t l = 2 * pos + 1, r = l + 1, largest = pos;
            if (l < count && h[l].key > h[largest].key) largest = l;
            if (r < count && h[r].key > h[largest].key) largest = r;
            if (largest == pos) break;
            kentry u = h[pos];
            h[pos] = h[largest];
            h[largest] = u;
            pos = largest;
        }
    }
}

static int cmp_entry_dist_id(const void *a, const void *b) {
    const entry *x = (const entry *)a, *y = (const entry *)b;
    if (x->distance < y->distance) return -1;
    if (x->distance > y->distance) return 1;
    return x->id < y->id ? -1 : (x->id > y->id ? 1 : 0);
}

/* BoundedExactScan.search (BoundedExactScan.swift:30-122).
 * mode 0: adaptive, proof-checked (the reference's semantics).
 * mode 1: one round at a fixed budget, no proof (the literal
 *         "prefilter top-B then rerank" configuration).
 * Returns the number of results, or -1 where the reference returns nil
 * (n < 16384 or missing norms for cosine/L2).  *out_budget receives the
 * final budget.  Rescored ties are ordered by id (the reference's
 * `sort { $0.distance < $1.distance }` leaves them unspecified). */
ORC_EXPORT int64_t orc_int8_search(const float *corpus, const float *norms, const int8_t *codes,
                                   const float *u_plane, const float *w_plane,
                                   const float *normsq_plane, const float *invsqrt_plane,
                                   int64_t n, int64_t dim, const float *q, int64_t k, int metric,
                                   int64_t cores, int mode, int64_t fixed_budget,
                                   int enforce_min_count, float *out_dist, uint32_t *out_ids,
                                   int64_t *out_budget) {
    if ((enforce_min_count && n < 16384) || dim <= 0 || k <= 0 || metric == METRIC_HAMMING)
        return -1;
    if ((metric == METRIC_COSINE || metric == METRIC_L2) && norms == NULL) return -1;
    if (dim > 8192) return -1;
    int64_t topk = k < 256 ? k : 256; /* FlatGPUSearch.swift:433 passes min(k, maxTopK) */
    if (topk > n) topk = n;
    float qn = (metric == METRIC_COSINE || metric == METRIC_L2) ? orc_query_norm(q, dim) : 0.0f;
    int8_t qcodes[8192];
    float coef[6];
    orc_int8_quantize_query(q, dim, qn, qcodes, coef);
    double qn_d = (double)qn;

    int64_t slices = orc_slice_count(n, cores);
    int64_t chunk = (n + slices - 1) / slices;
    float *dots = (float *)malloc(sizeof(float) * (size_t)n);
    orc_i8_dot_rows_f32(codes, qcodes, n, dim, dots); /* cached per slice in the reference */
    float *keys = (float *)malloc(sizeof(float) * (size_t)n);
    for (int64_t r = 0; r < n; ++r)
        keys[r] = int8_key(metric, coef, qn_d, dots[r], u_plane[r], w_plane[r], normsq_plane[r],
                           invsqrt_plane[r]);

    int64_t budget = 256 > topk * 16 ? 256 : topk * 16;
    if (mode == 1) budget = fixed_budget < n ? fixed_budget : n;
    int64_t result = -1;
    kentry *heaps = NULL;
    entry *rescored = NULL;
    uint32_t *ids = NULL;
    float *gd = NULL;
    for (;;) {
        int64_t per_slice = budget < chunk ? budget : chunk;
        heaps = (kentry *)realloc(heaps, sizeof(kentry) * (size_t)(slices * per_slice));
        int64_t lens[64];
        for (int64_t s = 0; s < slices; ++s) {
            int64_t start = s * chunk, end = start + chunk < n ? start + chunk : n;
            lens[s] = 0;
            if (start >= end) continue;
            kentry *h = heaps + s * per_slice;
            for (int64_t r = start; r < end; ++r)
                kheap_admit(h, &lens[s], per_slice, keys[r], (uint32_t)r);
            kheap_sorted(h, lens[s]);
        }
        /* mergeAscending (BoundedExactScan.swift:290-316) */
        ids = (uint32_t *)realloc(ids, sizeof(uint32_t) * (size_t)budget);
        int64_t cursors[64] = {0};
        int64_t nsel = 0;
        double cutoff = INFINITY;
        while (nsel < budget) {
            int64_t best = -1;
            float bk = INFINITY;
            for (int64_t s = 0; s < slices; ++s)
                if (cursors[s] < lens[s] && heaps[s * per_slice + cursors[s]].key < bk) {
                    bk = heaps[s * per_slice + cursors[s]].key;
                    best = s;
                }
            if (best < 0) break;
            ids[nsel++] = heaps[best * per_slice + cursors[best]].id;
            cutoff = (double)bk;
            cursors[best]++;
        }
        /* rescore (BoundedExactScan.swift:320-369) */
        gd = (float *)realloc(gd, sizeof(float) * (size_t)(nsel > 0 ? nsel : 1));
        rescored = (entry *)realloc(rescored, sizeof(entry) * (size_t)(nsel > 0 ? nsel : 1));
        orc_f32_dot_rows_gather(corpus, q, ids, nsel, dim, gd);
        for (int64_t i = 0; i < nsel; ++i) {
            float vn = norms ? norms[ids[i]] : 0.0f;
            rescored[i].distance = host_distance(gd[i], qn, vn, metric);
            rescored[i].id = ids[i];
        }
        qsort(rescored, (size_t)nsel, sizeof(entry), cmp_entry_dist_id);
        if (nsel < topk) {
            result = nsel;
            break;
        }
        float tau = rescored[topk - 1].distance;
        double margin = fabs((double)tau) * 1e-6;
        if (margin < 1e-7) margin = 1e-7;
        int proven = cutoff >= (double)tau + margin || nsel >= n;
        if (proven || mode == 1) {
            result = topk;
            break;
        }
        if (budget >= n) break;
        budget = budget * 4 < n ? budget * 4 : n;
    }
    if (out_budget) *out_budget = budget;
    for (int64_t i = 0; i < result; ++i) {
        out_dist[i] = rescored[i].distance;
        out_ids[i] = rescored[i].id;
    }
    free(dots);
    free(keys);
    free(heaps);
    free(rescored);
    free(ids);
    free(gd);
    return result;
}

/* HostBatchWork.run over a batch without a GPU context
 * (FlatGPUSearch.swift:754-779, 1003-1037): the queries fan out over
 * `threads` workers; each query takes FlatGPUSearch.boundedExactSearch
 * (FlatGPUSearch.swift:387-460: BoundedExactScan.search, mode 0, the
 * adaptive proven-exact scan) when int8 planes are given and n >= 16384,
 * and the fp32 host scan (hostSearch -> ParallelFlatScan with
 * orc_slice_count(n, cores) slices, run by the worker itself) otherwise.
 * Output stride = min(k, 256); route[i] (nullable): 1 int8, 0 fp32. */
typedef struct {
    const float *corpus, *norms, *queries;
    const int8_t *codes;
    const float *u, *w, *ns, *inv;
    int64_t n, dim, k, cores, stride;
    int metric;
    float *out_dist;
    uint32_t *out_ids;
    int64_t *out_counts;
    int32_t *route;
} host_batch_ctx;

static void host_batch_task(void *vctx, int64_t i) {
    host_batch_ctx *c = (host_batch_ctx *)vctx;
    const float *q = c->queries + i * c->dim;
    float *od = c->out_dist + i * c->stride;
    uint32_t *oi = c->out_ids + i * c->stride;
    int64_t m = -1;
    if (c->codes != NULL) {
        int64_t budget = 0;
        m = orc_int8_search(c->corpus, c->norms, c->codes, c->u, c->w, c->ns, c->inv, c->n, c->dim,
                            q, c->k, c->metric, c->cores, 0, 0, 1, od, oi, &budget);
    }
    if (c->route) c->route[i] = m >= 0 ? 1 : 0;
    if (m < 0)
        m = orc_flat_search(c->corpus, c->norms, c->n, c->dim, q, c->k, c->metric, c->cores, 1, od,
                            oi);
    if (c->out_counts) c->out_counts[i] = m;
}

ORC_EXPORT void orc_host_batch_search(const float *corpus, const float *norms, const int8_t *codes,
                                      const float *u_plane, const float *w_plane,
                                      const float *normsq_plane, const float *invsqrt_plane,
                                      int64_t n, int64_t dim, const float *queries, int64_t nq,
                                      int64_t k, int metric, int64_t cores, int threads,
                                      float *out_dist, uint32_t *out_ids, int64_t *out_counts,
                                      int32_t *route) {
    host_batch_ctx c = {corpus, norms, queries, codes, u_plane, w_plane, normsq_plane,
                        invsqrt_plane, n, dim, k, cores, k < 256 ? k : 256, metric, out_dist,
                        out_ids, out_counts, route};
    parallel_for(nq, threads, host_batch_task, &c);
}

/* ------------------------------------------------------------------------ */
/* IVF-flat (IVFFlatSearch.swift)                                            */
/* ------------------------------------------------------------------------ */

/* assignRows argmin (IVFFlatSearch.swift:633-703): ties -> lower cluster.
 * Scores come from cblas_sgemm in the reference (order unpublished); here
 * from the dots.c scalar order. */
ORC_EXPORT void orc_ivf_assign(const float *rows, const float *row_norms, int64_t n, int64_t dim,
                               const float *centroids, const float *cnorms, int64_t nlist,
                               int metric, int32_t *assign) {
    float *dots = (float *)malloc(sizeof(float) * (size_t)nlist);
    for (int64_t r = 0; r < n; ++r) {
        orc_f32_dot_rows(centroids, rows + r * dim, nlist, dim, dots);
        int32_t best = 0;
        float best_key = 3.4028234663852886e38f;
        float qn = row_norms[r];
        for (int64_t c = 0; c < nlist; ++c) {
            float key = host_distance(dots[c], qn, cnorms[c], metric);
            if (key < best_key || (key == best_key && c < best)) {
                best_key = key;
                best = (int32_t)c;
            }
        }
        assign[r] = best;
    }
    free(dots);
}

/* CSR lists in row order (IVFFlatSearch.swift:589-602). */
ORC_EXPORT void orc_ivf_lists(const int32_t *assign, int64_t n, int64_t nlist, int64_t *offsets,
                              uint32_t *list_ids) {
    for (int64_t c = 0; c <= nlist; ++c) offsets[c] = 0;
    for (int64_t r = 0; r < n; ++r) offsets[assign[r] + 1]++;
    for (int64_t c = 0; c < nlist; ++c) offsets[c + 1] += offsets[c];
    int64_t *cursor = (int64_t *)malloc(sizeof(int64_t) * (size_t)nlist);
    for (int64_t c = 0; c < nlist; ++c) cursor[c] = offsets[c];
    for (int64_t r = 0; r < n; ++r) list_ids[cursor[assign[r]]++] = (uint32_t)r;
    free(cursor);
}

typedef struct {
    float key;
    int64_t idx;
} kidx;

static int cmp_kidx(const void *a, const void *b) {
    const kidx *x = (const kidx *)a, *y = (const kidx *)b;
    if (x->key < y->key) return -1;
    if (x->key > y->key) return 1;
    return x->idx < y->idx ? -1 : (x->idx > y->idx ? 1 : 0);
}

static int cmp_i32(const void *a, const void *b) {
    int32_t x = *(const int32_t *)a, y = *(const int32_t *)b;
    return x < y ? -1 : (x > y ? 1 : 0);
}

/* Probe selection (IVFFlatSearch.swift:224-251): centroid keys, the nprobe
 * smallest by (key, index) (smallestIndices, :314-382), then sorted by
 * cluster id.  qn: vDSP_dotpr in the reference, sequential here. */
ORC_EXPORT int64_t orc_ivf_probe(const float *centroids, const float *cnorms, int64_t nlist,
                                 int64_t dim, const float *q, int64_t nprobe, int metric,
                                 int32_t *probes) {
    float qn = (metric == METRIC_COSINE || metric == METRIC_L2) ? orc_query_norm(q, dim) : 0.0f;
    float *dots = (float *)malloc(sizeof(float) * (size_t)nlist);
    kidx *keys = (kidx *)malloc(sizeof(kidx) * (size_t)nlist);
    orc_f32_dot_rows(centroids, q, nlist, dim, dots);
    for (int64_t c = 0; c < nlist; ++c) {
        keys[c].key = host_distance(dots[c], qn, cnorms[c], metric);
        keys[c].idx = c;
    }
    qsort(keys, (size_t)nlist, sizeof(kidx), cmp_kidx);
    int64_t p = nprobe < nlist ? nprobe : nlist;
    if (p < 1) p = 1;
    for (int64_t i = 0; i < p; ++i) probes[i] = (int32_t)keys[i].idx;
    qsort(probes, (size_t)p, sizeof(int32_t), cmp_i32);
    free(dots);
    free(keys);
    return p;
}

/* scanProbedLists (IVFFlatSearch.swift:214-291): per probed list (in
 * cluster-id order) exact dots over the packed segment, TopKHeap on
 * (distance, id) with original row ids, ascending output. */
ORC_EXPORT int64_t orc_ivf_search(const float *packed, const float *packed_norms,
                                  const int64_t *offsets, const uint32_t *list_ids,
                                  const float *centroids, const float *cnorms, int64_t nlist,
                                  int64_t count, int64_t dim, const float *q, int64_t k,
                                  int64_t nprobe, int metric, float *out_dist, uint32_t *out_ids,
                                  int32_t *out_probes) {
    if (k <= 0 || count <= 0) return 0;
    int64_t kk = k < count ? k : count;
    int64_t np = nprobe < nlist ? nprobe : nlist;
    if (np < 1) np = 1;
    int32_t *probes = (int32_t *)malloc(sizeof(int32_t) * (size_t)np);
    np = orc_ivf_probe(centroids, cnorms, nlist, dim, q, np, metric, probes);
    if (out_probes) memcpy(out_probes, probes, sizeof(int32_t) * (size_t)np);
    float qn = (metric == METRIC_COSINE || metric == METRIC_L2) ? orc_query_norm(q, dim) : 0.0f;
    int64_t cand = 0;
    for (int64_t i = 0; i < np; ++i) cand += offsets[probes[i] + 1] - offsets[probes[i]];
    if (cand == 0) {
        free(probes);
        return 0;
    }
    int64_t topk = kk < cand ? kk : cand;
    entry *all = (entry *)malloc(sizeof(entry) * (size_t)cand);
    float *dots = (float *)malloc(sizeof(float) * (size_t)cand);
    int64_t cur = 0;
    for (int64_t i = 0; i < np; ++i) {
        int64_t start = offsets[probes[i]], rows = offsets[probes[i] + 1] - start;
        if (rows <= 0) continue;
        orc_f32_dot_rows(packed + start * dim, q, rows, dim, dots + cur);
        for (int64_t l = 0; l < rows; ++l) {
            all[cur + l].distance = host_distance(dots[cur + l], qn, packed_norms[start + l], metric);
            all[cur + l].id = list_ids[start + l];
        }
        cur += rows;
    }
    /* A (distance, id) bounded heap keeps exactly the topk smallest pairs;
     * sorting all candidates by the same order gives the same list. */
    qsort(all, (size_t)cand, sizeof(entry), cmp_entry_dist_id);
    for (int64_t i = 0; i < topk; ++i) {
        out_dist[i] = all[i].distance;
        out_ids[i] = all[i].id;
    }
    free(all);
    free(dots);
    free(probes);
    return topk;
}

ORC_EXPORT float orc_simd_distance(const float *a, const float *b, int64_t dim, int metric);

/* KMeans.cluster (KMeans.swift:53-257) over `n` rows of `dim` floats read at
 * row stride `ld` (a subspace of wider rows when ld > dim, as
 * clusterSubspace does).  Lloyd loop (KMeans.swift:98-250), single-worker
 * order:
 *   - assignment: argmin over centroids of SIMDDistance.distance
 *     (orc_simd_distance), strict < so the first centroid wins ties
 *     (KMeans.swift:196-215);
 *   - stop before the update when no assignment changed (the previous
 *     assignments start at -1, so the first pass always changes);
 *   - update: per centroid the Float sum of its rows in row order times
 *     scale = 1 / Float(count) (KMeans.swift:224-250); empty clusters keep
 *     their centroid (KMeans.swift:242-246).
 * The reference seeds with k-means++ drawn from Swift's stdlib RNG
 * (KMeans.swift:259-328), which is not reproduced: the initial centroids
 * here are rows 0, s, 2s, ... with s = max(1, n / k).  assign_out
 * (nullable) receives Result.assignments: those of the last assignment
 * pass (-1 everywhere when iters == 0).  The multi-worker path of the
 * reference (KMeans.swift:108-188) adds per-worker partial sums whose split
 * depends on the core count; this is its single-worker order. */
ORC_EXPORT void orc_kmeans_ld(const float *rows, int64_t n, int64_t dim, int64_t ld, int64_t k,
                              int64_t iters, int metric, float *centroids, int32_t *assign_out) {
    int64_t stride = n / k > 1 ? n / k : 1;
    for (int64_t c = 0; c < k; ++c)
        memcpy(centroids + c * dim, rows + ((c * stride) % n) * ld, sizeof(float) * (size_t)dim);
    int32_t *assign = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
    float *sums = (float *)malloc(sizeof(float) * (size_t)(k * dim));
    int64_t *counts = (int64_t *)malloc(sizeof(int64_t) * (size_t)k);
    for (int64_t r = 0; r < n; ++r) assign[r] = -1;
    for (int64_t it = 0; it < iters; ++it) {
        int changed = 0;
        memset(sums, 0, sizeof(float) * (size_t)(k * dim));
        memset(counts, 0, sizeof(int64_t) * (size_t)k);
        for (int64_t r = 0; r < n; ++r) {
            const float *x = rows + r * ld;
            int32_t best = 0;
            float bestd = 3.4028234663852886e38f;
            for (int64_t c = 0; c < k; ++c) {
                float d = orc_simd_distance(x, centroids + c * dim, dim, metric);
                if (d < bestd) {
                    bestd = d;
                    best = (int32_t)c;
                }
            }
            if (assign[r] != best) {
                assign[r] = best;
                changed = 1;
            }
            counts[best]++;
            for (int64_t d = 0; d < dim; ++d) sums[best * dim + d] += x[d];
        }
        if (!changed) break;
        for (int64_t c = 0; c < k; ++c) {
            if (counts[c] == 0) continue;
            float scale = 1.0f / (float)counts[c];
            for (int64_t d = 0; d < dim; ++d) centroids[c * dim + d] = sums[c * dim + d] * scale;
        }
    }
    if (assign_out) memcpy(assign_out, assign, sizeof(int32_t) * (size_t)n);
    free(assign);
    free(sums);
    free(counts);
}

ORC_EXPORT void orc_kmeans(const float *rows, int64_t n, int64_t dim, int64_t k, int64_t iters,
                           int metric, float *centroids, int32_t *assign_out) {
    orc_kmeans_ld(rows, n, dim, dim, k, iters, metric, centroids, assign_out);
}

/* IVFFlatSearch.buildPartition's training (IVFFlatSearch.swift:517-551):
 * L = min(max(1, nlist), n) lists; a sample of
 * min(n, max(L, min(4096, max(16 L, L)))) rows taken at stride
 * max(1, n / sampleCount) from row 0, topped up with rows
 * sample.count % n; KMeans.cluster(k = L, maxIterations 8, metric).
 * Writes L x dim centroids, returns L. */
ORC_EXPORT int64_t orc_ivf_flat_train(const float *rows, int64_t n, int64_t dim, int64_t nlist,
                                      int metric, float *centroids) {
    int64_t lists = nlist < 1 ? 1 : nlist;
    if (lists > n) lists = n;
    int64_t sixteen = lists * 16 > lists ? lists * 16 : lists;
    int64_t cap = 4096 < sixteen ? 4096 : sixteen;
    int64_t want = lists > cap ? lists : cap;
    int64_t count = n < want ? n : want;
    int64_t stride = n / count > 1 ? n / count : 1;
    float *sample = (float *)malloc(sizeof(float) * (size_t)(count * dim));
    int64_t have = 0;
    for (int64_t cursor = 0; have < count && cursor < n; cursor += stride)
        memcpy(sample + (have++) * dim, rows + cursor * dim, sizeof(float) * (size_t)dim);
    while (have < count) {
        memcpy(sample + have * dim, rows + (have % n) * dim, sizeof(float) * (size_t)dim);
        ++have;
    }
    orc_kmeans(sample, count, dim, lists, 8, metric, centroids, NULL);
    free(sample);
    return lists;
}

/* ------------------------------------------------------------------------ */
/* IVF-PQ (IVFPQIndex.swift, ProductQuantizer.swift, BoundedSelection.swift) */
/* ------------------------------------------------------------------------ */

/* SIMDDistance.distance (SIMDDistance.swift:17-80); vDSP orders restated as
 * sequential sums. */
ORC_EXPORT float orc_simd_distance(const float *a, const float *b, int64_t dim, int metric) {
    switch (metric) {
    case METRIC_COSINE: {
        if (dim <= 0) return 1.0f;
        float dot = 0.0f, na = 0.0f, nb = 0.0f;
        for (int64_t d = 0; d < dim; ++d) dot += a[d] * b[d];
        for (int64_t d = 0; d < dim; ++d) na += a[d] * a[d];
        for (int64_t d = 0; d < dim; ++d) nb += b[d] * b[d];
        float denom = sqrtf(na) * sqrtf(nb);
        return denom < 1e-10f ? 1.0f : 1.0f - dot / denom;
    }
    case METRIC_L2: {
        if (dim <= 0) return 0.0f;
        float s = 0.0f;
        for (int64_t d = 0; d < dim; ++d) {
            float t = a[d] - b[d];
            s += t * t;
        }
        return s;
    }
    case METRIC_IP: {
        if (dim <= 0) return 0.0f;
        float dot = 0.0f;
        for (int64_t d = 0; d < dim; ++d) dot += a[d] * b[d];
        return -dot;
    }
    default: {
        float cnt = 0.0f;
        for (int64_t d = 0; d < dim; ++d) cnt += a[d] != b[d] ? 1.0f : 0.0f;
        return cnt;
    }
    }
}

/* nearestCoarseCentroid (IVFPQIndex.swift:514-550): strict <, first wins. */
ORC_EXPORT int32_t orc_nearest_coarse(const float *x, const float *centroids, int64_t nlist,
                                      int64_t dim, int metric) {
    int32_t best = 0;
    float bestd = 3.4028234663852886e38f;
    for (int64_t c = 0; c < nlist; ++c) {
        float d = orc_simd_distance(x, centroids + c * dim, dim, metric);
        if (d < bestd) {
            bestd = d;
            best = (int32_t)c;
        }
    }
    return best;
}

/* ProductQuantizer.encode(vector:subtracting:) (ProductQuantizer.swift:120-169).
 * codebooks: [M][256][dsub]. */
ORC_EXPORT void orc_pq_encode(const float *x, const float *centroid, const float *codebooks,
                              int64_t m, int64_t dsub, uint8_t *codes) {
    for (int64_t s = 0; s < m; ++s) {
        const float *xb = x + s * dsub, *cb = centroid + s * dsub;
        int best = 0;
        float bestd = 3.4028234663852886e38f;
        for (int c = 0; c < 256; ++c) {
            const float *book = codebooks + (s * 256 + c) * dsub;
            float sum = 0.0f;
            for (int64_t d = 0; d < dsub; ++d) {
                float delta = xb[d] - cb[d] - book[d];
                sum += delta * delta;
            }
            if (sum < bestd) {
                bestd = sum;
                best = c;
            }
        }
        codes[s] = (uint8_t)best;
    }
}

/* _IVFPQIndex.add coarse assignment + encode for a batch of rows
 * (IVFPQIndex.swift:140-159). */
ORC_EXPORT void orc_ivfpq_encode_rows(const float *rows, int64_t n, int64_t dim,
                                      const float *coarse, int64_t nlist, const float *codebooks,
                                      int64_t m, int metric, int32_t *assign, uint8_t *codes) {
    int64_t dsub = dim / m;
    for (int64_t r = 0; r < n; ++r) {
        int32_t c = orc_nearest_coarse(rows + r * dim, coarse, nlist, dim, metric);
        assign[r] = c;
        orc_pq_encode(rows + r * dim, coarse + (int64_t)c * dim, codebooks, m, dsub,
                      codes + r * m);
    }
}

/* _IVFPQIndex.train (IVFPQIndex.swift:54-104): coarse KMeans.cluster
 * (nlist, iters, metric) on the rows; residual = row - centroid of its
 * Result.assignments entry, elementwise in Float (IVFPQIndex.swift:366-368);
 * then ProductQuantizer.train (ProductQuantizer.swift:10-85): for every
 * subspace s, KMeans.clusterSubspace over the residuals' dims
 * [s dsub, (s + 1) dsub) with k = 256, L2 and maxIterations iters.
 * Needs n >= 256, n >= nlist, dim % m == 0 (checked by the caller). */
ORC_EXPORT void orc_ivfpq_train(const float *rows, int64_t n, int64_t dim, int64_t nlist,
                                int64_t m, int64_t iters, int metric, float *coarse,
                                float *codebooks) {
    int64_t dsub = dim / m;
    int32_t *assign = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
    orc_kmeans(rows, n, dim, nlist, iters, metric, coarse, assign);
    float *res = (float *)malloc(sizeof(float) * (size_t)(n * dim));
    for (int64_t r = 0; r < n; ++r) {
        const float *c = coarse + (int64_t)assign[r] * dim;
        for (int64_t d = 0; d < dim; ++d) res[r * dim + d] = rows[r * dim + d] - c[d];
    }
    for (int64_t s = 0; s < m; ++s)
        orc_kmeans_ld(res + s * dsub, n, dsub, dim, 256, iters, METRIC_L2,
                      codebooks + s * 256 * dsub, NULL);
    free(res);
    free(assign);
}

/* distanceTableFlattened (ProductQuantizer.swift:223-253). */
ORC_EXPORT void orc_pq_lut(const float *qres, const float *codebooks, int64_t m, int64_t dsub,
                           int metric, float *lut) {
    for (int64_t s = 0; s < m; ++s)
        for (int c = 0; c < 256; ++c)
            lut[s * 256 + c] =
                orc_simd_distance(qres + s * dsub, codebooks + (s * 256 + c) * dsub, dsub, metric);
}

/* BoundedSortedList (BoundedSelection.swift:158-214): capacity-limited list,
 * best first; insertion at the lower bound puts a newcomer ahead of equal
 * scores; when full, a newcomer must strictly beat the worst. */
typedef struct {
    float score;
    uint32_t id;
} sl_entry;

static void sorted_list_insert(sl_entry *list, int64_t *count, int64_t cap, float score,
                               uint32_t id) {
    if (cap <= 0) return;
    if (*count >= cap && !(score < list[*count - 1].score)) return;
    int64_t lo = 0, hi = *count;
    while (lo < hi) {
        int64_t mid = (lo + hi) / 2;
        if (list[mid].score < score) lo = mid + 1;
        else hi = mid;
    }
    int64_t n = *count < cap ? *count : cap - 1;
    for (int64_t i = n; i > lo; --i) list[i] = list[i - 1];
    list[lo].score = score;
    list[lo].id = id;
    if (*count < cap) (*count)++;
}

ORC_EXPORT int64_t orc_sorted_list_run(const float *scores, const uint32_t *ids, int64_t n,
                                       int64_t cap, float *out_scores, uint32_t *out_ids) {
    sl_entry *list = (sl_entry *)malloc(sizeof(sl_entry) * (size_t)(cap > 0 ? cap : 1));
    int64_t count = 0;
    for (int64_t i = 0; i < n; ++i) sorted_list_insert(list, &count, cap, scores[i], ids[i]);
    for (int64_t i = 0; i < count; ++i) {
        out_scores[i] = list[i].score;
        out_ids[i] = list[i].id;
    }
    free(list);
    return count;
}

/* selectClosestCentroids (IVFPQIndex.swift:484-512): later index first on
 * equal distance.  Writes the probe order (closest first). */
ORC_EXPORT int64_t orc_ivfpq_probe(const float *coarse, int64_t nlist, int64_t dim,
                                   const float *q, int64_t nprobe, int metric, int32_t *probes,
                                   float *probe_dist) {
    int64_t cap = nprobe < nlist ? nprobe : nlist;
    sl_entry *list = (sl_entry *)malloc(sizeof(sl_entry) * (size_t)(cap > 0 ? cap : 1));
    int64_t count = 0;
    for (int64_t c = 0; c < nlist; ++c)
        sorted_list_insert(list, &count, cap,
                           orc_simd_distance(q, coarse + c * dim, dim, metric), (uint32_t)c);
    for (int64_t i = 0; i < count; ++i) {
        probes[i] = (int32_t)list[i].id;
        if (probe_dist) probe_dist[i] = list[i].score;
    }
    free(list);
    return count;
}

/* _IVFPQIndex.search (IVFPQIndex.swift:177-226) with the CPU ADC path
 * (:418-452): per probe, residual, LUT, sequential sum over subspaces, merge
 * into BoundedSortedList(k).  Lists are CSR (offsets, ids) over internal
 * ids; codes are indexed by internal id ([id][M]).
 * If rows != NULL and rerank_k > 0, the k ADC results are re-ranked by the
 * exact host distance on the raw rows (sequential dot order) and the best
 * rerank_k are kept, ordered by (distance, id) -- this step has no
 * counterpart in the reference, which stops at ADC. */
ORC_EXPORT int64_t orc_ivfpq_search(const float *coarse, int64_t nlist, int64_t dim,
                                    const float *codebooks, int64_t m, const uint8_t *codes,
                                    const int64_t *offsets, const uint32_t *list_ids, int metric,
                                    const float *q, int64_t k, int64_t nprobe, const float *rows,
                                    int64_t rerank_k, float *out_score, uint32_t *out_ids) {
    if (k <= 0 || nlist <= 0) return 0;
    int64_t dsub = dim / m;
    int64_t np = nprobe < nlist ? nprobe : nlist;
    if (np < 1) np = 1;
    int32_t *probes = (int32_t *)malloc(sizeof(int32_t) * (size_t)np);
    np = orc_ivfpq_probe(coarse, nlist, dim, q, np, metric, probes, NULL);
    float *qres = (float *)malloc(sizeof(float) * (size_t)dim);
    float *lut = (float *)malloc(sizeof(float) * (size_t)(m * 256));
    sl_entry *list = (sl_entry *)malloc(sizeof(sl_entry) * (size_t)k);
    int64_t count = 0;
    for (int64_t p = 0; p < np; ++p) {
        const float *c = coarse + (int64_t)probes[p] * dim;
        for (int64_t d = 0; d < dim; ++d) qres[d] = q[d] - c[d];
        orc_pq_lut(qres, codebooks, m, dsub, metric, lut);
        for (int64_t i = offsets[probes[p]]; i < offsets[probes[p] + 1]; ++i) {
            uint32_t id = list_ids[i];
            const uint8_t *code = codes + (int64_t)id * m;
            float total = 0.0f;
            for (int64_t s = 0; s < m; ++s) total += lut[s * 256 + code[s]];
            sorted_list_insert(list, &count, k, total, id);
        }
    }
    int64_t out_n = count;
    if (rows != NULL && rerank_k > 0) {
        float qn = (metric == METRIC_COSINE || metric == METRIC_L2) ? orc_query_norm(q, dim) : 0.0f;
        entry *ex = (entry *)malloc(sizeof(entry) * (size_t)(count > 0 ? count : 1));
        for (int64_t i = 0; i < count; ++i) {
            const float *row = rows + (int64_t)list[i].id * dim;
            float dot = 0.0f, vn = 0.0f;
            for (int64_t d = 0; d < dim; ++d) dot += row[d] * q[d];
            for (int64_t d = 0; d < dim; ++d) vn += row[d] * row[d];
            ex[i].distance = host_distance(dot, qn, vn, metric);
            ex[i].id = list[i].id;
        }
        qsort(ex, (size_t)count, sizeof(entry), cmp_entry_dist_id);
        out_n = rerank_k < count ? rerank_k : count;
        for (int64_t i = 0; i < out_n; ++i) {
            out_score[i] = ex[i].distance;
            out_ids[i] = ex[i].id;
        }
        free(ex);
    } else {
        for (int64_t i = 0; i < count; ++i) {
            out_score[i] = list[i].score;
            out_ids[i] = list[i].id;
        }
    }
    free(probes);
    free(qres);
    free(lut);
    free(list);
    return out_n;
}

/* Host-formula distances of given row ids (dots.c scalar order): used by the
 * parity checks to confirm each returned id carries its exact distance. */
ORC_EXPORT void orc_distances_for_ids(const float *corpus, const float *norms, int64_t dim,
                                      const float *q, const uint32_t *ids, int64_t count,
                                      int metric, float *out) {
    float qn = (metric == METRIC_COSINE || metric == METRIC_L2) ? orc_query_norm(q, dim) : 0.0f;
    for (int64_t i = 0; i < count; ++i) {
        if (ids[i] == 0xFFFFFFFFu) {
            out[i] = 3.4028234663852886e38f;
            continue;
        }
        float dot;
        orc_f32_dot_rows_gather(corpus, q, &ids[i], 1, dim, &dot);
        float vn = norms ? norms[ids[i]] : 0.0f;
        out[i] = host_distance(dot, qn, vn, metric);
    }
}
