// IVF-PQ on gfx950: coarse assignment and encode (IVFPQIndex.swift:106-175,
// ProductQuantizer.swift:120-169), probe selection (IVFPQIndex.swift:484-550)
// and the ADC probe scan with BoundedSortedList merging
// (IVFPQIndex.swift:177-226, 418-452; BoundedSelection.swift:158-218).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <functional>
#include <vector>

#include "mans_hip.h"
#include "mans_ivf.hpp"
#include "mans_runtime.hpp"
#include "mans_scan.hpp"

namespace mans {

// ---------------------------------------------------------------------------
// IVF-PQ: _IVFPQIndex.add / search (IVFPQIndex.swift:106-226) with the CPU
// ADC path (:418-452) and ProductQuantizer (ProductQuantizer.swift:120-169,
// 223-253), bit-exact.
//
//  - Distances are SIMDDistance.distance restated as sequential sums
//    (SIMDDistance.swift:17-80); every (row, centroid) and (query,
//    centroid) pair is computed in full in that order -- the coarse
//    assignment is a brute-force argmin (strict <, first wins) with the
//    centroid values read through the scalar cache, and the probe order is
//    BoundedSortedList's (distance ascending, later index first on ties).
//  - Codes: per subspace the argmin over the 256 codewords of the
//    sequential squared distance of the residual, lowest code on ties.
//    They are stored packed list by list, so a probed list is contiguous.
//  - ADC: per (query, probe) the residual LUT (M x 256) is built in LDS; a
//    row's score is the sequential sum of its M LUT entries.  The k_adc
//    best of BoundedSortedList(k_adc) over the probes in order are the
//    candidates whose score is at most the k_adc-th smallest score T,
//    re-inserted in arrival order: with at most k_adc of them nothing is
//    evicted, so they come out sorted by score, later arrivals first among
//    equals; with more (ties at T) the list is replayed one insertion at a
//    time, and past the kept candidates (more ties than k_adc + 64)
//    ivfpq_tie_replay rescans the query's rows in arrival order.  Work
//    items of equal row counts cover each query's probed lists; the last
//    item of a query merges, orders, maps positions to ids and (with
//    rerank_k > 0) rescores exactly.
// ---------------------------------------------------------------------------


// Coarse assignment, one thread per row: argmin over every centroid of the
// sequential distance (IVFPQIndex.swift:514-550).  The centroid index is
// uniform across the wave, so its values come through scalar loads.
template <int DIM>
__global__ __launch_bounds__(256) void pq_assign(const float* __restrict__ rows, int64_t n,
                                                 const float* __restrict__ coarse, int nlist,
                                                 int metric, int32_t* __restrict__ assign) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool valid = r < n;
    float x[DIM];
    const float* xr = rows + (valid ? r : 0) * DIM;
#pragma unroll
    for (int d = 0; d < DIM; ++d) x[d] = xr[d];
    float xn = 0.0f;
    if (metric == kMetricCosine) {
#pragma unroll
        for (int d = 0; d < DIM; ++d) xn += x[d] * x[d];
    }
    int best = 0;
    float bestd = kFltMax;
    for (int c = 0; c < nlist; ++c) {
        const float* cr = coarse + (int64_t)c * DIM;
        float dist;
        if (metric == kMetricL2) {
            float s = 0.0f;
#pragma unroll
            for (int d = 0; d < DIM; ++d) {
                const float t = x[d] - cr[d];
                s += t * t;
            }
            dist = s;
        } else if (metric == kMetricIP) {
            float dot = 0.0f;
#pragma unroll
            for (int d = 0; d < DIM; ++d) dot += x[d] * cr[d];
            dist = -dot;
        } else {
            float dot = 0.0f, nb = 0.0f;
#pragma unroll
            for (int d = 0; d < DIM; ++d) dot += x[d] * cr[d];
#pragma unroll
            for (int d = 0; d < DIM; ++d) nb += cr[d] * cr[d];
            const float denom = sqrtf(xn) * sqrtf(nb);
            dist = denom < 1e-10f ? 1.0f : 1.0f - dot / denom;
        }
        if (dist < bestd) {
            bestd = dist;
            best = c;
        }
    }
    if (valid) assign[r] = best;
}

// Generic-dimension variant (the row is re-read from memory per centroid).
__global__ __launch_bounds__(256) void pq_assign_any(const float* __restrict__ rows, int64_t n,
                                                     int dim, const float* __restrict__ coarse,
                                                     int nlist, int metric,
                                                     int32_t* __restrict__ assign) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n) return;
    const float* xr = rows + r * dim;
    int best = 0;
    float bestd = kFltMax;
    for (int c = 0; c < nlist; ++c) {
        const float dist = simd_distance(xr, coarse + (int64_t)c * dim, dim, metric);
        if (dist < bestd) {
            bestd = dist;
            best = c;
        }
    }
    assign[r] = best;
}

// ProductQuantizer.encode(vector:subtracting:) for the row at each packed
// position (ProductQuantizer.swift:120-169): codes_packed[pos][m].
__global__ __launch_bounds__(256) void pq_encode(const float* __restrict__ rows, int dim,
                                                 const uint32_t* __restrict__ list_ids,
                                                 const int32_t* __restrict__ assign, int64_t n,
                                                 const float* __restrict__ coarse,
                                                 const float* __restrict__ books, int m, int dsub,
                                                 uint8_t* __restrict__ codes) {
    const int64_t pos = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (pos >= n) return;
    const int64_t row = list_ids[pos];
    const float* x = rows + row * dim;
    const float* cen = coarse + (int64_t)assign[row] * dim;
    for (int s = 0; s < m; ++s) {
        const float* xb = x + s * dsub;
        const float* cb = cen + s * dsub;
        int best = 0;
        float bestd = kFltMax;
        for (int c = 0; c < 256; ++c) {
            const float* book = books + ((int64_t)s * 256 + c) * dsub;
            float sum = 0.0f;
            for (int d = 0; d < dsub; ++d) {
                const float delta = xb[d] - cb[d] - book[d];
                sum += delta * delta;
            }
            if (sum < bestd) {
                bestd = sum;
                best = c;
            }
        }
        codes[pos * m + s] = (uint8_t)best;
    }
}

// One insertion into a BoundedSortedList(cap) held as (ls, lt) with `count`
// entries (BoundedSelection.swift:178-213): a newcomer goes in front of equal
// scores; a full list takes it only if it beats the worst.  Returns the new
// count.
__device__ inline int sorted_list_insert(float sc, uint32_t tag, int count, int cap, float* ls,
                                         uint32_t* lt) {
    if (count >= cap && !(sc < ls[count - 1])) return count;
    int lo = 0, hi = count;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (ls[mid] < sc) lo = mid + 1;
        else hi = mid;
    }
    const int last = count < cap ? count : cap - 1;
    for (int j = last; j > lo; --j) {
        ls[j] = ls[j - 1];
        lt[j] = lt[j - 1];
    }
    ls[lo] = sc;
    lt[lo] = tag;
    return count < cap ? count + 1 : count;
}

// The list replayed by one thread over `cnt` (score, tag) entries in arrival
// order, from empty.
__device__ inline int sorted_list_replay(const float* in_score, const uint32_t* in_tag, int cnt,
                                         int cap, float* ls, uint32_t* lt) {
    int count = 0;
    for (int i = 0; i < cnt; ++i) count = sorted_list_insert(in_score[i], in_tag[i], count, cap, ls, lt);
    return count;
}

// `m` more entries whose tags are tag0, tag0 + 1, ... inserted in order into
// a list that holds `count`.
__device__ inline int sorted_list_insert_run(const float* in_score, uint32_t tag0, int m, int cap,
                                             int count, float* ls, uint32_t* lt) {
    for (int i = 0; i < m; ++i) count = sorted_list_insert(in_score[i], tag0 + (uint32_t)i, count, cap, ls, lt);
    return count;
}

// dst[d][c] = src[c][d] for a rows x cols matrix.
__global__ void transpose_kernel(const float* __restrict__ src, int64_t rows, int cols,
                                 float* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * cols) return;
    const int64_t r = i / cols;
    const int c = (int)(i - r * cols);
    dst[(int64_t)c * rows + r] = src[i];
}

// Distances from kPqDistQ queries to every centroid (SIMDDistance.distance,
// SIMDDistance.swift:17-80, as sequential sums: each (query, centroid) pair
// in the same operations and order as simd_distance).  grid
// (ceil(nlist / 256), ceil(nq / kPqDistQ)), block 256: thread c takes
// centroid c for the block's queries, so each centroid value read from
// coarse_t ([dim][nlist]) serves all of them.  dist: [nq][nlist].
constexpr int kPqDistQ = 16;

template <int METRIC>
__global__ __launch_bounds__(256) void pq_coarse_dist(const float* __restrict__ queries, int64_t nq,
                                                      int dim, const float* __restrict__ coarse_t,
                                                      int nlist, float* __restrict__ dist) {
    extern __shared__ float qs[];  // [kPqDistQ][dim], then the queries' sums of squares
    float* qsq = qs + kPqDistQ * dim;
    const int tid = threadIdx.x;
    const int64_t q0 = (int64_t)blockIdx.y * kPqDistQ;
    for (int i = tid; i < kPqDistQ * dim; i += blockDim.x) {
        const int j = i / dim;
        qs[i] = q0 + j < nq ? queries[(q0 + j) * dim + (i - j * dim)] : 0.0f;
    }
    __syncthreads();
    if (METRIC == kMetricCosine && tid < kPqDistQ) {
        float na = 0.0f;
        for (int i = 0; i < dim; ++i) na += qs[tid * dim + i] * qs[tid * dim + i];
        qsq[tid] = na;
    }
    __syncthreads();
    const int c = blockIdx.x * blockDim.x + tid;
    if (c >= nlist) return;
    float acc[kPqDistQ];
#pragma unroll
    for (int j = 0; j < kPqDistQ; ++j) acc[j] = 0.0f;
    float nb = 0.0f;
    for (int i = 0; i < dim; ++i) {
        const float b = coarse_t[(int64_t)i * nlist + c];
#pragma unroll
        for (int j = 0; j < kPqDistQ; ++j) {
            const float a = qs[j * dim + i];
            if (METRIC == kMetricL2) {
                const float t = a - b;
                acc[j] += t * t;
            } else {
                acc[j] += a * b;
            }
        }
        if (METRIC == kMetricCosine) nb += b * b;
    }
#pragma unroll
    for (int j = 0; j < kPqDistQ; ++j) {
        if (q0 + j >= nq) break;
        float d;
        if (METRIC == kMetricL2) {
            d = acc[j];
        } else if (METRIC == kMetricIP) {
            d = -acc[j];
        } else if (dim <= 0) {
            d = 1.0f;
        } else {
            const float denom = sqrtf(qsq[j]) * sqrtf(nb);
            d = denom < 1e-10f ? 1.0f : 1.0f - acc[j] / denom;
        }
        dist[(q0 + j) * nlist + c] = d;
    }
}

// Probe selection, one block per query (selectClosestCentroids,
// IVFPQIndex.swift:484-512): from the query's distances to every centroid
// (pq_coarse_dist), the np + 64 smallest by (distance, index), then the
// BoundedSortedList(np) order over those at or below the np-th distance.
// When more centroids tie at the np-th distance than those kept (a zero
// query, duplicate centroids), the list is replayed over every centroid in
// index order instead.  dynamic LDS: 4 * cap slots; cap >= 2 np + 128.
// CAP: the lists' capacity when fixed at compile time (the sorts compiled
// for it; 256 for np <= 64), else 0.
template <int CAP>
__global__ __launch_bounds__(256) void pq_probes(const float* __restrict__ dists, int nlist,
                                                 int np, int kc, int cap,
                                                 uint32_t* __restrict__ probes) {
    extern __shared__ uint64_t lds[];
    __shared__ int s_cnt, s_over, s_len;
    const int tid = threadIdx.x, wave = tid >> 6;
    const int64_t q = blockIdx.x;
    const float* qd = dists + q * nlist;
    WaveTopKT<CAP> sel;
    sel.init(lds + wave * cap, cap, kc);
    for (int base = 0; base < nlist; base += blockDim.x) {
        const int c = base + tid;
        const bool v = c < nlist;
        sel.offer(v, v ? qd[c] : 0.0f, (uint32_t)c);
    }
    sel.finish();
    __syncthreads();
    if (wave == 0) {
        for (int w = 1; w < 4; ++w) sel.offer_slots(lds + w * cap, kc);
        sel.finish();
    }
    __syncthreads();
    // lds[0, kc): the kc smallest (distance, index); S = those <= T.
    uint64_t* top = lds;
    if (tid == 0) {
        int ncand = 0;
        while (ncand < kc && top[ncand] != kEmptySlot) ++ncand;
        const int take = np < ncand ? np : ncand;
        const float t = slot_key(top[take - 1]);
        int s = take;
        while (s < ncand && slot_key(top[s]) <= t) ++s;
        s_cnt = s;
        s_over = (s == kc && kc < nlist) ? 1 : 0;
    }
    __syncthreads();
    if (s_over) {
        // Every centroid, 256 at a time in index order: distances into LDS,
        // then one thread inserts them into the list.
        float* chunk = reinterpret_cast<float*>(lds + 2 * cap);
        float* ls = reinterpret_cast<float*>(lds + 3 * cap);
        uint32_t* lt = reinterpret_cast<uint32_t*>(ls + np);
        if (tid == 0) s_len = 0;
        for (int base = 0; base < nlist; base += 256) {
            const int c = base + tid;
            __syncthreads();
            if (c < nlist) chunk[tid] = qd[c];
            __syncthreads();
            if (tid == 0) {
                const int m = nlist - base < 256 ? nlist - base : 256;
                s_len = sorted_list_insert_run(chunk, (uint32_t)base, m, np, s_len, ls, lt);
            }
        }
        __syncthreads();
        if (tid == 0)
            for (int i = 0; i < np; ++i) probes[q * np + i] = i < s_len ? lt[i] : lt[0];
        return;
    }
    const int s = s_cnt;
    // Arrival order is ascending centroid index.
    uint64_t* ord = lds + cap;  // wave 1's buffer, free now
    int sort_n = 64;
    while (sort_n < s) sort_n <<= 1;
    for (int i = tid; i < sort_n; i += blockDim.x)
        ord[i] = i < s ? (((uint64_t)slot_id(top[i]) << 32) | (uint64_t)ordered_bits(slot_key(top[i])))
                       : kEmptySlot;
    __syncthreads();
    if (wave == 0) wave_bitonic_sort(ord, sort_n);
    __syncthreads();
    if (tid == 0) {
        float* in_s = reinterpret_cast<float*>(lds + 2 * cap);
        uint32_t* in_t = reinterpret_cast<uint32_t*>(in_s + s);
        float* ls = reinterpret_cast<float*>(lds + 3 * cap);
        uint32_t* lt = reinterpret_cast<uint32_t*>(ls + np);
        for (int i = 0; i < s; ++i) {
            in_s[i] = from_ordered_bits((uint32_t)ord[i]);
            in_t[i] = (uint32_t)(ord[i] >> 32);
        }
        const int cnt = sorted_list_replay(in_s, in_t, s, np, ls, lt);
        for (int i = 0; i < np; ++i) probes[q * np + i] = i < cnt ? lt[i] : lt[0];
    }
}

constexpr int kPqMaxM = 64;      // LUT of m x 256 floats in LDS

struct PqArgs {
    const uint8_t* codes;      // [n][m], packed list by list
    const uint32_t* list_ids;
    const float* coarse;
    const float* books;        // [m][256][dsub]
    const uint32_t* probes;    // [nq][np], probe order
    const int64_t* seg;        // [nq_launch][np][2]
    const int64_t* total;
    const int32_t* item_off;
    const int32_t* item_q;
    const float* rows;         // corpus rows and norms (exact rerank)
    const float* norms;
    float* tie;                // [nq_launch] the k_adc-th score of queries with status 1
    int64_t nq;                // queries in the launch
    int64_t chunk;             // rows per work item (multiple of 256)
    int np, m, dsub, dim, metric;
    int kadc, rerank;
};

// The residual's LUT, lut[s * 256 + c] = distance(residual_s, book_s,c)
// (distanceTableFlattened, ProductQuantizer.swift:223-253), built by the
// whole block.
__device__ __forceinline__ void pq_build_lut(const PqArgs& pa, const float* qres, float* lut) {
    const int tid = threadIdx.x;
    const int lut_n = pa.m * 256;
    if (pa.dsub == 2) {
        // Two-dimensional subvectors: each thread's codebook entries are
        // loaded in batches of 12 before any is used, so their latencies
        // overlap (one load at a time would serialise 48 of them).
        const float2* bk = reinterpret_cast<const float2*>(pa.books);
        constexpr int kB = 12;
        for (int e0 = tid; e0 < lut_n; e0 += 256 * kB) {
            float2 bv[kB];
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                const int e = e0 + 256 * u;
                bv[u] = e < lut_n ? bk[e] : make_float2(0.0f, 0.0f);
            }
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                const int e = e0 + 256 * u;
                if (e < lut_n) {
                    const float bb[2] = {bv[u].x, bv[u].y};
                    lut[e] = simd_distance(qres + 2 * (e >> 8), bb, 2, pa.metric);
                }
            }
        }
    } else {
        for (int e = tid; e < lut_n; e += 256) {
            const int s = e >> 8;
            lut[e] = simd_distance(qres + s * pa.dsub, pa.books + (int64_t)e * pa.dsub, pa.dsub,
                                   pa.metric);
        }
    }
}

// A row's ADC score: its m LUT entries added in code order
// (IVFPQIndex.swift:418-452).  cw: the row's codes as m / 4 words.
__device__ __forceinline__ float pq_score(const float* lut, const uint32_t* cw, int mw) {
    float score = 0.0f;
    for (int w = 0; w < mw; ++w) {
        const uint32_t word = cw[w];
        score += lut[(4 * w + 0) * 256 + (word & 0xFF)];
        score += lut[(4 * w + 1) * 256 + ((word >> 8) & 0xFF)];
        score += lut[(4 * w + 2) * 256 + ((word >> 16) & 0xFF)];
        score += lut[(4 * w + 3) * 256 + (word >> 24)];
    }
    return score;
}

// The query's final BoundedSortedList(k_adc) is (ls, lt)[0, nfin): scores
// and arrival indices.  Arrival indices become row ids; the list is written
// as it stands, or re-ranked by exact distance (rerank_k > 0).
template <int NCH>
__device__ __forceinline__ void pq_finish(const PqArgs& pa, const int64_t* seg, const float* qp,
                                          uint32_t q, int i, uint64_t* lds, float* ls,
                                          uint32_t* lt, int nfin, const FlatArgs& fa) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int kadc = pa.kadc;
    for (int t = tid; t < nfin; t += blockDim.x) {
        const int64_t arr = lt[t];
        int p = 0;
        while (p + 1 < pa.np && seg[2 * (p + 1) + 1] <= arr) ++p;
        lt[t] = pa.list_ids[seg[2 * p] + (arr - seg[2 * p + 1])];
    }
    __syncthreads();
    if (pa.rerank <= 0) {
        for (int t = tid; t < fa.k_stride; t += blockDim.x) {
            const bool in = t < nfin;
            fa.out_dist[(int64_t)q * fa.k_stride + t] = in ? ls[t] : kFltMax;
            fa.out_ids[(int64_t)q * fa.k_stride + t] = in ? lt[t] : kEmptyId;
        }
        if (tid == 0) fa.status[i] = 0;
        return;
    }
    // Exact rerank of the k_adc ids (no counterpart in the reference).
    uint64_t* rr = lds;  // candidates for final_rescore_f4: ids into the corpus
    for (int t = tid; t < kadc; t += blockDim.x) rr[t] = t < nfin ? pack_slot(0.0f, lt[t]) : kEmptySlot;
    __syncthreads();
    const int lr = lane & 15, dim4 = pa.dim >> 2;
    f4v qv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = lr + 16 * c;
        qv[c] = idx < dim4 ? *reinterpret_cast<const f4v*>(qp + 4 * idx) : f4v{0.f, 0.f, 0.f, 0.f};
    }
    final_rescore_f4<NCH>(qv, pa.rows, pa.norms, (int64_t)nfin, pa.dim, pa.metric, q, rr, kadc, fa,
                          kFltMax, kProofNone, nullptr, i);
}

// 1-D grid over work items; block 256; dynamic LDS: 4 * cap slots, then
// m * 256 + dim floats (LUT, residual).  Slots are (score, arrival index).
// MR > 0: two-dimensional subvectors with m <= MR a multiple of 16 (the
// codebook entries of this thread stay in registers, codes load as 16-byte
// words); MR = 0: any shape.  CAPT > 0: the wave lists' capacity is CAPT
// (their sorts compiled for that size).
template <int NCH, int MR, int CAPT>
__global__ __launch_bounds__(256) void ivfpq_scan(PqArgs pa, const float* __restrict__ queries,
                                                  const uint32_t* __restrict__ qidx, int kc, int cap,
                                                  FlatArgs fa) {
    extern __shared__ uint64_t lds[];
    float* lut = reinterpret_cast<float*>(lds + 4 * cap);
    float* qres = lut + pa.m * 256;
    __shared__ int s_cnt, s_over;
    const int tid = threadIdx.x, wave = tid >> 6;
    const int item = blockIdx.x;
    if (item >= pa.item_off[pa.nq]) return;  // past the last work item
    const int i = pa.item_q[item];
    const uint32_t q = qidx ? qidx[i] : (uint32_t)i;
    const int first = pa.item_off[i];
    const int nb = pa.item_off[i + 1] - first;
    const int j = item - first;
    const int64_t* seg = pa.seg + (int64_t)i * pa.np * 2;
    const uint32_t* probes = pa.probes + (int64_t)q * pa.np;
    const int64_t total = pa.total[i];
    const float* qp = queries + (int64_t)q * pa.dim;
    const int mw = pa.m >> 2;  // code words per row

    const int64_t lo = (int64_t)j * pa.chunk;
    const int64_t hi = lo + pa.chunk < total ? lo + pa.chunk : total;
    WaveTopKT<CAPT> sel;
    sel.init(lds + wave * cap, cap, kc);
    // MR > 0: this thread's codebook entries (code tid of every subspace)
    // stay in registers for all probes.
    constexpr int NB = MR > 0 ? MR : 1;
    constexpr int NC = MR > 0 ? MR / 16 : 4;  // 16-byte code words per row
    float2 bk[NB];
    if (MR > 0) {
        const float2* b2 = reinterpret_cast<const float2*>(pa.books);
#pragma unroll
        for (int u = 0; u < NB; ++u) bk[u] = u < pa.m ? b2[u * 256 + tid] : make_float2(0.0f, 0.0f);
    }
    // Codes of a row as 16-byte loads when m is a multiple of 16 (rows
    // then start 16-byte aligned), two 256-row batches ahead of their
    // scores (the first two while the LUT is built).  The score adds the m
    // entries in code order (IVFPQIndex.swift:418-452) either way.
    const int m16 = (pa.m & 15) == 0 && pa.m <= 16 * NC ? pa.m >> 4 : 0;
    for (int p = 0; p < pa.np; ++p) {
        const int64_t pre = seg[2 * p + 1];
        if (pre >= hi) break;
        const int64_t len = (p + 1 < pa.np ? seg[2 * p + 3] : total) - pre;
        const int64_t a = lo > pre ? lo - pre : 0;
        const int64_t b = hi - pre < len ? hi - pre : len;
        if (a >= b) continue;
        // The residual and its LUT (distanceTableFlattened, ProductQuantizer.swift:223-253).
        __syncthreads();
        const float* cen = pa.coarse + (int64_t)probes[p] * pa.dim;
        for (int d = tid; d < pa.dim; d += 256) qres[d] = qp[d] - cen[d];
        __syncthreads();
        const uint32_t* crow = reinterpret_cast<const uint32_t*>(pa.codes + (seg[2 * p] + a) * pa.m);
        const int64_t nrow = b - a;
        auto load_codes = [&](int64_t r, i4v (&c4)[NC]) {
            const uint32_t* cw = crow + (r < nrow ? r : 0) * mw;
#pragma unroll
            for (int c = 0; c < NC; ++c)
                c4[c] = c < m16 ? reinterpret_cast<const i4v*>(cw)[c] : i4v{0, 0, 0, 0};
        };
        i4v ca[NC], cb[NC], cc[NC];
        if (m16 > 0) {
            load_codes(tid, ca);
            load_codes(256 + tid, cb);
        }
        if (MR > 0) {
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                if (u < pa.m) {
                    const float2 r2 = reinterpret_cast<const float2*>(qres)[u];
                    const float ra[2] = {r2.x, r2.y}, bb[2] = {bk[u].x, bk[u].y};
                    lut[u * 256 + tid] = simd_distance(ra, bb, 2, pa.metric);
                }
            }
        } else {
            pq_build_lut(pa, qres, lut);
        }
        __syncthreads();
        // Scores rows base + tid (codes c4 when m16 > 0) and offers them.
        auto score_batch = [&](int64_t base, const i4v (&c4)[NC]) {
            const int64_t r = base + tid;
            const bool v = r < nrow;
            float score = 0.0f;
            if (m16 > 0) {
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    if (c < m16) {
#pragma unroll
                        for (int w = 0; w < 4; ++w) {
                            const uint32_t word = (uint32_t)c4[c][w];
                            const int sb = 16 * c + 4 * w;
                            score += lut[(sb + 0) * 256 + (word & 0xFF)];
                            score += lut[(sb + 1) * 256 + ((word >> 8) & 0xFF)];
                            score += lut[(sb + 2) * 256 + ((word >> 16) & 0xFF)];
                            score += lut[(sb + 3) * 256 + (word >> 24)];
                        }
                    }
                }
            } else {
                const uint32_t* cw = crow + (v ? r : 0) * mw;
                for (int w = 0; w < mw; ++w) {
                    const uint32_t word = cw[w];
                    score += lut[(4 * w + 0) * 256 + (word & 0xFF)];
                    score += lut[(4 * w + 1) * 256 + ((word >> 8) & 0xFF)];
                    score += lut[(4 * w + 2) * 256 + ((word >> 16) & 0xFF)];
                    score += lut[(4 * w + 3) * 256 + (word >> 24)];
                }
            }
            sel.offer(v, score, (uint32_t)(pre + a + r));
        };
        for (int64_t base = 0; base < nrow; base += 768) {
            if (m16 > 0) load_codes(base + 512 + tid, cc);
            score_batch(base, ca);
            if (base + 256 >= nrow) break;
            if (m16 > 0) load_codes(base + 768 + tid, ca);
            score_batch(base + 256, cb);
            if (base + 512 >= nrow) break;
            if (m16 > 0) load_codes(base + 1024 + tid, cb);
            score_batch(base + 512, cc);
        }
    }
    sel.finish();
    block_fold(sel, lds, cap);
    if (tid < 64)
        for (int s = tid; s < kc; s += 64)
            store_shared_slot(&fa.cand[(int64_t)item * kc + s], s < sel.count ? sel.buf[s] : kEmptySlot);
    uint32_t* cnt = fa.counters + i;
    if (!block_arrive_last(cnt, (uint32_t)nb)) return;
    if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    block_select_lists(fa.cand + (int64_t)first * kc, (int64_t)nb * kc, lds, cap, kc, sel);

    // lds[0, kc): the kc smallest (score, arrival).  S: those <= T, the
    // k_adc-th smallest score.
    uint64_t* top = lds;
    const int kadc = pa.kadc;
    if (tid == 0) {
        int ncand = 0;
        while (ncand < kc && top[ncand] != kEmptySlot) ++ncand;
        int s = ncand;
        if (ncand >= kadc) {
            const float t = slot_key(top[kadc - 1]);
            s = kadc;
            while (s < ncand && slot_key(top[s]) <= t) ++s;
        }
        s_cnt = s;
        s_over = (s == kc && (int64_t)kc < total) ? 1 : 0;
    }
    __syncthreads();
    const int s = s_cnt;
    if (s_over) {
        // More rows may tie at T than were kept: ivfpq_tie_replay finishes
        // the query.
        if (tid == 0) {
            fa.status[i] = 1;
            pa.tie[i] = slot_key(top[kadc - 1]);
        }
        return;
    }
    // Order: arrival ascending.
    uint64_t* ord = lds + cap;
    int sort_n = 64;
    while (sort_n < s) sort_n <<= 1;
    for (int t = tid; t < sort_n; t += blockDim.x)
        ord[t] = t < s ? (((uint64_t)slot_id(top[t]) << 32) | (uint64_t)ordered_bits(slot_key(top[t])))
                       : kEmptySlot;
    __syncthreads();
    if (wave == 0) wave_bitonic_sort(ord, sort_n);
    __syncthreads();
    // Final BoundedSortedList(kadc) content in lds[2 cap ...]: score, arrival.
    float* ls = reinterpret_cast<float*>(lds + 2 * cap);
    uint32_t* lt = reinterpret_cast<uint32_t*>(ls + kadc);
    __shared__ int s_final;
    if (s <= kadc) {
        // Nothing is evicted: (score ascending, later arrival first).
        uint64_t* fin = lds;  // top is no longer needed
        for (int t = tid; t < sort_n; t += blockDim.x)
            fin[t] = t < s ? (((uint64_t)(uint32_t)ord[t] << 32) | (uint64_t)(~(uint32_t)(ord[t] >> 32)))
                           : kEmptySlot;
        __syncthreads();
        if (wave == 0) wave_bitonic_sort(fin, sort_n);
        __syncthreads();
        for (int t = tid; t < s; t += blockDim.x) {
            ls[t] = from_ordered_bits((uint32_t)(fin[t] >> 32));
            lt[t] = ~(uint32_t)fin[t];
        }
        if (tid == 0) s_final = s;
    } else if (tid == 0) {
        float* in_s = reinterpret_cast<float*>(lds + 3 * cap);
        uint32_t* in_t = reinterpret_cast<uint32_t*>(in_s + s);
        for (int t = 0; t < s; ++t) {
            in_s[t] = from_ordered_bits((uint32_t)ord[t]);
            in_t[t] = (uint32_t)(ord[t] >> 32);
        }
        s_final = sorted_list_replay(in_s, in_t, s, kadc, ls, lt);
    }
    __syncthreads();
    pq_finish<NCH>(pa, seg, qp, q, i, lds, ls, lt, s_final, fa);
}

// Queries with more rows tied at the k_adc-th score T than ivfpq_scan kept
// (a zero query, duplicate rows): one block per query scores every probed
// row again in arrival order and one thread inserts those at or below T
// into the BoundedSortedList in that order, which is the list's outcome for
// any number of ties (rows above T never enter it: k_adc rows score at or
// below T).  grid: the queries' launch indices `over`; LDS as ivfpq_scan.
template <int NCH>
__global__ __launch_bounds__(256) void ivfpq_tie_replay(PqArgs pa, const float* __restrict__ queries,
                                                        const uint32_t* __restrict__ qidx,
                                                        const int32_t* __restrict__ over, int cap,
                                                        FlatArgs fa) {
    extern __shared__ uint64_t lds[];
    float* lut = reinterpret_cast<float*>(lds + 4 * cap);
    float* qres = lut + pa.m * 256;
    __shared__ int s_len, s_wcnt[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i = over[blockIdx.x];
    const uint32_t q = qidx ? qidx[i] : (uint32_t)i;
    const int64_t* seg = pa.seg + (int64_t)i * pa.np * 2;
    const uint32_t* probes = pa.probes + (int64_t)q * pa.np;
    const int64_t total = pa.total[i];
    const float* qp = queries + (int64_t)q * pa.dim;
    const float t_cut = pa.tie[i];
    const int mw = pa.m >> 2;
    float* ls = reinterpret_cast<float*>(lds + 2 * cap);
    uint32_t* lt = reinterpret_cast<uint32_t*>(ls + pa.kadc);
    float* st_s = reinterpret_cast<float*>(lds + 3 * cap);
    uint32_t* st_t = reinterpret_cast<uint32_t*>(st_s + 256);
    if (tid == 0) s_len = 0;
    for (int p = 0; p < pa.np; ++p) {
        const int64_t pre = seg[2 * p + 1];
        const int64_t len = (p + 1 < pa.np ? seg[2 * p + 3] : total) - pre;
        if (len <= 0) continue;
        __syncthreads();
        const float* cen = pa.coarse + (int64_t)probes[p] * pa.dim;
        for (int d = tid; d < pa.dim; d += 256) qres[d] = qp[d] - cen[d];
        __syncthreads();
        pq_build_lut(pa, qres, lut);
        __syncthreads();
        const uint32_t* crow = reinterpret_cast<const uint32_t*>(pa.codes + seg[2 * p] * pa.m);
        for (int64_t base = 0; base < len; base += 256) {
            const int64_t r = base + tid;
            float score = 0.0f;
            bool keep = false;
            if (r < len) {
                score = pq_score(lut, crow + r * mw, mw);
                keep = score <= t_cut;
            }
            const uint64_t bal = __ballot(keep);
            if (lane == 0) s_wcnt[wave] = __popcll(bal);
            __syncthreads();
            int off = 0;
            for (int w = 0; w < wave; ++w) off += s_wcnt[w];
            const int nkeep = s_wcnt[0] + s_wcnt[1] + s_wcnt[2] + s_wcnt[3];
            if (keep) {
                const int pos = off + __popcll(bal & lanemask_lt());
                st_s[pos] = score;
                st_t[pos] = (uint32_t)(pre + r);
            }
            __syncthreads();
            if (tid == 0) {
                int cnt = s_len;
                for (int t = 0; t < nkeep; ++t) cnt = sorted_list_insert(st_s[t], st_t[t], cnt, pa.kadc, ls, lt);
                s_len = cnt;
            }
            __syncthreads();
        }
    }
    __syncthreads();
    pq_finish<NCH>(pa, seg, qp, q, i, lds, ls, lt, s_len, fa);
}

}  // namespace mans

struct mans_ivfpq {
    mans_ctx* ctx = nullptr;
    const mans_corpus* corpus = nullptr;  // rows for the exact rerank (outlives the index)
    int64_t n = 0, dim = 0, nlist = 0, m = 0, dsub = 0;
    uint32_t metric = 0;
    mans::DevBuf coarse, books, offsets, list_ids, codes, assign;
    mans::DevBuf coarse_t;  // centroids dimension-major ([dim][nlist]) for the probe scan
    std::vector<int64_t> h_offsets;
};

namespace mans {

constexpr int kPqMaxKadc = 512;

template <int NCH>
static void launch_pq_scan(int64_t items, int cap, int kc, const PqArgs& pa, const float* queries,
                           const uint32_t* qidx, const FlatArgs& fa, hipStream_t s) {
    const size_t shmem = sizeof(uint64_t) * 4 * (size_t)cap + sizeof(float) * ((size_t)pa.m * 256 + pa.dim);
    // Two-dimensional subvectors, m a multiple of 16 up to 48: codebook
    // entries in registers (and wave lists of 512 slots compiled for that
    // size); any other shape takes the general kernel.
    const bool regs = pa.dsub == 2 && (pa.m & 15) == 0 && pa.m <= 48;
    if (regs && cap == 512)
        hipLaunchKernelGGL((ivfpq_scan<NCH, 48, 512>), dim3((unsigned)items), dim3(256), shmem, s,
                           pa, queries, qidx, kc, cap, fa);
    else if (regs)
        hipLaunchKernelGGL((ivfpq_scan<NCH, 48, 0>), dim3((unsigned)items), dim3(256), shmem, s, pa,
                           queries, qidx, kc, cap, fa);
    else
        hipLaunchKernelGGL((ivfpq_scan<NCH, 0, 0>), dim3((unsigned)items), dim3(256), shmem, s, pa,
                           queries, qidx, kc, cap, fa);
}

template <int NCH>
static void launch_pq_replay(unsigned grid, int cap, const PqArgs& pa, const float* queries,
                             const int32_t* over, const FlatArgs& fa, hipStream_t s) {
    const size_t shmem = sizeof(uint64_t) * 4 * (size_t)cap + sizeof(float) * ((size_t)pa.m * 256 + pa.dim);
    hipLaunchKernelGGL(ivfpq_tie_replay<NCH>, dim3(grid), dim3(256), shmem, s, pa, queries,
                       (const uint32_t*)nullptr, over, cap, fa);
}

static int ivfpq_search_run(mans_ctx* ctx, const mans_ivfpq* pq, const float* d_q, int64_t nq,
                            int64_t k_adc, int64_t nprobe, int64_t rerank_k, float* d_score,
                            uint32_t* d_ids, hipStream_t st, Slot* slot) {
    if (nq <= 0 || k_adc <= 0) return MANS_OK;
    if (ctx->fail_launch) return fail(MANS_EXECUTION_FAILED, "injected launch failure");
    if (k_adc > kPqMaxKadc) return fail(MANS_SEARCH_FAILED, "IVF-PQ: k above 512");
    if (rerank_k > k_adc) return fail(MANS_SEARCH_FAILED, "IVF-PQ: rerank_k above k");
    if (rerank_k > 0 && !pq->corpus)
        return fail(MANS_SEARCH_FAILED, "IVF-PQ: the exact rerank needs the index's corpus rows");
    if (nq > 16384) return fail(MANS_SEARCH_FAILED, "IVF-PQ: at most 16384 queries per call");
    if ((reinterpret_cast<uintptr_t>(d_q) & 15u) != 0)
        return fail(MANS_SEARCH_FAILED, "IVF-PQ: queries must be 16-byte aligned");
    const int dim = (int)pq->dim;
    const int nch = flat_nch_for_dim(dim);
    if (rerank_k > 0 && (nch == 0 || nch > 8))
        return fail(MANS_PIPELINE_UNAVAILABLE, "IVF-PQ rerank: dim must be a multiple of 4, at most 512");
    const int np = (int)std::max<int64_t>(1, std::min<int64_t>(nprobe, pq->nlist));
    if (np > 960) return fail(MANS_SEARCH_FAILED, "IVF-PQ: nprobe above 960");
    const int kout = rerank_k > 0 ? (int)rerank_k : (int)k_adc;

    hipError_t e = slot->aux1.ensure((size_t)nq * np * sizeof(uint32_t), ctx->fail_alloc);
    if (e != hipSuccess) return hip_fail(e, "IVF-PQ probe workspace");
    const uint32_t* d_probes = (const uint32_t*)slot->aux1.p;

    const int64_t avg_rows = std::max<int64_t>(1, pq->n * np / std::max<int64_t>(1, pq->nlist));
    int64_t max_rows = 0;
    {
        std::vector<int64_t> sizes((size_t)pq->nlist);
        for (int64_t c = 0; c < pq->nlist; ++c) sizes[c] = pq->h_offsets[c + 1] - pq->h_offsets[c];
        std::nth_element(sizes.begin(), sizes.begin() + (np - 1), sizes.end(), std::greater<int64_t>());
        for (int p = 0; p < np; ++p) max_rows += sizes[p];
    }
    static const int64_t target_items = [] {
        const char* ev = std::getenv("MANS_IVFPQ_BLOCKS");
        return ev ? std::max<int64_t>(1, std::atoll(ev)) : (int64_t)512;
    }();
    // One pass keeps the k_adc + 64 smallest (score, arrival) per query;
    // queries with more ties at the k_adc-th score than that are finished by
    // ivfpq_tie_replay.
    const int kc = (int)k_adc + 64;
    const int cap = flat_cap_for(kc);
    const int64_t npend = nq;
    int64_t chunk = (avg_rows * npend + target_items - 1) / target_items;
    chunk = std::max<int64_t>(256, (chunk + 255) / 256 * 256);
    const int64_t items_bound = npend * std::max<int64_t>(1, (max_rows + chunk - 1) / chunk);
    const size_t seg_bytes = (size_t)npend * np * 2 * sizeof(int64_t);
    e = slot->aux2.ensure(seg_bytes + (size_t)npend * (sizeof(int64_t) + sizeof(float)), ctx->fail_alloc);
    if (e == hipSuccess)
        e = slot->aux3.ensure((size_t)(2 * npend + 1 + items_bound) * sizeof(int32_t), ctx->fail_alloc);
    // The candidates' workspace first holds the probes' centroid distances.
    if (e == hipSuccess)
        e = slot->cand.ensure(std::max((size_t)items_bound * kc * sizeof(uint64_t),
                                       (size_t)npend * pq->nlist * sizeof(float)),
                              ctx->fail_alloc);
    if (e == hipSuccess) e = slot->status.ensure((size_t)npend, ctx->fail_alloc);
    if (e == hipSuccess) e = slot->qidx.ensure((size_t)npend * sizeof(int32_t), ctx->fail_alloc);
    if (e == hipSuccess && (slot->counters.bytes < (size_t)npend * sizeof(uint32_t) || slot->counters_dirty)) {
        e = slot->counters.ensure((size_t)npend * sizeof(uint32_t), ctx->fail_alloc);
        if (e == hipSuccess) e = hipMemsetAsync(slot->counters.p, 0, slot->counters.bytes, st);
        slot->counters_dirty = false;
    }
    if (e == hipSuccess) e = slot->status_h.ensure((size_t)npend);
    if (e != hipSuccess) return hip_fail(e, "IVF-PQ workspace");
    // Probes (BoundedSortedList order): every query's centroid distances
    // (in the candidate workspace, free until the scan), then the selection.
    const int pkc = np + 64;
    const int pcap = flat_cap_for(pkc);
    ctx->time_begin(slot, st);
    {
        const dim3 grid((unsigned)((pq->nlist + 255) / 256), (unsigned)((nq + kPqDistQ - 1) / kPqDistQ));
        const size_t shm = sizeof(float) * ((size_t)kPqDistQ * dim + kPqDistQ);
        float* dists = (float*)slot->cand.p;
        const float* ct = (const float*)pq->coarse_t.p;
        const int nl = (int)pq->nlist;
        switch ((int)pq->metric) {
        case kMetricL2:
            hipLaunchKernelGGL(pq_coarse_dist<kMetricL2>, grid, dim3(256), shm, st, d_q, nq, dim, ct, nl, dists);
            break;
        case kMetricIP:
            hipLaunchKernelGGL(pq_coarse_dist<kMetricIP>, grid, dim3(256), shm, st, d_q, nq, dim, ct, nl, dists);
            break;
        default:
            hipLaunchKernelGGL(pq_coarse_dist<kMetricCosine>, grid, dim3(256), shm, st, d_q, nq, dim, ct, nl, dists);
            break;
        }
        if (pcap == 256)
            hipLaunchKernelGGL(pq_probes<256>, dim3((unsigned)nq), dim3(256),
                               sizeof(uint64_t) * 4 * (size_t)pcap, st, (const float*)dists, nl, np,
                               pkc, pcap, (uint32_t*)slot->aux1.p);
        else
            hipLaunchKernelGGL(pq_probes<0>, dim3((unsigned)nq), dim3(256),
                               sizeof(uint64_t) * 4 * (size_t)pcap, st, (const float*)dists, nl, np,
                               pkc, pcap, (uint32_t*)slot->aux1.p);
    }
    e = hipGetLastError();
    ctx->time_end(slot, st, "ivfpq_probe");
    if (e != hipSuccess) return hip_fail(e, "IVF-PQ probes");
    ctx->time_begin(slot, st);
    int64_t* d_seg = (int64_t*)slot->aux2.p;
    int64_t* d_total = (int64_t*)((char*)slot->aux2.p + seg_bytes);
    float* d_tie = (float*)(d_total + npend);
    int32_t* d_nitems = (int32_t*)slot->aux3.p;
    int32_t* d_item_off = d_nitems + npend;
    int32_t* d_item_q = d_item_off + npend + 1;
    hipLaunchKernelGGL(ivf_plan, dim3((unsigned)((npend + 3) / 4)), dim3(256), 0, st, d_probes, np,
                       (const uint32_t*)nullptr, npend, (const int64_t*)pq->offsets.p, chunk, d_seg,
                       d_total, d_nitems);
    hipLaunchKernelGGL(ivf_items, dim3(1), dim3(1024), 0, st, (const int32_t*)d_nitems, npend,
                       d_item_off, d_item_q);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "IVF-PQ plan");
    PqArgs pa;
    pa.codes = (const uint8_t*)pq->codes.p;
    pa.list_ids = (const uint32_t*)pq->list_ids.p;
    pa.coarse = (const float*)pq->coarse.p;
    pa.books = (const float*)pq->books.p;
    pa.probes = d_probes;
    pa.seg = d_seg;
    pa.total = d_total;
    pa.item_off = d_item_off;
    pa.item_q = d_item_q;
    // Rows serve only the exact rerank (refused above without a corpus).
    pa.rows = pq->corpus ? (const float*)pq->corpus->rows.p : nullptr;
    pa.norms = pq->corpus ? (const float*)pq->corpus->norms.p : nullptr;
    pa.tie = d_tie;
    pa.nq = npend;
    pa.chunk = chunk;
    pa.np = np;
    pa.m = (int)pq->m;
    pa.dsub = (int)pq->dsub;
    pa.dim = dim;
    pa.metric = (int)pq->metric;
    pa.kadc = (int)k_adc;
    pa.rerank = (int)rerank_k;
    FlatArgs fa = {};
    fa.cand = (uint64_t*)slot->cand.p;
    fa.counters = (uint32_t*)slot->counters.p;
    fa.out_dist = d_score;
    fa.out_ids = d_ids;
    fa.status = (uint8_t*)slot->status.p;
    fa.k = kout;
    fa.k_stride = kout;
    const int lnch = rerank_k > 0 ? nch : 1;
    switch (lnch) {
    case 1: launch_pq_scan<1>(items_bound, cap, kc, pa, d_q, nullptr, fa, st); break;
    case 2: launch_pq_scan<2>(items_bound, cap, kc, pa, d_q, nullptr, fa, st); break;
    case 3: launch_pq_scan<3>(items_bound, cap, kc, pa, d_q, nullptr, fa, st); break;
    case 4: launch_pq_scan<4>(items_bound, cap, kc, pa, d_q, nullptr, fa, st); break;
    case 6: launch_pq_scan<6>(items_bound, cap, kc, pa, d_q, nullptr, fa, st); break;
    case 8: launch_pq_scan<8>(items_bound, cap, kc, pa, d_q, nullptr, fa, st); break;
    default: return fail(MANS_PIPELINE_UNAVAILABLE, "IVF-PQ: unsupported dim");
    }
    e = hipGetLastError();
    ctx->time_end(slot, st, "ivfpq_scan");
    if (e == hipSuccess)
        e = hipMemcpyAsync(slot->status_h.p, slot->status.p, (size_t)npend, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        slot->counters_dirty = true;
        return hip_fail(e, "IVF-PQ scan");
    }
    const uint8_t* sh = (const uint8_t*)slot->status_h.p;
    std::vector<int32_t> over;
    for (int64_t i = 0; i < npend; ++i)
        if (sh[i]) over.push_back((int32_t)i);
    if (!over.empty()) {
        e = hipMemcpyAsync(slot->qidx.p, over.data(), over.size() * sizeof(int32_t),
                           hipMemcpyHostToDevice, st);
        if (e != hipSuccess) return hip_fail(e, "IVF-PQ tie replay");
        const unsigned grid = (unsigned)over.size();
        const int32_t* d_over = (const int32_t*)slot->qidx.p;
        ctx->time_begin(slot, st);
        switch (lnch) {
        case 1: launch_pq_replay<1>(grid, cap, pa, d_q, d_over, fa, st); break;
        case 2: launch_pq_replay<2>(grid, cap, pa, d_q, d_over, fa, st); break;
        case 3: launch_pq_replay<3>(grid, cap, pa, d_q, d_over, fa, st); break;
        case 4: launch_pq_replay<4>(grid, cap, pa, d_q, d_over, fa, st); break;
        case 6: launch_pq_replay<6>(grid, cap, pa, d_q, d_over, fa, st); break;
        case 8: launch_pq_replay<8>(grid, cap, pa, d_q, d_over, fa, st); break;
        }
        e = hipGetLastError();
        ctx->time_end(slot, st, "ivfpq_tie_replay");
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "IVF-PQ tie replay");
    }
    return MANS_OK;
}

}  // namespace mans

using namespace mans;

extern "C" {

int mans_ivfpq_build(mans_ctx* ctx, const mans_corpus* corpus, const float* coarse, int64_t nlist,
                     const float* codebooks, int64_t m, uint32_t metric, mans_ivfpq** out) {
    if (out) *out = nullptr;
    if (!ctx || !corpus || !coarse || !codebooks || !out)
        return fail(MANS_SEARCH_FAILED, "mans_ivfpq_build: NULL argument");
    const int64_t n = corpus->n, dim = corpus->dim;
    if (nlist < 1) return fail(MANS_SEARCH_FAILED, "mans_ivfpq_build: nlist must be >= 1");
    if (m < 1 || dim % m != 0) return fail(MANS_DIMENSION_MISMATCH, "IVF-PQ: dim must be a multiple of m");
    if (m % 4 != 0 || m > kPqMaxM)
        return fail(MANS_PIPELINE_UNAVAILABLE, "IVF-PQ: m must be a multiple of 4, at most 64");
    if (metric > 2) return fail(MANS_SEARCH_FAILED, "IVF-PQ does not support this metric");
    DeviceGuard dg(ctx->device);
    SlotLease lease(ctx);
    if (!lease.slot) return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    hipStream_t st = lease.slot->stream;
    auto* pq = new mans_ivfpq();
    pq->ctx = ctx;
    pq->corpus = corpus;
    pq->n = n;
    pq->dim = dim;
    pq->nlist = nlist;
    pq->m = m;
    pq->dsub = dim / m;
    pq->metric = metric;
    const size_t nn = (size_t)(n ? n : 1);
    hipError_t e = pq->coarse.ensure((size_t)nlist * dim * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = pq->books.ensure((size_t)m * 256 * pq->dsub * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = pq->offsets.ensure((nlist + 1) * sizeof(int64_t), ctx->fail_alloc);
    if (e == hipSuccess) e = pq->list_ids.ensure(nn * sizeof(uint32_t), ctx->fail_alloc);
    if (e == hipSuccess) e = pq->codes.ensure(nn * m, ctx->fail_alloc);
    if (e == hipSuccess) e = pq->assign.ensure(nn * sizeof(int32_t), ctx->fail_alloc);
    if (e == hipSuccess)
        e = hipMemcpyAsync(pq->coarse.p, coarse, (size_t)nlist * dim * sizeof(float), hipMemcpyHostToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(pq->books.p, codebooks, (size_t)m * 256 * pq->dsub * sizeof(float),
                           hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = pq->coarse_t.ensure((size_t)nlist * dim * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess && nlist > 0) {
        const int64_t cells = nlist * dim;
        hipLaunchKernelGGL(transpose_kernel, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, st,
                           (const float*)pq->coarse.p, nlist, (int)dim, (float*)pq->coarse_t.p);
        e = hipGetLastError();
    }
    if (e != hipSuccess) {
        delete pq;
        return hip_fail(e, "IVF-PQ upload");
    }
    // Coarse assignment in row order.
    const unsigned blocks = (unsigned)((n + 255) / 256);
    const float* rows = (const float*)corpus->rows.p;
    int32_t* d_assign = (int32_t*)pq->assign.p;
    if (n > 0) {
        switch (dim) {
        case 32: hipLaunchKernelGGL(pq_assign<32>, dim3(blocks), dim3(256), 0, st, rows, n, (const float*)pq->coarse.p, (int)nlist, (int)metric, d_assign); break;
        case 64: hipLaunchKernelGGL(pq_assign<64>, dim3(blocks), dim3(256), 0, st, rows, n, (const float*)pq->coarse.p, (int)nlist, (int)metric, d_assign); break;
        case 96: hipLaunchKernelGGL(pq_assign<96>, dim3(blocks), dim3(256), 0, st, rows, n, (const float*)pq->coarse.p, (int)nlist, (int)metric, d_assign); break;
        case 128: hipLaunchKernelGGL(pq_assign<128>, dim3(blocks), dim3(256), 0, st, rows, n, (const float*)pq->coarse.p, (int)nlist, (int)metric, d_assign); break;
        default:
            hipLaunchKernelGGL(pq_assign_any, dim3(blocks), dim3(256), 0, st, rows, n, (int)dim,
                               (const float*)pq->coarse.p, (int)nlist, (int)metric, d_assign);
        }
        e = hipGetLastError();
    }
    std::vector<int32_t> assign((size_t)n);
    if (e == hipSuccess && n > 0)
        e = hipMemcpyAsync(assign.data(), d_assign, n * sizeof(int32_t), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        delete pq;
        return hip_fail(e, "IVF-PQ assignment");
    }
    // Lists in add order (IVFPQIndex.swift:140-159: rows are appended as added).
    pq->h_offsets.assign((size_t)nlist + 1, 0);
    for (int64_t r = 0; r < n; ++r) pq->h_offsets[assign[r] + 1]++;
    for (int64_t c = 0; c < nlist; ++c) pq->h_offsets[c + 1] += pq->h_offsets[c];
    std::vector<uint32_t> ids((size_t)n);
    {
        std::vector<int64_t> cur(pq->h_offsets.begin(), pq->h_offsets.end() - 1);
        for (int64_t r = 0; r < n; ++r) ids[cur[assign[r]]++] = (uint32_t)r;
    }
    e = hipMemcpyAsync(pq->offsets.p, pq->h_offsets.data(), (nlist + 1) * sizeof(int64_t),
                       hipMemcpyHostToDevice, st);
    if (e == hipSuccess && n > 0)
        e = hipMemcpyAsync(pq->list_ids.p, ids.data(), n * sizeof(uint32_t), hipMemcpyHostToDevice, st);
    if (e == hipSuccess && n > 0) {
        hipLaunchKernelGGL(pq_encode, dim3(blocks), dim3(256), 0, st, rows, (int)dim,
                           (const uint32_t*)pq->list_ids.p, (const int32_t*)d_assign, n,
                           (const float*)pq->coarse.p, (const float*)pq->books.p, (int)m,
                           (int)pq->dsub, (uint8_t*)pq->codes.p);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        delete pq;
        return hip_fail(e, "IVF-PQ encode");
    }
    *out = pq;
    return MANS_OK;
}

int mans_ivfpq_search_device(mans_ctx* ctx, const mans_ivfpq* pq, const float* d_queries, int64_t nq,
                             int64_t k_adc, int64_t nprobe, int64_t rerank_k, float* d_out_score,
                             uint32_t* d_out_ids, void* stream) {
    if (!ctx || !pq) return fail(MANS_SEARCH_FAILED, "NULL context or index");
    if (check_k(k_adc) != MANS_OK || check_k(rerank_k) != MANS_OK) return MANS_SEARCH_FAILED;
    if (nq > 0 && k_adc > 0 && (!d_queries || !d_out_score || !d_out_ids))
        return fail(MANS_SEARCH_FAILED, "NULL buffer");
    DeviceGuard dg(ctx->device);
    SlotLease lease(ctx);
    if (!lease.slot) return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    hipStream_t st = stream ? (hipStream_t)stream : lease.slot->stream;
    return ivfpq_search_run(ctx, pq, d_queries, nq, k_adc, nprobe, rerank_k, d_out_score, d_out_ids,
                            st, lease.slot);
}

int mans_ivfpq_search(mans_ctx* ctx, const mans_ivfpq* pq, const float* queries, int64_t nq,
                      int64_t k_adc, int64_t nprobe, int64_t rerank_k, float* out_score,
                      uint32_t* out_ids) {
    if (!ctx || !pq) return fail(MANS_SEARCH_FAILED, "NULL context or index");
    if (check_k(k_adc) != MANS_OK || check_k(rerank_k) != MANS_OK) return MANS_SEARCH_FAILED;
    if (nq <= 0 || k_adc <= 0) return MANS_OK;
    if (!queries || !out_score || !out_ids) return fail(MANS_SEARCH_FAILED, "NULL buffer");
    DeviceGuard dg(ctx->device);
    SlotLease lease(ctx);
    Slot* s = lease.slot;
    if (!s) return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    const int64_t kout = rerank_k > 0 ? rerank_k : k_adc;
    const size_t qbytes = (size_t)nq * pq->dim * sizeof(float);
    const size_t obytes = (size_t)nq * kout * sizeof(float);
    hipError_t e = s->queries.ensure(qbytes, ctx->fail_alloc);
    if (e == hipSuccess) e = s->dist.ensure(obytes, ctx->fail_alloc);
    if (e == hipSuccess) e = s->ids.ensure(obytes, ctx->fail_alloc);
    if (e == hipSuccess) e = stage_to_device(s, s->queries.p, queries, qbytes);
    if (e != hipSuccess) return hip_fail(e, "IVF-PQ staging");
    int rc = ivfpq_search_run(ctx, pq, (const float*)s->queries.p, nq, k_adc, nprobe, rerank_k,
                              (float*)s->dist.p, (uint32_t*)s->ids.p, s->stream, s);
    if (rc != MANS_OK) return rc;
    e = stage_from_device(s, out_score, s->dist.p, obytes, out_ids, s->ids.p, obytes);
    return e == hipSuccess ? MANS_OK : hip_fail(e, "IVF-PQ results");
}

int mans_ivfpq_download_codes(const mans_ivfpq* pq, uint8_t* codes, int32_t* assign) {
    if (!pq) return fail(MANS_SEARCH_FAILED, "NULL index");
    DeviceGuard dg(pq->ctx->device);
    const int64_t n = pq->n, m = pq->m;
    hipError_t e = hipSuccess;
    if (codes && n > 0) {
        std::vector<uint8_t> packed((size_t)(n * m));
        std::vector<uint32_t> ids((size_t)n);
        e = hipMemcpy(packed.data(), pq->codes.p, packed.size(), hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(ids.data(), pq->list_ids.p, n * sizeof(uint32_t), hipMemcpyDeviceToHost);
        if (e == hipSuccess)
            for (int64_t pos = 0; pos < n; ++pos)
                std::memcpy(codes + (int64_t)ids[pos] * m, packed.data() + pos * m, (size_t)m);
    }
    if (e == hipSuccess && assign && n > 0)
        e = hipMemcpy(assign, pq->assign.p, n * sizeof(int32_t), hipMemcpyDeviceToHost);
    return e == hipSuccess ? MANS_OK : hip_fail(e, "IVF-PQ codes download");
}

void mans_ivfpq_release(mans_ivfpq* pq) {
    if (!pq) return;
    DeviceGuard dg(pq->ctx->device);
    (void)hipDeviceSynchronize();
    delete pq;
}

// ---------------------------------------------------------------------------
// Binary persistence (in place of the JSON "IVFP" state of
// IVFPQIndex.swift:252-324): a 48-byte header -- "IVPB", version, dim,
// metric, n, nlist, m, dsub -- then the coarse centroids (nlist x dim f32),
// the codebooks (m x 256 x dsub f32), the list offsets (nlist + 1 i64), the
// list ids (n u32, row ids list by list), the codes (n x m u8 in list
// order) and the coarse assignment (n i32 in row order), little-endian.

namespace {

constexpr uint32_t kIvpbVersion = 1;
constexpr size_t kIvpbHeader = 48;

struct IvpbHeader {
    char magic[4];
    uint32_t version, dim, metric;
    uint64_t n, nlist;
    uint32_t m, dsub;
    uint64_t reserved;
};
static_assert(sizeof(IvpbHeader) == kIvpbHeader, "IVPB header layout");

// Byte offsets of the sections after the header, overflow-checked.
bool ivpb_layout(uint64_t n, uint64_t nlist, uint64_t dim, uint64_t m, uint64_t dsub,
                 uint64_t off[7]) {
    uint64_t sz[6], t;
    if (__builtin_mul_overflow(nlist, dim, &t) || __builtin_mul_overflow(t, 4, &sz[0])) return false;
    if (__builtin_mul_overflow(m, 256 * dsub, &t) || __builtin_mul_overflow(t, 4, &sz[1])) return false;
    if (__builtin_add_overflow(nlist, 1, &t) || __builtin_mul_overflow(t, 8, &sz[2])) return false;
    if (__builtin_mul_overflow(n, 4, &sz[3])) return false;
    if (__builtin_mul_overflow(n, m, &sz[4])) return false;
    sz[5] = sz[3];
    off[0] = kIvpbHeader;
    for (int i = 0; i < 6; ++i)
        if (__builtin_add_overflow(off[i], sz[i], &off[i + 1])) return false;
    return true;
}

int write_all(FILE* f, const void* p, size_t bytes) {
    return fwrite(p, 1, bytes, f) == bytes ? MANS_OK : fail(MANS_SEARCH_FAILED, "IVF-PQ save: write failed");
}

}  // namespace

int mans_ivfpq_save(const mans_ivfpq* pq, const char* path) {
    if (!pq || !path) return fail(MANS_SEARCH_FAILED, "mans_ivfpq_save: NULL argument");
    DeviceGuard dg(pq->ctx->device);
    const int64_t n = pq->n, nlist = pq->nlist, dim = pq->dim, m = pq->m, dsub = pq->dsub;
    std::vector<float> coarse((size_t)(nlist * dim)), books((size_t)(m * 256 * dsub));
    std::vector<uint32_t> ids((size_t)n);
    std::vector<uint8_t> codes((size_t)(n * m));
    std::vector<int32_t> assign((size_t)n);
    hipError_t e = hipMemcpy(coarse.data(), pq->coarse.p, coarse.size() * sizeof(float), hipMemcpyDeviceToHost);
    if (e == hipSuccess)
        e = hipMemcpy(books.data(), pq->books.p, books.size() * sizeof(float), hipMemcpyDeviceToHost);
    if (e == hipSuccess && n > 0) {
        e = hipMemcpy(ids.data(), pq->list_ids.p, ids.size() * sizeof(uint32_t), hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(codes.data(), pq->codes.p, codes.size(), hipMemcpyDeviceToHost);
        if (e == hipSuccess)
            e = hipMemcpy(assign.data(), pq->assign.p, assign.size() * sizeof(int32_t), hipMemcpyDeviceToHost);
    }
    if (e != hipSuccess) return hip_fail(e, "IVF-PQ save download");
    IvpbHeader h = {};
    std::memcpy(h.magic, "IVPB", 4);
    h.version = kIvpbVersion;
    h.dim = (uint32_t)dim;
    h.metric = pq->metric;
    h.n = (uint64_t)n;
    h.nlist = (uint64_t)nlist;
    h.m = (uint32_t)m;
    h.dsub = (uint32_t)dsub;
    const std::string tmp = std::string(path) + ".tmp";
    FILE* f = std::fopen(tmp.c_str(), "wb");
    if (!f) return fail(MANS_SEARCH_FAILED, std::string("IVF-PQ save: cannot open ") + tmp);
    int rc = write_all(f, &h, sizeof(h));
    if (rc == MANS_OK) rc = write_all(f, coarse.data(), coarse.size() * sizeof(float));
    if (rc == MANS_OK) rc = write_all(f, books.data(), books.size() * sizeof(float));
    if (rc == MANS_OK) rc = write_all(f, pq->h_offsets.data(), (size_t)(nlist + 1) * sizeof(int64_t));
    if (rc == MANS_OK) rc = write_all(f, ids.data(), ids.size() * sizeof(uint32_t));
    if (rc == MANS_OK) rc = write_all(f, codes.data(), codes.size());
    if (rc == MANS_OK) rc = write_all(f, assign.data(), assign.size() * sizeof(int32_t));
    if (std::fclose(f) != 0 && rc == MANS_OK) rc = fail(MANS_SEARCH_FAILED, "IVF-PQ save: close failed");
    if (rc == MANS_OK && std::rename(tmp.c_str(), path) != 0)
        rc = fail(MANS_SEARCH_FAILED, std::string("IVF-PQ save: cannot rename onto ") + path);
    if (rc != MANS_OK) std::remove(tmp.c_str());
    return rc;
}

int mans_ivfpq_load(mans_ctx* ctx, const mans_corpus* corpus, const char* path, mans_ivfpq** out) {
    if (out) *out = nullptr;
    if (!ctx || !path || !out) return fail(MANS_SEARCH_FAILED, "mans_ivfpq_load: NULL argument");
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(MANS_CORRUPT_FILE, std::string("cannot open ") + path);
    struct stat st_;
    if (fstat(fd, &st_) != 0) {
        close(fd);
        return fail(MANS_CORRUPT_FILE, "cannot stat the file");
    }
    const uint64_t len = (uint64_t)st_.st_size;
    if (len < kIvpbHeader) {
        close(fd);
        return fail(MANS_CORRUPT_FILE, "Unexpected EOF");
    }
    void* map = mmap(nullptr, (size_t)len, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return fail(MANS_CORRUPT_FILE, "cannot map the file");
    struct Unmap {
        void* p;
        size_t len;
        ~Unmap() { munmap(p, len); }
    } unmap{map, (size_t)len};
    const uint8_t* base = (const uint8_t*)map;
    IvpbHeader h;
    std::memcpy(&h, base, sizeof(h));
    if (std::memcmp(h.magic, "IVPB", 4) != 0) return fail(MANS_CORRUPT_FILE, "Invalid file magic");
    if (h.version != kIvpbVersion)
        return fail(MANS_CORRUPT_FILE, "Unsupported IVF-PQ file version " + std::to_string(h.version));
    if (h.metric > 2) return fail(MANS_CORRUPT_FILE, "Unsupported metric code");
    if (h.dim == 0 || h.m == 0 || h.nlist == 0 || h.dsub == 0 || (uint64_t)h.m * h.dsub != h.dim)
        return fail(MANS_CORRUPT_FILE, "Inconsistent dimension, subspaces or list count");
    if (h.m % 4 != 0 || h.m > 64)
        return fail(MANS_CORRUPT_FILE, "IVF-PQ: m must be a multiple of 4, at most 64");
    if (h.n > 0xFFFFFFFEull) return fail(MANS_CORRUPT_FILE, "More rows than the 32-bit id space");
    uint64_t off[7];
    if (!ivpb_layout(h.n, h.nlist, h.dim, h.m, h.dsub, off))
        return fail(MANS_CORRUPT_FILE, "Integer overflow while computing serialized sizes");
    if (off[6] != len) return fail(MANS_CORRUPT_FILE, "File size does not match the header");
    const int64_t n = (int64_t)h.n, nlist = (int64_t)h.nlist, dim = h.dim, m = h.m;
    std::vector<int64_t> offsets((size_t)nlist + 1);
    std::memcpy(offsets.data(), base + off[2], offsets.size() * sizeof(int64_t));
    if (offsets[0] != 0 || offsets[nlist] != n) return fail(MANS_CORRUPT_FILE, "List offsets are corrupt");
    for (int64_t c = 0; c < nlist; ++c)
        if (offsets[c + 1] < offsets[c]) return fail(MANS_CORRUPT_FILE, "List offsets are corrupt");
    // Every row once, in the list its assignment names.
    const uint32_t* ids = (const uint32_t*)(base + off[3]);
    const int32_t* assign = (const int32_t*)(base + off[5]);
    std::vector<uint8_t> seen((size_t)n, 0);
    for (int64_t c = 0; c < nlist; ++c)
        for (int64_t pos = offsets[c]; pos < offsets[c + 1]; ++pos) {
            const uint32_t id = ids[pos];
            if ((int64_t)id >= n || seen[id] || assign[id] != (int32_t)c)
                return fail(MANS_CORRUPT_FILE, "List ids and assignments disagree");
            seen[id] = 1;
        }
    if (corpus && (corpus->n != n || corpus->dim != dim))
        return fail(MANS_DIMENSION_MISMATCH, "the rerank corpus does not match the index's rows");
    DeviceGuard dg(ctx->device);
    auto* pq = new mans_ivfpq();
    pq->ctx = ctx;
    pq->corpus = corpus;
    pq->n = n;
    pq->dim = dim;
    pq->nlist = nlist;
    pq->m = m;
    pq->dsub = h.dsub;
    pq->metric = h.metric;
    pq->h_offsets = offsets;
    const size_t nn = (size_t)(n ? n : 1);
    hipError_t e = pq->coarse.ensure((size_t)nlist * dim * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = pq->coarse_t.ensure((size_t)nlist * dim * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = pq->books.ensure((size_t)m * 256 * h.dsub * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = pq->offsets.ensure((size_t)(nlist + 1) * sizeof(int64_t), ctx->fail_alloc);
    if (e == hipSuccess) e = pq->list_ids.ensure(nn * sizeof(uint32_t), ctx->fail_alloc);
    if (e == hipSuccess) e = pq->codes.ensure(nn * m, ctx->fail_alloc);
    if (e == hipSuccess) e = pq->assign.ensure(nn * sizeof(int32_t), ctx->fail_alloc);
    const struct {
        void* dst;
        uint64_t off, bytes;
    } parts[] = {{pq->coarse.p, off[0], off[1] - off[0]}, {pq->books.p, off[1], off[2] - off[1]},
                 {pq->offsets.p, off[2], off[3] - off[2]}, {pq->list_ids.p, off[3], off[4] - off[3]},
                 {pq->codes.p, off[4], off[5] - off[4]},   {pq->assign.p, off[5], off[6] - off[5]}};
    for (const auto& pt : parts)
        if (e == hipSuccess && pt.bytes > 0)
            e = hipMemcpy(pt.dst, base + pt.off, (size_t)pt.bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        const int64_t cells = nlist * dim;
        hipLaunchKernelGGL(transpose_kernel, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, 0,
                           (const float*)pq->coarse.p, nlist, (int)dim, (float*)pq->coarse_t.p);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        delete pq;
        return hip_fail(e, "IVF-PQ load");
    }
    *out = pq;
    return MANS_OK;
}

}  // extern "C"
