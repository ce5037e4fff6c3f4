// IVF-flat on gfx950: partition build (IVFFlatSearch.swift:517-703),
// probe selection and probed-list scan (IVFFlatSearch.swift:115-311), and
// the Lloyd k-means that makes its centroids.
//
// Assignment and probe selection are exact nearest-centroid searches: the
// centroids form a corpus and the rows (or queries) are the queries of the
// flat scan, whose results are the exact (distance, index) order of the
// host formulas -- the argmin with ties to the lower list of
// IVFFlatSearch.swift:673-700 and smallestIndices of :314-382.  The lists
// are CSR in row order (a stable counting sort of the assignment) with the
// rows packed list by list.  The scan of a query's probed lists is the
// streaming scan over its segments of the packed rows: lower-bound keys,
// WaveTopK, the cross-block merge, the exact rescore in the dots.c order
// with the list ids as the reported ids, and the proof, re-run with a
// larger candidate count where it fails.
#include <algorithm>
#include <cstring>
#include <vector>

#include "mans_hip.h"
#include "mans_runtime.hpp"
#include "mans_scan.hpp"

struct mans_ivf {
    mans_ctx* ctx = nullptr;
    int64_t n = 0, dim = 0, nlist = 0;
    uint32_t metric = 0;
    mans_corpus* cent = nullptr;  // centroids with their norms
    mans::DevBuf offsets;         // int64 [nlist + 1]
    mans::DevBuf list_ids;        // uint32 [n]
    mans::DevBuf packed;          // f32 [n][dim], rows in list order
    mans::DevBuf packed_norms;    // f32 [n]
    std::vector<int64_t> h_offsets;
    ~mans_ivf() {
        if (cent) mans_corpus_release(cent);
    }
};

namespace mans {

// A corpus whose rows are already in device memory (copied).
static int corpus_from_device(mans_ctx* ctx, const float* d_rows, int64_t n, int64_t dim,
                              hipStream_t st, mans_corpus** out) {
    auto* c = new mans_corpus();
    c->ctx = ctx;
    c->n = n;
    c->dim = dim;
    const size_t bytes = (size_t)n * dim * sizeof(float);
    hipError_t e = c->rows.ensure(bytes ? bytes : 4, ctx->fail_alloc);
    if (e == hipSuccess) e = c->norms.ensure((size_t)(n ? n : 1) * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess && n > 0) e = hipMemcpyAsync(c->rows.p, d_rows, bytes, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess && n > 0)
        e = launch_row_norms((const float*)c->rows.p, n, (int)dim, (float*)c->norms.p, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        delete c;
        return hip_fail(e, "centroid upload");
    }
    *out = c;
    return MANS_OK;
}

// dst[i] = src[idx[i]] for rows of `width` floats; norms likewise when given.
__global__ void ivf_gather_rows(const float* __restrict__ src, const float* __restrict__ src_norms,
                                const uint32_t* __restrict__ idx, int64_t count, int width,
                                float* __restrict__ dst, float* __restrict__ dst_norms) {
    const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= count) return;
    const int lane = threadIdx.x & 63;
    const int64_t s = idx[i];
    for (int j = lane; j < width; j += 64) dst[i * width + j] = src[s * width + j];
    if (lane == 0 && dst_norms) dst_norms[i] = src_norms[s];
}

// Nearest centroid of every row (top-1 of the exact flat scan over the
// centroids), then CSR lists in row order.  assign_h (n) receives the
// assignment on the host.
static int ivf_assign_and_lists(mans_ctx* ctx, mans_corpus* cent, const float* d_rows, int64_t n,
                                uint32_t metric, Slot* slot, std::vector<int32_t>* assign_h,
                                std::vector<int64_t>* offsets, std::vector<uint32_t>* list_ids) {
    hipStream_t st = slot->stream;
    DevBuf d_dist, d_ids;
    hipError_t e = d_dist.ensure((size_t)n * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = d_ids.ensure((size_t)n * sizeof(uint32_t), ctx->fail_alloc);
    if (e != hipSuccess) return hip_fail(e, "assignment workspace");
    int rc = flat_search_run(ctx, cent, d_rows, n, 1, metric, (float*)d_dist.p, (uint32_t*)d_ids.p,
                             st, slot, nullptr, nullptr);
    if (rc != MANS_OK) return rc;
    assign_h->resize((size_t)n);
    e = hipMemcpyAsync(assign_h->data(), d_ids.p, (size_t)n * sizeof(uint32_t), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "assignment download");
    const int64_t nlist = cent->n;
    offsets->assign((size_t)nlist + 1, 0);
    for (int64_t r = 0; r < n; ++r) {
        const int32_t a = (*assign_h)[r];
        if (a < 0 || a >= nlist) return fail(MANS_EXECUTION_FAILED, "assignment out of range");
        (*offsets)[a + 1]++;
    }
    for (int64_t c = 0; c < nlist; ++c) (*offsets)[c + 1] += (*offsets)[c];
    list_ids->resize((size_t)n);
    std::vector<int64_t> cur(offsets->begin(), offsets->end() - 1);
    for (int64_t r = 0; r < n; ++r) (*list_ids)[cur[(*assign_h)[r]]++] = (uint32_t)r;
    return MANS_OK;
}

// fp64 means in ascending row order (the oracle's Lloyd step): one thread
// per (centroid, dimension); empty lists keep their centroid.
__global__ void kmeans_update(const float* __restrict__ rows, const int64_t* __restrict__ offsets,
                              const uint32_t* __restrict__ list_ids, int64_t k, int dim,
                              float* __restrict__ centroids) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= k * dim) return;
    const int64_t c = t / dim;
    const int d = (int)(t % dim);
    const int64_t a = offsets[c], b = offsets[c + 1];
    if (a == b) return;
    double sum = 0.0;
    for (int64_t i = a; i < b; ++i) sum += (double)rows[(int64_t)list_ids[i] * dim + d];
    centroids[t] = (float)(sum / (double)(b - a));
}

struct IvfArgs {
    const float* packed;
    const float* packed_norms;
    const uint32_t* list_ids;
    const int64_t* seg;        // [nq_launch][np][2]: packed start, concatenated start
    const int64_t* total;      // [nq_launch] candidate rows
    const int32_t* item_off;   // [nq_launch + 1] first work item of each query
    const int32_t* item_q;     // [items] launch index of each work item
    int np;
    int64_t nq;                // queries in the launch
    int64_t chunk;             // rows per work item (multiple of 32)
};

// One wave per query of the launch: its probed lists' packed starts and
// concatenated starts, its candidate count and its number of work items.
__global__ __launch_bounds__(256) void ivf_plan(const uint32_t* __restrict__ probes, int np,
                                                const uint32_t* __restrict__ qidx, int64_t nq,
                                                const int64_t* __restrict__ offsets, int64_t chunk,
                                                int64_t* __restrict__ seg, int64_t* __restrict__ total,
                                                int32_t* __restrict__ nitems) {
    const int lane = threadIdx.x & 63;
    const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= nq) return;  // the whole wave leaves together
    const uint32_t q = qidx ? qidx[i] : (uint32_t)i;
    int64_t carry = 0;
    for (int base = 0; base < np; base += 64) {
        const int p = base + lane;
        int64_t start = 0, len = 0;
        if (p < np) {
            const uint32_t list = probes[(int64_t)q * np + p];
            start = offsets[list];
            len = offsets[list + 1] - start;
        }
        int64_t incl = len;  // inclusive scan over the wave
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int64_t t = __shfl_up(incl, o);
            if (lane >= o) incl += t;
        }
        if (p < np) {
            seg[(i * np + p) * 2 + 0] = start;
            seg[(i * np + p) * 2 + 1] = carry + incl - len;
        }
        carry += __shfl(incl, 63);
    }
    if (lane == 0) {
        total[i] = carry;
        nitems[i] = carry > 0 ? (int32_t)((carry + chunk - 1) / chunk) : 1;
    }
}

// One block: exclusive scan of the per-query item counts, then the item ->
// query map.  item_off[nq] holds the number of items.
__global__ __launch_bounds__(1024) void ivf_items(const int32_t* __restrict__ nitems, int64_t nq,
                                                   int32_t* __restrict__ item_off,
                                                   int32_t* __restrict__ item_q) {
    __shared__ int32_t part[1024];
    const int tid = threadIdx.x;
    const int64_t per = (nq + 1023) / 1024;
    const int64_t a = tid * per, b = a + per < nq ? a + per : nq;
    int32_t s = 0;
    for (int64_t i = a; i < b; ++i) s += nitems[i];
    part[tid] = s;
    __syncthreads();
    if (tid == 0) {
        int32_t run = 0;
        for (int t = 0; t < 1024; ++t) {
            const int32_t v = part[t];
            part[t] = run;
            run += v;
        }
        item_off[nq] = run;
    }
    __syncthreads();
    int32_t run = part[tid];
    for (int64_t i = a; i < b; ++i) {
        item_off[i] = run;
        for (int32_t j = 0; j < nitems[i]; ++j) item_q[run + j] = (int32_t)i;
        run += nitems[i];
    }
}

// 1-D grid over work items (an upper bound; blocks past the last item leave
// at once); block 256; dynamic LDS: 4 * cap slots.  Item j of a query scans
// rows [j chunk, (j + 1) chunk) of the concatenation of its probed lists,
// so every block has the same work whatever the list sizes.  The last of a
// query's items to arrive merges their lists and rescores.  EXACT: keys are
// the exact distances (terminal round).
template <int NCH, bool EXACT>
__global__ __launch_bounds__(256) void ivf_scan(
    IvfArgs ia, int dim, const float* __restrict__ queries, const uint32_t* __restrict__ qidx,
    int metric, BoundCoef bc, int kc, int cap, FlatArgs fa) {
    extern __shared__ uint64_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = lane >> 4, lr = lane & 15;
    const int item = blockIdx.x;
    if (item >= ia.item_off[ia.nq]) return;  // past the last work item
    const int i = ia.item_q[item];
    const uint32_t q = qidx ? qidx[i] : (uint32_t)i;
    const int first = ia.item_off[i];
    const int nb = ia.item_off[i + 1] - first;
    const int j = item - first;
    const int dim4 = dim >> 2;
    const float* qp = queries + (int64_t)q * dim;
    const int64_t* seg = ia.seg + (int64_t)i * ia.np * 2;
    const int64_t total = ia.total[i];

    f4v qv[NCH];
    float qsq = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = lr + 16 * c;
        qv[c] = idx < dim4 ? *reinterpret_cast<const f4v*>(qp + 4 * idx) : f4v{0.f, 0.f, 0.f, 0.f};
        qsq = fmaf(qv[c].x, qv[c].x, qsq);
        qsq = fmaf(qv[c].y, qv[c].y, qsq);
        qsq = fmaf(qv[c].z, qv[c].z, qsq);
        qsq = fmaf(qv[c].w, qv[c].w, qsq);
    }
    const float qn = EXACT ? (metric == kMetricIP ? 0.0f : chain_dot<NCH>(qv, qv, dim4)) : row16_sum(qsq);

    const int64_t lo = (int64_t)j * ia.chunk;
    const int64_t hi = lo + ia.chunk < total ? lo + ia.chunk : total;
    WaveTopK sel;
    sel.init(lds + wave * cap, cap, kc);
    for (int p = 0; p < ia.np; ++p) {
        const int64_t pre = seg[2 * p + 1];
        if (pre >= hi) break;
        const int64_t len = (p + 1 < ia.np ? seg[2 * p + 3] : total) - pre;
        const int64_t a = lo > pre ? lo - pre : 0;
        const int64_t b = hi - pre < len ? hi - pre : len;
        if (a >= b) continue;
        const int64_t start = seg[2 * p] + a, end = seg[2 * p] + b;  // packed rows
        if constexpr (!EXACT) {
            // The streaming scan's step: the next 16 rows' loads are in
            // flight while the current ones are reduced and offered.
            const int slot = wave * 4 + grp;
            f4v ra[1][NCH], rb[1][NCH];
            float va[1], vb[1];
            scan_load<NCH, false, 1>(ia.packed, ia.packed_norms, dim, dim4, start, end, slot, lr, ra, va);
            for (int64_t base = start; base < end; base += 32) {
                scan_load<NCH, false, 1>(ia.packed, ia.packed_norms, dim, dim4, base + 16, end, slot, lr, rb, vb);
                scan_offer<NCH, 1>(ra, va, qv, qn, metric, bc, base, end, slot, lr, sel);
                scan_load<NCH, false, 1>(ia.packed, ia.packed_norms, dim, dim4, base + 32, end, slot, lr, ra, va);
                scan_offer<NCH, 1>(rb, vb, qv, qn, metric, bc, base + 16, end, slot, lr, sel);
            }
            continue;
        }
        for (int64_t base = start; base < end; base += 32) {
            const int64_t r0 = base + wave * 4 + grp;
            const int64_t r1 = r0 + 16;
            const bool v0 = r0 < end, v1 = r1 < end;
            const int64_t c0 = v0 ? r0 : end - 1, c1 = v1 ? r1 : end - 1;
            const float* p0 = ia.packed + c0 * dim;
            const float* p1 = ia.packed + c1 * dim;
            const float vn0 = ia.packed_norms[c0], vn1 = ia.packed_norms[c1];
            f4v x[NCH], y[NCH];
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int idx = lr + 16 * c;
                const bool in = idx < dim4;
                const int ci = in ? idx : dim4 - 1;
                const f4v tx = load_stream(p0 + 4 * ci), ty = load_stream(p1 + 4 * ci);
                x[c] = in ? tx : f4v{0.f, 0.f, 0.f, 0.f};
                y[c] = in ? ty : f4v{0.f, 0.f, 0.f, 0.f};
            }
            float k0, k1;
            if (EXACT) {
                k0 = host_distance(chain_dot<NCH>(x, qv, dim4), qn, vn0, metric);
                k1 = host_distance(chain_dot<NCH>(y, qv, dim4), qn, vn1, metric);
            } else {
                float f0 = 0.0f, f1 = 0.0f;
#pragma unroll
                for (int c = 0; c < NCH; ++c) {
                    f0 = fmaf(x[c].x, qv[c].x, f0);
                    f0 = fmaf(x[c].y, qv[c].y, f0);
                    f0 = fmaf(x[c].z, qv[c].z, f0);
                    f0 = fmaf(x[c].w, qv[c].w, f0);
                    f1 = fmaf(y[c].x, qv[c].x, f1);
                    f1 = fmaf(y[c].y, qv[c].y, f1);
                    f1 = fmaf(y[c].z, qv[c].z, f1);
                    f1 = fmaf(y[c].w, qv[c].w, f1);
                }
                k0 = lower_key(row16_sum(f0), qn, vn0, metric, bc);
                k1 = lower_key(row16_sum(f1), qn, vn1, metric, bc);
            }
            sel.offer(lr == 0 && v0, k0, (uint32_t)r0);
            sel.offer(lr == 0 && v1, k1, (uint32_t)r1);
        }
    }
    sel.finish();
    // Item lists, then the last of the query's items merges them.
    block_fold(sel, lds, cap);
    if (tid < 64)
        for (int s = tid; s < kc; s += 64)
            store_shared_slot(&fa.cand[(int64_t)item * kc + s], s < sel.count ? sel.buf[s] : kEmptySlot);
    uint32_t* cnt = fa.counters + i;
    if (!block_arrive_last(cnt, (uint32_t)nb)) return;
    if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    block_select_lists(fa.cand + (int64_t)first * kc, (int64_t)nb * kc, lds, cap, kc, sel);
    final_rescore_f4<NCH>(qv, ia.packed, ia.packed_norms, total, dim, metric, q, lds, kc, fa,
                          kFltMax, kProofFlat, ia.list_ids, i);
}

template <int NCH, bool EXACT>
static void launch_ivf_scan(int64_t max_items, int cap, int kc, const IvfArgs& ia, int dim,
                            const float* queries, const uint32_t* qidx, int metric,
                            const BoundCoef& bc, const FlatArgs& fa, hipStream_t s) {
    size_t shmem = sizeof(uint64_t) * 4 * (size_t)cap;
    hipLaunchKernelGGL((ivf_scan<NCH, EXACT>), dim3((unsigned)max_items), dim3(256), shmem, s, ia,
                       dim, queries, qidx, metric, bc, kc, cap, fa);
}

template <bool EXACT>
static hipError_t launch_ivf_nch(int nch, int64_t max_items, int cap, int kc, const IvfArgs& ia,
                                 int dim, const float* queries, const uint32_t* qidx, int metric,
                                 const BoundCoef& bc, const FlatArgs& fa, hipStream_t s) {
    switch (nch) {
    case 1: launch_ivf_scan<1, EXACT>(max_items, cap, kc, ia, dim, queries, qidx, metric, bc, fa, s); break;
    case 2: launch_ivf_scan<2, EXACT>(max_items, cap, kc, ia, dim, queries, qidx, metric, bc, fa, s); break;
    case 3: launch_ivf_scan<3, EXACT>(max_items, cap, kc, ia, dim, queries, qidx, metric, bc, fa, s); break;
    case 4: launch_ivf_scan<4, EXACT>(max_items, cap, kc, ia, dim, queries, qidx, metric, bc, fa, s); break;
    case 6: launch_ivf_scan<6, EXACT>(max_items, cap, kc, ia, dim, queries, qidx, metric, bc, fa, s); break;
    case 8: launch_ivf_scan<8, EXACT>(max_items, cap, kc, ia, dim, queries, qidx, metric, bc, fa, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

constexpr int kIvfMaxDim = 512;

// Queries and outputs in device memory.  h_probes (nullable, host): nq x np
// ascending list ids.
static int ivf_search_run(mans_ctx* ctx, const mans_ivf* ivf, const float* d_q, int64_t nq,
                          int64_t k, int64_t nprobe, float* d_dist, uint32_t* d_ids,
                          int32_t* h_probes, hipStream_t st, Slot* slot) {
    if (nq <= 0 || k <= 0) return MANS_OK;
    if (ctx->fail_launch) return fail(MANS_EXECUTION_FAILED, "injected launch failure");
    if (k > MANS_MAX_TOP_K) return fail(MANS_SEARCH_FAILED, "IVF scan: k above 256");
    if (nq > 16384) return fail(MANS_SEARCH_FAILED, "IVF scan: at most 16384 queries per call");
    if ((reinterpret_cast<uintptr_t>(d_q) & 15u) != 0)
        return fail(MANS_SEARCH_FAILED, "IVF scan: queries must be 16-byte aligned");
    const int dim = (int)ivf->dim;
    const int nch = flat_nch_for_dim(dim);
    if (nch == 0 || dim > kIvfMaxDim)
        return fail(MANS_PIPELINE_UNAVAILABLE, "IVF scan: dim must be a multiple of 4, at most 512");
    const int np = (int)std::max<int64_t>(1, std::min<int64_t>(nprobe, ivf->nlist));
    if (np > MANS_MAX_TOP_K) return fail(MANS_SEARCH_FAILED, "IVF scan: nprobe above 256");
    const uint32_t metric = ivf->metric;

    // Probes: the np nearest centroids by (distance, index).  The scan does
    // not depend on their order; the reported probe lists are ascending.
    hipError_t e = slot->aux0.ensure((size_t)nq * np * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = slot->aux1.ensure((size_t)nq * np * sizeof(uint32_t), ctx->fail_alloc);
    if (e != hipSuccess) return hip_fail(e, "IVF probe workspace");
    int rc = flat_search_run(ctx, ivf->cent, d_q, nq, np, metric, (float*)slot->aux0.p,
                             (uint32_t*)slot->aux1.p, st, slot, nullptr, nullptr);
    if (rc != MANS_OK) return rc;
    const uint32_t* d_probes = (const uint32_t*)slot->aux1.p;
    if (h_probes) {
        std::vector<uint32_t> pr((size_t)nq * np);
        e = hipMemcpyAsync(pr.data(), d_probes, pr.size() * sizeof(uint32_t), hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "IVF probes download");
        for (int64_t i = 0; i < nq; ++i) {
            std::sort(pr.begin() + i * np, pr.begin() + (i + 1) * np);
            for (int p = 0; p < np; ++p) h_probes[i * np + p] = (int32_t)pr[i * np + p];
        }
    }

    // Work items: rows per item about 512 items' worth of the batch's
    // average work, at least 128 (fewer, longer items keep the per-item
    // list, merge and rescore costs small); the launch covers the largest
    // queries.
    const int64_t avg_rows = std::max<int64_t>(1, ivf->n * np / std::max<int64_t>(1, ivf->nlist));
    int64_t max_rows = 0;
    {
        std::vector<int64_t> sizes((size_t)ivf->nlist);
        for (int64_t c = 0; c < ivf->nlist; ++c) sizes[c] = ivf->h_offsets[c + 1] - ivf->h_offsets[c];
        std::nth_element(sizes.begin(), sizes.begin() + (np - 1), sizes.end(), std::greater<int64_t>());
        for (int p = 0; p < np; ++p) max_rows += sizes[p];
    }
    static const int64_t target_items = [] {
        const char* ev = std::getenv("MANS_IVF_BLOCKS");
        return ev ? std::max<int64_t>(1, std::atoll(ev)) : (int64_t)512;
    }();

    const int keff = (int)std::min<int64_t>(std::min<int64_t>(k, MANS_MAX_TOP_K), ivf->n);
    int kc = 32;
    while (kc < 2 * keff) kc <<= 1;
    bool exact = false;
    std::vector<uint32_t> pending;
    int64_t npend = nq;
    ctx->time_begin(slot, st);
    for (;;) {
        if (exact) {
            kc = 32;
            while (kc < keff) kc <<= 1;
        }
        int64_t chunk = (avg_rows * npend + target_items - 1) / target_items;
        chunk = std::max<int64_t>(128, (chunk + 31) / 32 * 32);
        const int64_t items_bound = npend * std::max<int64_t>(1, (max_rows + chunk - 1) / chunk);
        const uint32_t* d_qidx = nullptr;
        if (!pending.empty()) {
            e = slot->qidx.ensure(pending.size() * sizeof(uint32_t), ctx->fail_alloc);
            if (e == hipSuccess)
                e = hipMemcpyAsync(slot->qidx.p, pending.data(), pending.size() * sizeof(uint32_t),
                                   hipMemcpyHostToDevice, st);
            d_qidx = (const uint32_t*)slot->qidx.p;
        }
        // aux2: seg [npend][np][2] int64, total [npend] int64;
        // aux3: nitems [npend], item_off [npend + 1], item_q [items_bound] int32.
        const size_t seg_bytes = (size_t)npend * np * 2 * sizeof(int64_t);
        if (e == hipSuccess) e = slot->aux2.ensure(seg_bytes + (size_t)npend * sizeof(int64_t), ctx->fail_alloc);
        if (e == hipSuccess)
            e = slot->aux3.ensure((size_t)(2 * npend + 1 + items_bound) * sizeof(int32_t), ctx->fail_alloc);
        FlatPlan p = plan_flat(1, npend, kc, 0);
        p.nblk = (int)std::min<int64_t>(items_bound, INT32_MAX);  // cand: items_bound lists
        p.ngroups = 0;
        FlatBuffers fb;
        if (e == hipSuccess) e = prepare_flat_buffers(ctx, slot, p, 1, st, &fb);
        if (e == hipSuccess) e = slot->status.ensure((size_t)npend, ctx->fail_alloc);
        if (e == hipSuccess && slot->counters.bytes < (size_t)npend * sizeof(uint32_t)) {
            // Counters grow zeroed (the kernels leave them at zero).
            e = slot->counters.ensure((size_t)npend * sizeof(uint32_t), ctx->fail_alloc);
            if (e == hipSuccess) e = hipMemsetAsync(slot->counters.p, 0, slot->counters.bytes, st);
        }
        if (e == hipSuccess) e = slot->status_h.ensure((size_t)npend);
        if (e != hipSuccess) return hip_fail(e, "IVF scan workspace");
        int64_t* d_seg = (int64_t*)slot->aux2.p;
        int64_t* d_total = (int64_t*)((char*)slot->aux2.p + seg_bytes);
        int32_t* d_nitems = (int32_t*)slot->aux3.p;
        int32_t* d_item_off = d_nitems + npend;
        int32_t* d_item_q = d_item_off + npend + 1;
        hipLaunchKernelGGL(ivf_plan, dim3((unsigned)((npend + 3) / 4)), dim3(256), 0, st, d_probes, np,
                           d_qidx, npend, (const int64_t*)ivf->offsets.p, chunk, d_seg, d_total, d_nitems);
        hipLaunchKernelGGL(ivf_items, dim3(1), dim3(1024), 0, st, (const int32_t*)d_nitems, npend,
                           d_item_off, d_item_q);
        e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(e, "IVF plan");

        IvfArgs ia;
        ia.packed = (const float*)ivf->packed.p;
        ia.packed_norms = (const float*)ivf->packed_norms.p;
        ia.list_ids = (const uint32_t*)ivf->list_ids.p;
        ia.seg = d_seg;
        ia.total = d_total;
        ia.item_off = d_item_off;
        ia.item_q = d_item_q;
        ia.np = np;
        ia.nq = npend;
        ia.chunk = chunk;
        FlatArgs fa = {};
        fa.cand = (uint64_t*)slot->cand.p;
        fa.counters = (uint32_t*)slot->counters.p;
        fa.out_dist = d_dist;
        fa.out_ids = d_ids;
        fa.status = (uint8_t*)slot->status.p;
        fa.k = keff;
        fa.k_stride = (int)k;
        const BoundCoef bc = make_bounds(dim);
        const int cap = flat_cap_for(kc);
        e = exact ? launch_ivf_nch<true>(nch, items_bound, cap, kc, ia, dim, d_q, d_qidx, (int)metric, bc, fa, st)
                  : launch_ivf_nch<false>(nch, items_bound, cap, kc, ia, dim, d_q, d_qidx, (int)metric, bc, fa, st);
        if (e == hipSuccess)
            e = hipMemcpyAsync(slot->status_h.p, slot->status.p, (size_t)npend, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) {
            slot->counters_dirty = true;
            return hip_fail(e, "IVF scan");
        }
        const uint8_t* sh = (const uint8_t*)slot->status_h.p;
        std::vector<uint32_t> next;
        for (int64_t i = 0; i < npend; ++i)
            if (sh[i]) next.push_back(pending.empty() ? (uint32_t)i : pending[i]);
        if (next.empty()) break;
        if (exact) return fail(MANS_SEARCH_FAILED, "IVF exact round failed its own proof");
        pending.swap(next);
        npend = (int64_t)pending.size();
        kc *= 4;
        if (kc > 1024) exact = true;
        ctx->proof_retries += npend;
    }
    ctx->time_end(slot, st, "ivf_scan");
    return MANS_OK;
}

static int ivf_build_from_centroids(mans_ctx* ctx, const mans_corpus* corpus, mans_corpus* cent,
                                    uint32_t metric, mans_ivf** out) {
    SlotLease lease(ctx);
    if (!lease.slot) {
        mans_corpus_release(cent);
        return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    }
    auto* ivf = new mans_ivf();
    ivf->ctx = ctx;
    ivf->n = corpus->n;
    ivf->dim = corpus->dim;
    ivf->nlist = cent->n;
    ivf->metric = metric;
    ivf->cent = cent;
    std::vector<int32_t> assign;
    std::vector<uint32_t> list_ids;
    int rc = ivf_assign_and_lists(ctx, cent, (const float*)corpus->rows.p, corpus->n, metric,
                                  lease.slot, &assign, &ivf->h_offsets, &list_ids);
    if (rc != MANS_OK) {
        delete ivf;
        return rc;
    }
    const int64_t n = corpus->n, dim = corpus->dim;
    hipStream_t st = lease.slot->stream;
    hipError_t e = ivf->offsets.ensure((ivf->nlist + 1) * sizeof(int64_t), ctx->fail_alloc);
    if (e == hipSuccess) e = ivf->list_ids.ensure((size_t)(n ? n : 1) * sizeof(uint32_t), ctx->fail_alloc);
    if (e == hipSuccess) e = ivf->packed.ensure((size_t)(n ? n : 1) * dim * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = ivf->packed_norms.ensure((size_t)(n ? n : 1) * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess)
        e = hipMemcpyAsync(ivf->offsets.p, ivf->h_offsets.data(), (ivf->nlist + 1) * sizeof(int64_t),
                           hipMemcpyHostToDevice, st);
    if (e == hipSuccess && n > 0)
        e = hipMemcpyAsync(ivf->list_ids.p, list_ids.data(), n * sizeof(uint32_t), hipMemcpyHostToDevice, st);
    if (e == hipSuccess && n > 0) {
        hipLaunchKernelGGL(ivf_gather_rows, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st,
                           (const float*)corpus->rows.p, (const float*)corpus->norms.p,
                           (const uint32_t*)ivf->list_ids.p, n, (int)dim, (float*)ivf->packed.p,
                           (float*)ivf->packed_norms.p);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        delete ivf;
        return hip_fail(e, "IVF build");
    }
    *out = ivf;
    return MANS_OK;
}

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
//    time.  Work items of equal row counts cover each query's probed lists;
//    the last item of a query merges, orders, maps positions to ids and
//    (with rerank_k > 0) rescores exactly.
// ---------------------------------------------------------------------------

__device__ __forceinline__ float simd_distance(const float* a, const float* b, int d, int metric) {
    if (metric == kMetricL2) {
        float s = 0.0f;
        for (int i = 0; i < d; ++i) {
            const float t = a[i] - b[i];
            s += t * t;
        }
        return s;
    }
    if (metric == kMetricIP) {
        float dot = 0.0f;
        for (int i = 0; i < d; ++i) dot += a[i] * b[i];
        return -dot;
    }
    if (d <= 0) return 1.0f;
    float dot = 0.0f, na = 0.0f, nb = 0.0f;
    for (int i = 0; i < d; ++i) dot += a[i] * b[i];
    for (int i = 0; i < d; ++i) na += a[i] * a[i];
    for (int i = 0; i < d; ++i) nb += b[i] * b[i];
    const float denom = sqrtf(na) * sqrtf(nb);
    return denom < 1e-10f ? 1.0f : 1.0f - dot / denom;
}

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

// BoundedSortedList(cap) replayed by one thread over `cnt` (score, tag)
// entries in arrival order (BoundedSelection.swift:158-214): a newcomer goes
// in front of equal scores; a full list takes it only if it beats the worst.
__device__ inline int sorted_list_replay(const float* in_score, const uint32_t* in_tag, int cnt,
                                         int cap, float* ls, uint32_t* lt) {
    int count = 0;
    for (int i = 0; i < cnt; ++i) {
        const float sc = in_score[i];
        if (count >= cap && !(sc < ls[count - 1])) continue;
        int lo = 0, hi = count;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (ls[mid] < sc) lo = mid + 1;
            else hi = mid;
        }
        int last = count < cap ? count : cap - 1;
        for (int j = last; j > lo; --j) {
            ls[j] = ls[j - 1];
            lt[j] = lt[j - 1];
        }
        ls[lo] = sc;
        lt[lo] = in_tag[i];
        if (count < cap) ++count;
    }
    return count;
}

// simd_distance with b read at stride bstride (centroids stored
// dimension-major, so consecutive lanes read consecutive floats); the same
// operations in the same order.
__device__ __forceinline__ float simd_distance_strided(const float* a, const float* b, int d,
                                                       int64_t bstride, int metric) {
    if (metric == kMetricL2) {
        float s = 0.0f;
        for (int i = 0; i < d; ++i) {
            const float t = a[i] - b[i * bstride];
            s += t * t;
        }
        return s;
    }
    if (metric == kMetricIP) {
        float dot = 0.0f;
        for (int i = 0; i < d; ++i) dot += a[i] * b[i * bstride];
        return -dot;
    }
    if (d <= 0) return 1.0f;
    float dot = 0.0f, na = 0.0f, nb = 0.0f;
    for (int i = 0; i < d; ++i) dot += a[i] * b[i * bstride];
    for (int i = 0; i < d; ++i) na += a[i] * a[i];
    for (int i = 0; i < d; ++i) nb += b[i * bstride] * b[i * bstride];
    const float denom = sqrtf(na) * sqrtf(nb);
    return denom < 1e-10f ? 1.0f : 1.0f - dot / denom;
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

// Probe selection, one block per query (selectClosestCentroids,
// IVFPQIndex.swift:484-512): the sequential distance to every centroid, the
// np + 64 smallest by (distance, index), then the BoundedSortedList(np)
// order over those at or below the np-th distance.  status 1: more ties at
// the boundary than the selection kept.  dynamic LDS: 4 * cap slots + dim
// floats.
__global__ __launch_bounds__(256) void pq_probes(const float* __restrict__ queries, int dim,
                                                 const float* __restrict__ coarse_t, int nlist,
                                                 int metric, int np, int kc, int cap,
                                                 uint32_t* __restrict__ probes,
                                                 uint8_t* __restrict__ status) {
    extern __shared__ uint64_t lds[];
    float* qs = reinterpret_cast<float*>(lds + 4 * cap);
    __shared__ int s_cnt, s_over;
    const int tid = threadIdx.x, wave = tid >> 6;
    const int64_t q = blockIdx.x;
    for (int d = tid; d < dim; d += blockDim.x) qs[d] = queries[q * dim + d];
    __syncthreads();
    WaveTopK sel;
    sel.init(lds + wave * cap, cap, kc);
    for (int base = 0; base < nlist; base += blockDim.x) {
        const int c = base + tid;
        const bool v = c < nlist;
        const float dist = v ? simd_distance_strided(qs, coarse_t + c, dim, nlist, metric) : 0.0f;
        sel.offer(v, dist, (uint32_t)c);
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
        status[q] = (uint8_t)s_over;
    }
}

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
    int64_t nq;                // queries in the launch
    int64_t chunk;             // rows per work item (multiple of 256)
    int np, m, dsub, dim, metric;
    int kadc, rerank;
};

// 1-D grid over work items; block 256; dynamic LDS: 4 * cap slots, then
// m * 256 + dim floats (LUT, residual).  Slots are (score, arrival index).
template <int NCH>
__global__ __launch_bounds__(256) void ivfpq_scan(PqArgs pa, const float* __restrict__ queries,
                                                  const uint32_t* __restrict__ qidx, int kc, int cap,
                                                  FlatArgs fa) {
    extern __shared__ uint64_t lds[];
    float* lut = reinterpret_cast<float*>(lds + 4 * cap);
    float* qres = lut + pa.m * 256;
    __shared__ int s_cnt, s_over, s_n;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
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
    WaveTopK sel;
    sel.init(lds + wave * cap, cap, kc);
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
        // Codes of a row as 16-byte loads when m is a multiple of 16 (rows
        // then start 16-byte aligned); the next 256 rows' codes load while
        // the current ones are scored, and the first ones while the LUT is
        // built.  The score adds the m entries in code order
        // (IVFPQIndex.swift:418-452) either way.
        const int m16 = (pa.m & 15) == 0 && pa.m <= 64 ? pa.m >> 4 : 0;
        const int64_t nrow = b - a;
        auto load_codes = [&](int64_t r, i4v (&c4)[4]) {
            const uint32_t* cw = crow + (r < nrow ? r : 0) * mw;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                c4[c] = c < m16 ? reinterpret_cast<const i4v*>(cw)[c] : i4v{0, 0, 0, 0};
        };
        i4v cur[4];
        if (m16 > 0) load_codes(tid, cur);
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
        __syncthreads();
        for (int64_t base = 0; base < nrow; base += 256) {
            const int64_t r = base + tid;
            const bool v = r < nrow;
            const uint32_t* cw = crow + (v ? r : 0) * mw;
            float score = 0.0f;
            if (m16 > 0) {
                i4v c4[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) c4[c] = cur[c];
                if (base + 256 < nrow) load_codes(r + 256, cur);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
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
                for (int w = 0; w < mw; ++w) {
                    const uint32_t word = cw[w];
                    score += lut[(4 * w + 0) * 256 + (word & 0xFF)];
                    score += lut[(4 * w + 1) * 256 + ((word >> 8) & 0xFF)];
                    score += lut[(4 * w + 2) * 256 + ((word >> 16) & 0xFF)];
                    score += lut[(4 * w + 3) * 256 + (word >> 24)];
                }
            }
            sel.offer(v, score, (uint32_t)(pre + a + r));
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
        s_n = ncand;
        s_cnt = s;
        s_over = (s == kc && (int64_t)kc < total) ? 1 : 0;
    }
    __syncthreads();
    const int s = s_cnt;
    if (s_over) {
        if (tid == 0) fa.status[i] = 1;
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
    const int nfin = s_final;
    // Arrival index -> packed position -> row id.
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

constexpr int kPqMaxM = 64;      // LUT of m x 256 floats in LDS
constexpr int kPqMaxKadc = 512;

template <int NCH>
static void launch_pq_scan(int64_t items, int cap, int kc, const PqArgs& pa, const float* queries,
                           const uint32_t* qidx, const FlatArgs& fa, hipStream_t s) {
    const size_t shmem = sizeof(uint64_t) * 4 * (size_t)cap + sizeof(float) * ((size_t)pa.m * 256 + pa.dim);
    hipLaunchKernelGGL(ivfpq_scan<NCH>, dim3((unsigned)items), dim3(256), shmem, s, pa, queries, qidx,
                       kc, cap, fa);
}

static int ivfpq_search_run(mans_ctx* ctx, const mans_ivfpq* pq, const float* d_q, int64_t nq,
                            int64_t k_adc, int64_t nprobe, int64_t rerank_k, float* d_score,
                            uint32_t* d_ids, hipStream_t st, Slot* slot) {
    if (nq <= 0 || k_adc <= 0) return MANS_OK;
    if (ctx->fail_launch) return fail(MANS_EXECUTION_FAILED, "injected launch failure");
    if (k_adc > kPqMaxKadc) return fail(MANS_SEARCH_FAILED, "IVF-PQ: k above 512");
    if (rerank_k > k_adc) return fail(MANS_SEARCH_FAILED, "IVF-PQ: rerank_k above k");
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

    // Probes (BoundedSortedList order).
    int pkc = np + 64;
    int pcap = flat_cap_for(pkc);
    hipError_t e = slot->aux1.ensure((size_t)nq * np * sizeof(uint32_t), ctx->fail_alloc);
    if (e == hipSuccess) e = slot->status.ensure((size_t)nq, ctx->fail_alloc);
    if (e == hipSuccess) e = slot->status_h.ensure((size_t)nq);
    if (e != hipSuccess) return hip_fail(e, "IVF-PQ probe workspace");
    ctx->time_begin(slot, st);
    hipLaunchKernelGGL(pq_probes, dim3((unsigned)nq), dim3(256),
                       sizeof(uint64_t) * 4 * (size_t)pcap + sizeof(float) * dim, st, d_q, dim,
                       (const float*)pq->coarse_t.p, (int)pq->nlist, (int)pq->metric, np, pkc, pcap,
                       (uint32_t*)slot->aux1.p, (uint8_t*)slot->status.p);
    e = hipGetLastError();
    if (e == hipSuccess)
        e = hipMemcpyAsync(slot->status_h.p, slot->status.p, (size_t)nq, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "IVF-PQ probes");
    for (int64_t i = 0; i < nq; ++i)
        if (((const uint8_t*)slot->status_h.p)[i])
            return fail(MANS_SEARCH_FAILED, "IVF-PQ: too many coarse distances tie at the probe boundary");
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
    int kc = (int)k_adc + 64;
    std::vector<uint32_t> pending;
    int64_t npend = nq;
    for (;;) {
        const int cap = flat_cap_for(kc);
        int64_t chunk = (avg_rows * npend + target_items - 1) / target_items;
        chunk = std::max<int64_t>(256, (chunk + 255) / 256 * 256);
        const int64_t items_bound = npend * std::max<int64_t>(1, (max_rows + chunk - 1) / chunk);
        const uint32_t* d_qidx = nullptr;
        if (!pending.empty()) {
            e = slot->qidx.ensure(pending.size() * sizeof(uint32_t), ctx->fail_alloc);
            if (e == hipSuccess)
                e = hipMemcpyAsync(slot->qidx.p, pending.data(), pending.size() * sizeof(uint32_t),
                                   hipMemcpyHostToDevice, st);
            d_qidx = (const uint32_t*)slot->qidx.p;
        }
        const size_t seg_bytes = (size_t)npend * np * 2 * sizeof(int64_t);
        if (e == hipSuccess) e = slot->aux2.ensure(seg_bytes + (size_t)npend * sizeof(int64_t), ctx->fail_alloc);
        if (e == hipSuccess)
            e = slot->aux3.ensure((size_t)(2 * npend + 1 + items_bound) * sizeof(int32_t), ctx->fail_alloc);
        if (e == hipSuccess) e = slot->cand.ensure((size_t)items_bound * kc * sizeof(uint64_t), ctx->fail_alloc);
        if (e == hipSuccess && (slot->counters.bytes < (size_t)npend * sizeof(uint32_t) || slot->counters_dirty)) {
            e = slot->counters.ensure((size_t)npend * sizeof(uint32_t), ctx->fail_alloc);
            if (e == hipSuccess) e = hipMemsetAsync(slot->counters.p, 0, slot->counters.bytes, st);
            slot->counters_dirty = false;
        }
        if (e == hipSuccess) e = slot->status_h.ensure((size_t)npend);
        if (e != hipSuccess) return hip_fail(e, "IVF-PQ workspace");
        int64_t* d_seg = (int64_t*)slot->aux2.p;
        int64_t* d_total = (int64_t*)((char*)slot->aux2.p + seg_bytes);
        int32_t* d_nitems = (int32_t*)slot->aux3.p;
        int32_t* d_item_off = d_nitems + npend;
        int32_t* d_item_q = d_item_off + npend + 1;
        hipLaunchKernelGGL(ivf_plan, dim3((unsigned)((npend + 3) / 4)), dim3(256), 0, st, d_probes, np,
                           d_qidx, npend, (const int64_t*)pq->offsets.p, chunk, d_seg, d_total, d_nitems);
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
        pa.rows = (const float*)pq->corpus->rows.p;
        pa.norms = (const float*)pq->corpus->norms.p;
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
        switch (rerank_k > 0 ? nch : 1) {
        case 1: launch_pq_scan<1>(items_bound, cap, kc, pa, d_q, d_qidx, fa, st); break;
        case 2: launch_pq_scan<2>(items_bound, cap, kc, pa, d_q, d_qidx, fa, st); break;
        case 3: launch_pq_scan<3>(items_bound, cap, kc, pa, d_q, d_qidx, fa, st); break;
        case 4: launch_pq_scan<4>(items_bound, cap, kc, pa, d_q, d_qidx, fa, st); break;
        case 6: launch_pq_scan<6>(items_bound, cap, kc, pa, d_q, d_qidx, fa, st); break;
        case 8: launch_pq_scan<8>(items_bound, cap, kc, pa, d_q, d_qidx, fa, st); break;
        default: return fail(MANS_PIPELINE_UNAVAILABLE, "IVF-PQ: unsupported dim");
        }
        e = hipGetLastError();
        if (e == hipSuccess)
            e = hipMemcpyAsync(slot->status_h.p, slot->status.p, (size_t)npend, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) {
            slot->counters_dirty = true;
            return hip_fail(e, "IVF-PQ scan");
        }
        const uint8_t* sh = (const uint8_t*)slot->status_h.p;
        std::vector<uint32_t> next;
        for (int64_t i = 0; i < npend; ++i)
            if (sh[i]) next.push_back(pending.empty() ? (uint32_t)i : pending[i]);
        if (next.empty()) break;
        if (kc >= 2048) return fail(MANS_SEARCH_FAILED, "IVF-PQ: too many scores tie at the k-th");
        pending.swap(next);
        npend = (int64_t)pending.size();
        kc = std::min(kc * 4, 2048);
    }
    ctx->time_end(slot, st, "ivfpq_scan");
    return MANS_OK;
}

}  // namespace mans

using namespace mans;

extern "C" {

int mans_ivf_flat_build(mans_ctx* ctx, const mans_corpus* corpus, const float* centroids,
                        int64_t nlist, uint32_t metric, mans_ivf** out) {
    if (out) *out = nullptr;
    if (!ctx || !corpus || !out || (nlist > 0 && !centroids))
        return fail(MANS_SEARCH_FAILED, "mans_ivf_flat_build: NULL argument");
    if (nlist < 1) return fail(MANS_SEARCH_FAILED, "mans_ivf_flat_build: nlist must be >= 1");
    if (metric > 2) return fail(MANS_SEARCH_FAILED, "IVF-flat does not support this metric");
    DeviceGuard dg(ctx->device);
    mans_corpus* cent = nullptr;
    int rc = mans_corpus_upload_f32(ctx, centroids, nlist, corpus->dim, &cent);
    if (rc != MANS_OK) return rc;
    return ivf_build_from_centroids(ctx, corpus, cent, metric, out);
}

int mans_kmeans(mans_ctx* ctx, const mans_corpus* corpus, int64_t k, int64_t iters, uint32_t metric,
                float* out_centroids) {
    if (!ctx || !corpus || !out_centroids) return fail(MANS_SEARCH_FAILED, "mans_kmeans: NULL argument");
    if (k < 1 || k > corpus->n) return fail(MANS_SEARCH_FAILED, "mans_kmeans: need 1 <= k <= n");
    if (iters < 0) return fail(MANS_SEARCH_FAILED, "mans_kmeans: iters must be >= 0");
    if (metric > 2) return fail(MANS_SEARCH_FAILED, "k-means does not support this metric");
    DeviceGuard dg(ctx->device);
    SlotLease lease(ctx);
    if (!lease.slot) return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    hipStream_t st = lease.slot->stream;
    const int64_t n = corpus->n, dim = corpus->dim;
    // Rows 0, s, 2s, ... with s = max(1, n / k).
    const int64_t stride = n / k > 1 ? n / k : 1;
    std::vector<uint32_t> init((size_t)k);
    for (int64_t c = 0; c < k; ++c) init[c] = (uint32_t)((c * stride) % n);
    DevBuf d_idx, d_cent, d_off, d_ids;
    hipError_t e = d_idx.ensure(k * sizeof(uint32_t), ctx->fail_alloc);
    if (e == hipSuccess) e = d_cent.ensure((size_t)k * dim * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = d_off.ensure((k + 1) * sizeof(int64_t), ctx->fail_alloc);
    if (e == hipSuccess) e = d_ids.ensure((size_t)n * sizeof(uint32_t), ctx->fail_alloc);
    if (e == hipSuccess) e = hipMemcpyAsync(d_idx.p, init.data(), k * sizeof(uint32_t), hipMemcpyHostToDevice, st);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(ivf_gather_rows, dim3((unsigned)((k + 3) / 4)), dim3(256), 0, st,
                           (const float*)corpus->rows.p, (const float*)nullptr,
                           (const uint32_t*)d_idx.p, k, (int)dim, (float*)d_cent.p, (float*)nullptr);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return hip_fail(e, "k-means init");
    for (int64_t it = 0; it < iters; ++it) {
        mans_corpus* cent = nullptr;
        int rc = corpus_from_device(ctx, (const float*)d_cent.p, k, dim, st, &cent);
        if (rc != MANS_OK) return rc;
        std::vector<int32_t> assign;
        std::vector<int64_t> offsets;
        std::vector<uint32_t> ids;
        rc = ivf_assign_and_lists(ctx, cent, (const float*)corpus->rows.p, n, metric, lease.slot,
                                  &assign, &offsets, &ids);
        mans_corpus_release(cent);
        if (rc != MANS_OK) return rc;
        e = hipMemcpyAsync(d_off.p, offsets.data(), (k + 1) * sizeof(int64_t), hipMemcpyHostToDevice, st);
        if (e == hipSuccess)
            e = hipMemcpyAsync(d_ids.p, ids.data(), n * sizeof(uint32_t), hipMemcpyHostToDevice, st);
        if (e == hipSuccess) {
            const int64_t threads = k * dim;
            hipLaunchKernelGGL(kmeans_update, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                               (const float*)corpus->rows.p, (const int64_t*)d_off.p,
                               (const uint32_t*)d_ids.p, k, (int)dim, (float*)d_cent.p);
            e = hipGetLastError();
        }
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "k-means iteration");
    }
    e = hipMemcpyAsync(out_centroids, d_cent.p, (size_t)k * dim * sizeof(float), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? MANS_OK : hip_fail(e, "k-means download");
}

int mans_ivf_flat_search_device(mans_ctx* ctx, const mans_ivf* ivf, const float* d_queries,
                                int64_t nq, int64_t k, int64_t nprobe, float* d_out_dist,
                                uint32_t* d_out_ids, void* stream) {
    if (!ctx || !ivf) return fail(MANS_SEARCH_FAILED, "NULL context or index");
    if (nq > 0 && k > 0 && (!d_queries || !d_out_dist || !d_out_ids))
        return fail(MANS_SEARCH_FAILED, "NULL buffer");
    DeviceGuard dg(ctx->device);
    SlotLease lease(ctx);
    if (!lease.slot) return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    hipStream_t st = stream ? (hipStream_t)stream : lease.slot->stream;
    int rc = ivf_search_run(ctx, ivf, d_queries, nq, k, nprobe, d_out_dist, d_out_ids, nullptr, st,
                            lease.slot);
    if (rc == MANS_OK) {
        hipError_t e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "IVF scan");
    }
    return rc;
}

int mans_ivf_flat_search(mans_ctx* ctx, const mans_ivf* ivf, const float* queries, int64_t nq,
                         int64_t k, int64_t nprobe, float* out_dist, uint32_t* out_ids,
                         int32_t* out_probes) {
    if (!ctx || !ivf) return fail(MANS_SEARCH_FAILED, "NULL context or index");
    if (nq <= 0 || k <= 0) return MANS_OK;
    if (!queries || !out_dist || !out_ids) return fail(MANS_SEARCH_FAILED, "NULL buffer");
    DeviceGuard dg(ctx->device);
    SlotLease lease(ctx);
    Slot* s = lease.slot;
    if (!s) return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    const size_t qbytes = (size_t)nq * ivf->dim * sizeof(float);
    const size_t obytes = (size_t)nq * k * sizeof(float);
    hipError_t e = s->queries.ensure(qbytes, ctx->fail_alloc);
    if (e == hipSuccess) e = s->dist.ensure(obytes, ctx->fail_alloc);
    if (e == hipSuccess) e = s->ids.ensure(obytes, ctx->fail_alloc);
    if (e == hipSuccess) e = stage_to_device(s, s->queries.p, queries, qbytes);
    if (e != hipSuccess) return hip_fail(e, "IVF scan staging");
    int rc = ivf_search_run(ctx, ivf, (const float*)s->queries.p, nq, k, nprobe, (float*)s->dist.p,
                            (uint32_t*)s->ids.p, out_probes, s->stream, s);
    if (rc != MANS_OK) return rc;
    e = stage_from_device(s, out_dist, s->dist.p, obytes, out_ids, s->ids.p, obytes);
    return e == hipSuccess ? MANS_OK : hip_fail(e, "IVF scan results");
}

int mans_ivf_download_lists(const mans_ivf* ivf, int64_t* offsets, uint32_t* list_ids) {
    if (!ivf) return fail(MANS_SEARCH_FAILED, "NULL index");
    DeviceGuard dg(ivf->ctx->device);
    if (offsets) std::memcpy(offsets, ivf->h_offsets.data(), (ivf->nlist + 1) * sizeof(int64_t));
    hipError_t e = hipSuccess;
    if (list_ids && ivf->n > 0)
        e = hipMemcpy(list_ids, ivf->list_ids.p, ivf->n * sizeof(uint32_t), hipMemcpyDeviceToHost);
    return e == hipSuccess ? MANS_OK : hip_fail(e, "IVF lists download");
}

void mans_ivf_release(mans_ivf* ivf) {
    if (!ivf) return;
    DeviceGuard dg(ivf->ctx->device);
    (void)hipDeviceSynchronize();
    delete ivf;
}

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

}  // extern "C"
