// IVF-flat on gfx950: partition build (IVFFlatSearch.swift:517-703) and
// probe selection and probed-list scan (IVFFlatSearch.swift:115-311).  The
// k-means that trains the centroids is in mans_kmeans.hip.
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
#include "mans_ivf.hpp"
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

int mans_ivf_flat_search_device(mans_ctx* ctx, const mans_ivf* ivf, const float* d_queries,
                                int64_t nq, int64_t k, int64_t nprobe, float* d_out_dist,
                                uint32_t* d_out_ids, void* stream) {
    if (!ctx || !ivf) return fail(MANS_SEARCH_FAILED, "NULL context or index");
    if (check_k(k) != MANS_OK) return MANS_SEARCH_FAILED;
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
    if (check_k(k) != MANS_OK) return MANS_SEARCH_FAILED;
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

}  // extern "C"
