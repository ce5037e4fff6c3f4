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
#include <cstdlib>
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
    mans::DevBuf cent_t;          // f32 [dim][nlist], the centroids transposed
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

// Exclusive scan of one value per thread of a 1024-thread block (wave
// shuffles, then the 16 wave sums from LDS); *total gets the block's sum.
template <typename T>
__device__ __forceinline__ T block1024_exclusive_scan(T v, T* wsum, T* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    T incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const T t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    T before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
        const T x = wsum[w];
        before += w < wave ? x : (T)0;
        all += x;
    }
    *total = all;
    return before + incl - v;
}

// One block: exclusive scan of the per-query item counts, then the item ->
// query map.  item_off[nq] holds the number of items.
__global__ __launch_bounds__(1024) void ivf_items(const int32_t* __restrict__ nitems, int64_t nq,
                                                   int32_t* __restrict__ item_off,
                                                   int32_t* __restrict__ item_q) {
    __shared__ int32_t wsum[16];
    const int tid = threadIdx.x;
    const int64_t per = (nq + 1023) / 1024;
    const int64_t a = tid * per < nq ? tid * per : nq;
    const int64_t b = a + per < nq ? a + per : nq;
    int32_t s = 0;
    for (int64_t i = a; i < b; ++i) s += nitems[i];
    int32_t total;
    int32_t run = block1024_exclusive_scan(s, wsum, &total);
    if (tid == 0) item_off[nq] = total;
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

// ---------------------------------------------------------------------------
// Probe selection (IVFFlatSearch.swift:224-251, smallestIndices :314-382):
// every centroid's key from its dot with the query in the scalar order of
// dots.c:40-47 and the host formulas, then the nprobe smallest by (key,
// index).  The scan does not depend on the probes' order.

// dst[d][c] = src[c][d].
__global__ __launch_bounds__(256) void ivf_transpose(const float* __restrict__ src, int64_t rows,
                                                     int dim, float* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * dim) return;
    const int64_t c = i / dim, d = i - c * dim;
    dst[d * rows + c] = src[i];
}

constexpr int kCoarseQ = 16;  // queries per block row

// grid (ceil(nlist / 256), ceil(nq / kCoarseQ)); block 256; dim a multiple
// of 4.  keys: [nq][nlist].  Thread per centroid, kCoarseQ queries per
// block: the queries' elements are uniform across the block and come in
// through scalar loads, so the loop is the centroid column load and the
// mul + add of each (query, dim) in the dots.c order.
__global__ __launch_bounds__(256) void ivf_coarse_keys(const float* __restrict__ queries, int64_t nq,
                                                       int dim, const float* __restrict__ cent_t,
                                                       const float* __restrict__ cnorms, int nlist,
                                                       int metric, float* __restrict__ keys) {
    __shared__ float cqn[kCoarseQ];
    const int tid = threadIdx.x;
    const int64_t q0 = (int64_t)blockIdx.y * kCoarseQ;
    const float* qrow[kCoarseQ];
#pragma unroll
    for (int j = 0; j < kCoarseQ; ++j) qrow[j] = queries + (q0 + j < nq ? q0 + j : nq - 1) * dim;
    if (tid < kCoarseQ) {
        const float* qp = queries + (q0 + tid < nq ? q0 + tid : nq - 1) * dim;
        float s = 0.0f;
        for (int d = 0; d < dim; ++d) s = s + qp[d] * qp[d];
        cqn[tid] = metric == kMetricIP ? 0.0f : s;
    }
    __syncthreads();
    const int c = blockIdx.x * blockDim.x + tid;
    if (c >= nlist) return;
    float acc[kCoarseQ];
#pragma unroll
    for (int j = 0; j < kCoarseQ; ++j) acc[j] = 0.0f;
    for (int d0 = 0; d0 < dim; d0 += 4) {
        float b[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) b[t] = cent_t[(int64_t)(d0 + t) * nlist + c];
#pragma unroll
        for (int j = 0; j < kCoarseQ; ++j) {
            const f4v qv = *reinterpret_cast<const f4v*>(qrow[j] + d0);
            acc[j] = acc[j] + qv.x * b[0];
            acc[j] = acc[j] + qv.y * b[1];
            acc[j] = acc[j] + qv.z * b[2];
            acc[j] = acc[j] + qv.w * b[3];
        }
    }
    const float cn = metric == kMetricIP ? 0.0f : cnorms[c];
#pragma unroll
    for (int j = 0; j < kCoarseQ; ++j)
        if (q0 + j < nq) keys[(q0 + j) * nlist + c] = host_distance(acc[j], cqn[j], cn, metric);
}

constexpr int kProbeLdsSlots = 8192;

// Block per query: the np smallest (key, index) of its nlist keys, written
// in any order.  dynamic LDS: nlist slots when nlist <= kProbeLdsSlots.
__global__ __launch_bounds__(256) void ivf_probe_select(const float* __restrict__ keys, int nlist,
                                                        int np, uint32_t* __restrict__ probes) {
    extern __shared__ uint64_t lds[];
    __shared__ uint32_t hist[256];
    __shared__ int cnt;
    const int tid = threadIdx.x;
    const int64_t q = blockIdx.x;
    const float* kq = keys + q * nlist;
    const bool in_lds = nlist <= kProbeLdsSlots;
    if (in_lds)
        for (int c = tid; c < nlist; c += blockDim.x) lds[c] = pack_slot(kq[c], (uint32_t)c);
    if (tid == 0) cnt = 0;
    __syncthreads();
    auto get = [&](int64_t c) { return in_lds ? lds[c] : pack_slot(kq[c], (uint32_t)c); };
    uint64_t kth;
    const uint64_t cut = block_radix_cut(get, nlist, np, hist, &kth);
    for (int c = tid; c < nlist; c += blockDim.x) {
        if (get(c) <= cut) {
            const int p = atomicAdd(&cnt, 1);
            if (p < np) probes[q * np + p] = (uint32_t)c;
        }
    }
}

constexpr int kProbeWaveMax = 64;  // np served by ivf_probe_select_waves

// Block per query, np <= kProbeWaveMax: the same np smallest (key, index)
// slots as ivf_probe_select, ascending.  Wave w offers keys w 64 + 256 i to
// its own list (WaveTopKT keeps the np smallest slots, ties by index), then
// wave 0 takes the other three lists.  A NaN key counts as +inf.  The radix
// cut's first passes put nearly every key of a query in one or two bins of
// the float's top bytes, where the LDS atomics serialise; these lists look
// at each key once.
__global__ __launch_bounds__(256) void ivf_probe_select_waves(const float* __restrict__ keys,
                                                              int nlist, int np,
                                                              uint32_t* __restrict__ probes) {
    __shared__ uint64_t lists[4 * 128];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t q = blockIdx.x;
    const float* kq = keys + q * nlist;
    WaveTopKT<128> sel;
    sel.init(lists + wave * 128, 128, np);
    for (int base = wave * 64; base < nlist; base += 256) {
        const int c = base + lane;
        const bool v = c < nlist;
        float key = v ? kq[c] : 0.0f;
        key = key == key ? key : __int_as_float(0x7F800000);
        sel.offer(v, key, (uint32_t)c);
    }
    sel.finish();
    __syncthreads();
    if (wave == 0) {
        for (int w = 1; w < 4; ++w) sel.offer_slots(lists + w * 128, np);
        sel.finish();
        if (lane < np) probes[q * np + lane] = slot_id(lists[lane]);
    }
}

// ---------------------------------------------------------------------------
// List-major batch scan (first round of a batch of at least kLmMinBatch
// queries).  The per-query scan above reads a list once for every query
// that probes it; here each probed list is read once per batch: the
// (query, probe) pairs are grouped by list, and a work item takes one chunk
// of up to kLmRows rows of a list and up to kLmQueries of the queries
// probing it.  The item stages its queries and, tile by tile, the chunk's
// rows in LDS (the next tile's loads in flight), forms every (query, row)
// fast dot -- on fp32 MFMA for dim <= 128, else with fused multiply-adds in
// register tiles of one query by several rows (the tile's query width
// follows the item's query count: 4, 8 or 16) -- turns them into the
// streaming scan's lower-bound keys and offers
// each query's keys of the tile to that query's selection (a wave keeps
// four queries' kc best).  Each (query, chunk) leaves one candidate list.
// A query's chunk lists hold its kc best keys over all its probed rows (an
// entry of the kc best has fewer than kc smaller keys in its own chunk), so
// the per-query merge, exact rescore and proof are those of the per-query
// scan; queries whose proof fails go back to it with a larger candidate
// count.  A chunk list that fills lowers its query's shared bound (the
// smallest kc-th key of any filled list, an upper bound on the query's kc-th
// key over all its rows); later items of the query offer only keys at or
// below it.  The rows this turns away have keys above the merge's cutoff.
constexpr int kLmRows = 512;
constexpr int kLmQueries = 16;
constexpr int64_t kLmMinBatch = 64;
constexpr int kLmMaxNch = 4;  // dim <= 256
constexpr int kLmMergeCap = 128;  // merge selection slots per wave (kc <= 64)

template <int NCH>
struct LmShape {
    static constexpr int kT = NCH <= 2 ? 64 : 32;         // rows per LDS tile
    static constexpr int kRowF = 64 * NCH + 4;            // floats per staged row
    static constexpr int kQF = 64 * NCH + 4;              // floats per staged query
    static constexpr int kLoads = kT * 16 * NCH / 256;    // float4 tile loads per thread
    static constexpr int kMinGp = NCH <= 2 ? 4 : 8;       // narrowest register tile
    static constexpr size_t kQsOff = 0;
    static constexpr size_t kQnOff = kQsOff + sizeof(float) * kLmQueries * kQF;
    static constexpr size_t kTileOff = kQnOff + sizeof(float) * kLmQueries;
    static constexpr size_t kVnOff = kTileOff + sizeof(float) * kT * kRowF;
    static constexpr size_t kKeyOff = kVnOff + sizeof(float) * kT;
    // Keys per query, padded for the banks: the MFMA path writes rows 16 w + j
    // of queries 4 g + r from lane 16 g + j (4 stride = 16 mod 64 banks), the
    // VALU path query t % GP of row t / GP + ... from thread t.
    static constexpr int kKeyStride = NCH <= 2 ? kT + 4 : kT + 1;
    static constexpr size_t kSelOff =
        (kKeyOff + sizeof(float) * kLmQueries * kKeyStride + 15) / 16 * 16;
    static constexpr size_t kBytes = kSelOff + sizeof(uint64_t) * kLmQueries * 128;
};

struct LmArgs {
    const float* packed;
    const float* packed_norms;
    const int64_t* offsets;   // [nlist + 1] packed rows of each list
    const uint32_t* probes;   // [nq][np]
    const int32_t* lstart;    // [nlist + 1] first (query, probe) pair of each list
    const int32_t* lpairs;    // [nq np] pairs q np + p grouped by list
    const int32_t* item_off;  // [nlist] first work item of each list, [nlist] the item count
    const int2* items;        // [items] (list, chunk + group << 16) of each work item
    const int32_t* qchunk;    // [nq][np] the query's first chunk list of probe p
    const int64_t* qbase;     // [nq + 1] the query's first candidate list
    uint32_t* qbound;         // [nq] ordered bits of a bound on the query's kc-th key
    int np;
    int nlist;
};

// Thread per (query, probe) pair: lcount[list] += 1.
__global__ __launch_bounds__(256) void ivf_lm_count(const uint32_t* __restrict__ probes,
                                                    int64_t pairs, int32_t* __restrict__ lcount) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < pairs) atomicAdd(&lcount[probes[i]], 1);
}

// Work items of a list of `rows` rows probed by m queries: its 512-row
// chunks times its groups of up to 16 queries.
__device__ __forceinline__ int32_t lm_items_of(int64_t rows, int32_t m) {
    if (m == 0 || rows == 0) return 0;
    return (int32_t)(((rows + kLmRows - 1) / kLmRows) * ((m + kLmQueries - 1) / kLmQueries));
}

// Class of a list's work rows x m on a half-octave scale (0 .. 63).
__device__ __forceinline__ int lm_work_class(int64_t rows, int32_t m) {
    const uint64_t x = (uint64_t)rows * (uint64_t)m;
    if (x < 2) return 0;
    const int fl = 63 - __clzll((long long)x);
    const int c = 2 * fl + (int)((x >> (fl - 1)) & 1);
    return c < 63 ? c : 63;
}

// One block: lstart = exclusive scan of the lists' pair counts; item_off[L]
// = the first work item of list L, with the lists laid out by ascending
// work (rows x probing queries, half-octave classes, any order within a
// class): the short items run first and their filled chunk lists set their
// queries' shared kc-th key bounds before the long items of the same
// queries start (at 1M x 128, nprobe 4 / 32: scan 178 / 637 us in list
// order, 184 / 636 longest first by item count, 157 / 585 shortest first by
// item count, 149 / 581 by work).  item_off[nlist] = the number of items.
// The order of the items changes no result (each writes its own candidate
// lists).  lcount is cleared for ivf_lm_fill.
__global__ __launch_bounds__(1024) void ivf_lm_lists(int32_t* __restrict__ lcount,
                                                     const int64_t* __restrict__ offsets, int nlist,
                                                     int32_t* __restrict__ lstart,
                                                     int32_t* __restrict__ item_off) {
    constexpr int kClasses = 64;
    __shared__ int32_t wsum_p[16];
    __shared__ int32_t class_items[kClasses], class_base[kClasses], class_fill[kClasses];
    const int tid = threadIdx.x, lane = tid & 63;
    const int per = (nlist + 1023) / 1024;
    const int a = tid * per < nlist ? tid * per : nlist;
    const int b = a + per < nlist ? a + per : nlist;
    if (tid < kClasses) {
        class_items[tid] = 0;
        class_fill[tid] = 0;
    }
    int32_t sp = 0;
    for (int L = a; L < b; ++L) sp += lcount[L];
    int32_t tp;
    int32_t rp = block1024_exclusive_scan(sp, wsum_p, &tp);  // its barrier orders the clears
    for (int L = a; L < b; ++L) {
        const int64_t rows = offsets[L + 1] - offsets[L];
        const int32_t ni = lm_items_of(rows, lcount[L]);
        if (ni > 0) atomicAdd(&class_items[lm_work_class(rows, lcount[L])], ni);
    }
    __syncthreads();
    if (tid < 64) {
        // Lane l takes class l: the classes' first items, smallest first.
        const int32_t own = class_items[lane];
        int32_t incl = own;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int32_t t = __shfl_up(incl, o);
            if (lane >= o) incl += t;
        }
        class_base[lane] = incl - own;
        if (lane == 63) item_off[nlist] = incl;
    }
    if (tid == 0) lstart[nlist] = tp;
    __syncthreads();
    for (int L = a; L < b; ++L) {
        const int32_t m = lcount[L];
        const int64_t rows = offsets[L + 1] - offsets[L];
        const int32_t ni = lm_items_of(rows, m);
        const int cls = lm_work_class(rows, m);
        lstart[L] = rp;
        item_off[L] = ni > 0 ? class_base[cls] + atomicAdd(&class_fill[cls], ni) : 0;
        rp += m;
        lcount[L] = 0;
    }
}

// Wave per list: the descriptors of its work items (chunk-major within a
// query group: item g nchunk + c).
__global__ __launch_bounds__(256) void ivf_lm_items(const int32_t* __restrict__ item_off,
                                                    const int32_t* __restrict__ lstart,
                                                    const int64_t* __restrict__ offsets, int nlist,
                                                    int2* __restrict__ items) {
    const int L = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (L >= nlist) return;
    const int64_t rows = offsets[L + 1] - offsets[L];
    const int count = lm_items_of(rows, lstart[L + 1] - lstart[L]);
    if (count == 0) return;
    const int first = item_off[L];
    const int nchunk = (int)((rows + kLmRows - 1) / kLmRows);
    for (int li = lane; li < count; li += 64) {
        const int g = li / nchunk, c = li - g * nchunk;
        items[first + li] = make_int2(L, c | (g << 16));
    }
}

// Thread per pair: its place among its list's pairs (any order).
__global__ __launch_bounds__(256) void ivf_lm_fill(const uint32_t* __restrict__ probes,
                                                   int64_t pairs, const int32_t* __restrict__ lstart,
                                                   int32_t* __restrict__ lfill,
                                                   int32_t* __restrict__ lpairs) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= pairs) return;
    const uint32_t L = probes[i];
    lpairs[lstart[L] + atomicAdd(&lfill[L], 1)] = (int32_t)i;
}

// No bound on a query's kc-th key yet (above every ordered key).
constexpr uint32_t kNoBound = 0xFFFFFFFFu;

// Wave per query: the first chunk list of each probe among the query's
// lists, the query's list count and its probed rows; its kc-th key bound is
// reset.
__global__ __launch_bounds__(256) void ivf_lm_qplan(const uint32_t* __restrict__ probes, int np,
                                                    int64_t nq, const int64_t* __restrict__ offsets,
                                                    int32_t* __restrict__ qchunk,
                                                    int32_t* __restrict__ qcount,
                                                    int64_t* __restrict__ qtotal,
                                                    uint32_t* __restrict__ qbound) {
    const int lane = threadIdx.x & 63;
    const int64_t q = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (q >= nq) return;  // the whole wave leaves together
    int32_t carry = 0;
    int64_t rows_all = 0;
    for (int base = 0; base < np; base += 64) {
        const int p = base + lane;
        int32_t nch = 0;
        int64_t rows = 0;
        if (p < np) {
            const uint32_t L = probes[q * np + p];
            rows = offsets[L + 1] - offsets[L];
            nch = (int32_t)((rows + kLmRows - 1) / kLmRows);
        }
        int32_t incl = nch;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int32_t t = __shfl_up(incl, o);
            if (lane >= o) incl += t;
        }
        if (p < np) qchunk[q * np + p] = carry + incl - nch;
        carry += __shfl(incl, 63);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) rows += __shfl_xor(rows, o);
        rows_all += rows;
    }
    if (lane == 0) {
        qcount[q] = carry;
        qtotal[q] = rows_all;
        qbound[q] = kNoBound;
    }
}

// One block: qbase = exclusive scan of the queries' list counts.
__global__ __launch_bounds__(1024) void ivf_lm_qscan(const int32_t* __restrict__ qcount, int64_t nq,
                                                     int64_t* __restrict__ qbase) {
    __shared__ int64_t wsum[16];
    const int tid = threadIdx.x;
    const int64_t per = (nq + 1023) / 1024;
    const int64_t a = tid * per < nq ? tid * per : nq;
    const int64_t b = a + per < nq ? a + per : nq;
    int64_t sum = 0;
    for (int64_t i = a; i < b; ++i) sum += qcount[i];
    int64_t total;
    int64_t run = block1024_exclusive_scan(sum, wsum, &total);
    if (tid == 0) qbase[nq] = total;
    for (int64_t i = a; i < b; ++i) {
        qbase[i] = run;
        run += qcount[i];
    }
}

// The dots of one tile for GP queries: thread t takes query t % GP and rows
// t / GP + (256 / GP) j; their keys go to tkeys[query][row].
template <int NCH, int GP>
__device__ __forceinline__ void lm_tile_keys(const float* qs, const float* qnorm, const float* tile,
                                             const float* vn, float* tkeys, int dim4, int nvalid,
                                             int metric, const BoundCoef& bc) {
    using S = LmShape<NCH>;
    constexpr int kStep = 256 / GP, kPer = S::kT / kStep;
    const int tid = threadIdx.x, gq = tid % GP, rs = tid / GP;
    float acc[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) acc[j] = 0.0f;
    const float* qrow = qs + gq * S::kQF;
    for (int d4 = 0; d4 < dim4; ++d4) {
        const f4v x = *reinterpret_cast<const f4v*>(qrow + 4 * d4);
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const f4v y = *reinterpret_cast<const f4v*>(tile + (rs + kStep * j) * S::kRowF + 4 * d4);
            acc[j] = fmaf(x.x, y.x, acc[j]);
            acc[j] = fmaf(x.y, y.y, acc[j]);
            acc[j] = fmaf(x.z, y.z, acc[j]);
            acc[j] = fmaf(x.w, y.w, acc[j]);
        }
    }
    auto put = [&](auto key_of) {
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int r = rs + kStep * j;
            if (r < nvalid) tkeys[gq * S::kKeyStride + r] = key_of(acc[j], qnorm[gq], vn[r]);
        }
    };
    if (metric == kMetricL2)
        put([&](float f, float qn, float v) { return lower_key_m<kMetricL2>(f, qn, v, bc); });
    else if (metric == kMetricIP)
        put([&](float f, float qn, float v) { return lower_key_m<kMetricIP>(f, qn, v, bc); });
    else
        put([&](float f, float qn, float v) { return lower_key_m<kMetricCosine>(f, qn, v, bc); });
}

// The dots of one 64-row tile on fp32 MFMA (dim <= 128): wave w takes tile
// rows 16 w .. 16 w + 15 against all 16 queries with
// v_mfma_f32_16x16x4f32 (lane l: query l % 16 in A, row l % 16 in B, dims
// g 16 NCH + s of lane group g = l / 16 at step s: any order of the d
// products is within the keys' bound); lane l gets (query 4 g + r, row
// l % 16) for r < 4.  qa: the lane's query values (16 NCH, loaded once per
// item).  abs_slack covers products and sums the MFMA flushes below
// 2^-126.
template <int NCH>
__device__ __forceinline__ void lm_tile_keys_mfma(const float (&qa)[16 * NCH], const float* qnorm,
                                                  const float* tile, const float* vn, float* tkeys,
                                                  int nvalid, int metric, const BoundCoef& bc,
                                                  float abs_slack) {
    using S = LmShape<NCH>;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const float* brow = tile + (16 * wave + j) * S::kRowF + g * 16 * NCH;
    f4v c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4 * NCH; ++t) {
        const f4v b = *reinterpret_cast<const f4v*>(brow + 4 * t);
        c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * t + 0], b.x, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * t + 1], b.y, c1, 0, 0, 0);
        c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * t + 2], b.z, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * t + 3], b.w, c1, 0, 0, 0);
    }
    const int row = 16 * wave + j;
    if (row < nvalid) {
        const float v = vn[row];
        auto put = [&](auto key_of) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int q = 4 * g + r;
                tkeys[q * S::kKeyStride + row] = key_of(c0[r] + c1[r], qnorm[q]) - abs_slack;
            }
        };
        if (metric == kMetricL2)
            put([&](float f, float qn) { return lower_key_m<kMetricL2>(f, qn, v, bc); });
        else if (metric == kMetricIP)
            put([&](float f, float qn) { return lower_key_m<kMetricIP>(f, qn, v, bc); });
        else
            put([&](float f, float qn) { return lower_key_m<kMetricCosine>(f, qn, v, bc); });
    }
}

// Grid of blocks striding over the work items; block 256; dynamic LDS
// LmShape<NCH>::kBytes.  cand: kc slots per (query, chunk) list.
template <int NCH>
__global__ __launch_bounds__(256) void ivf_lm_scan(LmArgs la, int dim,
                                                   const float* __restrict__ queries, int metric,
                                                   BoundCoef bc, float abs_slack, int kc,
                                                   uint64_t* __restrict__ cand) {
    using S = LmShape<NCH>;
    constexpr int kT = S::kT;
    extern __shared__ __align__(16) uint8_t lm_lds[];
    float* qs = reinterpret_cast<float*>(lm_lds + S::kQsOff);
    float* qnorm = reinterpret_cast<float*>(lm_lds + S::kQnOff);
    float* tile = reinterpret_cast<float*>(lm_lds + S::kTileOff);
    float* vn = reinterpret_cast<float*>(lm_lds + S::kVnOff);
    float* tkeys = reinterpret_cast<float*>(lm_lds + S::kKeyOff);
    uint64_t* selbuf = reinterpret_cast<uint64_t*>(lm_lds + S::kSelOff);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int dim4 = dim >> 2;
    const int total_items = la.item_off[la.nlist];
    for (int item = blockIdx.x; item < total_items; item += gridDim.x) {
        const int2 desc = la.items[item];
        const int L = desc.x, c = desc.y & 0xFFFF, g = desc.y >> 16;
        const int64_t r0 = la.offsets[L], nrows = la.offsets[L + 1] - r0;
        const int p0 = la.lstart[L] + g * kLmQueries;
        const int mg = min(kLmQueries, la.lstart[L + 1] - p0);
        const int gp = mg <= S::kMinGp ? S::kMinGp : (mg <= 8 ? 8 : 16);
        const int64_t a = r0 + (int64_t)c * kLmRows;
        const int64_t b = a + kLmRows < r0 + nrows ? a + kLmRows : r0 + nrows;
        uint32_t qbound_in[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int qq = wave + 4 * i;
            qbound_in[i] = kNoBound;
            if (qq < mg)
                qbound_in[i] = __hip_atomic_load(la.qbound + la.lpairs[p0 + qq] / la.np,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();  // the previous item is done with the LDS
        for (int e = tid; e < kLmQueries * 16 * NCH; e += 256) {
            const int qq = e / (16 * NCH), d4 = e - qq * 16 * NCH;
            f4v v = {0.f, 0.f, 0.f, 0.f};
            if (qq < mg && d4 < dim4) {
                const int q = la.lpairs[p0 + qq] / la.np;
                v = *reinterpret_cast<const f4v*>(queries + (int64_t)q * dim + 4 * d4);
            }
            *reinterpret_cast<f4v*>(qs + qq * S::kQF + 4 * d4) = v;
        }
        __syncthreads();
        {
            // Fast query norms: 16 lanes per query.
            const int qq = wave * 4 + (lane >> 4), lr = lane & 15;
            float acc = 0.0f;
            for (int d4 = lr; d4 < 16 * NCH; d4 += 16) {
                const f4v v = *reinterpret_cast<const f4v*>(qs + qq * S::kQF + 4 * d4);
                acc = fmaf(v.x, v.x, acc);
                acc = fmaf(v.y, v.y, acc);
                acc = fmaf(v.z, v.z, acc);
                acc = fmaf(v.w, v.w, acc);
            }
            acc = row16_sum(acc);
            if (lr == 0) qnorm[qq] = acc;
        }
        // The MFMA path's A fragment: query lane % 16, dims g 16 NCH + s.
        float qa[16 * NCH];
        if constexpr (NCH <= 2) {
            const float* qsrc = qs + (lane & 15) * S::kQF + (lane >> 4) * 16 * NCH;
#pragma unroll
            for (int t = 0; t < 4 * NCH; ++t) {
                const f4v v = *reinterpret_cast<const f4v*>(qsrc + 4 * t);
                qa[4 * t + 0] = v.x;
                qa[4 * t + 1] = v.y;
                qa[4 * t + 2] = v.z;
                qa[4 * t + 3] = v.w;
            }
        }
        // Wave w keeps the selections of queries w, w + 4, w + 8, w + 12.
        WaveTopKT<128> sel[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sel[i].init(selbuf + (wave + 4 * i) * 128, 128, kc);
            // A chunk list of the same query that has already filled gives
            // a bound on the query's kc-th key: rows above it are not among
            // the query's kc smallest keys, and every row this list turns
            // away still has a key above the merge's cutoff.
            const uint32_t qb = qbound_in[i];
            if (qb != kNoBound) sel[i].thresh = from_ordered_bits(qb);
        }
        // Row tiles, the next one's loads in flight during the current one's dots.
        f4v pf[S::kLoads];
        float pvn = 0.0f;
        auto load_tile = [&](int64_t t0) {
#pragma unroll
            for (int j = 0; j < S::kLoads; ++j) {
                const int e = tid + 256 * j;
                const int r = e / (16 * NCH), d4 = e - r * 16 * NCH;
                const bool in = t0 + r < b && d4 < dim4;
                const int64_t row = in ? t0 + r : a;
                const f4v t = load_stream(la.packed + row * dim + (in ? 4 * d4 : 0));
                pf[j] = in ? t : f4v{0.f, 0.f, 0.f, 0.f};
            }
            pvn = tid < kT && t0 + tid < b ? la.packed_norms[t0 + tid] : 0.0f;
        };
        load_tile(a);
        for (int64_t t0 = a; t0 < b; t0 += kT) {
            __syncthreads();  // the previous tile's dots are done
#pragma unroll
            for (int j = 0; j < S::kLoads; ++j) {
                const int e = tid + 256 * j;
                const int r = e / (16 * NCH), d4 = e - r * 16 * NCH;
                *reinterpret_cast<f4v*>(tile + r * S::kRowF + 4 * d4) = pf[j];
            }
            if (tid < kT) vn[tid] = pvn;
            __syncthreads();
            if (t0 + kT < b) load_tile(t0 + kT);
            const int nvalid = b - t0 < kT ? (int)(b - t0) : kT;
            if constexpr (NCH <= 2) {
                lm_tile_keys_mfma<NCH>(qa, qnorm, tile, vn, tkeys, nvalid, metric, bc, abs_slack);
            } else {
                if (gp == 16) lm_tile_keys<NCH, 16>(qs, qnorm, tile, vn, tkeys, dim4, nvalid, metric, bc);
                else if (gp == 8) lm_tile_keys<NCH, 8>(qs, qnorm, tile, vn, tkeys, dim4, nvalid, metric, bc);
                else lm_tile_keys<NCH, S::kMinGp>(qs, qnorm, tile, vn, tkeys, dim4, nvalid, metric, bc);
            }
            __syncthreads();  // the tile's keys are in tkeys
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int qq = wave + 4 * i;
                if (qq < mg) {
                    const bool v = lane < nvalid;
                    sel[i].offer(v, v ? tkeys[qq * S::kKeyStride + lane] : 0.0f, (uint32_t)(t0 + lane));
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int qq = wave + 4 * i;
            if (qq >= mg) continue;
            sel[i].finish();
            const int pair = la.lpairs[p0 + qq];
            const int q = pair / la.np, pr = pair - q * la.np;
            uint64_t* dst = cand + (la.qbase[q] + la.qchunk[(int64_t)q * la.np + pr] + c) * (int64_t)kc;
            for (int sidx = lane; sidx < kc; sidx += 64)
                dst[sidx] = sidx < sel[i].count ? sel[i].buf[sidx] : kEmptySlot;
            if (sel[i].count == kc && lane == 0)
                atomicMin(la.qbound + q, ordered_bits(slot_key(sel[i].buf[kc - 1])));
        }
    }
}

// Block per query: the kc best of its chunk lists, exact rescore (list ids
// reported), proof.  dynamic LDS: 4 * cap slots.
template <int NCH>
__global__ __launch_bounds__(256) void ivf_lm_merge(LmArgs la, const int64_t* __restrict__ qtotal,
                                                    int dim, const float* __restrict__ queries,
                                                    const uint32_t* __restrict__ list_ids,
                                                    int metric, int kc, int cap,
                                                    const uint64_t* __restrict__ cand, FlatArgs fa) {
    extern __shared__ uint64_t lds[];
    const int lane = threadIdx.x & 63, lr = lane & 15;
    const uint32_t q = blockIdx.x;
    const int dim4 = dim >> 2;
    const float* qp = queries + (int64_t)q * dim;
    f4v qv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = lr + 16 * c;
        qv[c] = idx < dim4 ? *reinterpret_cast<const f4v*>(qp + 4 * idx) : f4v{0.f, 0.f, 0.f, 0.f};
    }
    const int64_t first = la.qbase[q], nlists = la.qbase[q + 1] - first;
    WaveTopKT<kLmMergeCap> sel;  // the sorts compiled for 128 slots
    block_select_lists(cand + first * kc, nlists * kc, lds, cap, kc, sel);
    final_rescore_f4<NCH>(qv, la.packed, la.packed_norms, qtotal[q], dim, metric, q, lds, kc, fa,
                          kFltMax, kProofFlat, list_ids, (int)q);
}

template <int NCH>
static hipError_t launch_lm(const LmArgs& la, const int64_t* qtotal, int64_t nq, int dim,
                            const float* queries, const uint32_t* list_ids, int metric,
                            const BoundCoef& bc, int kc, uint64_t* cand, const FlatArgs& fa,
                            hipStream_t st) {
    using S = LmShape<NCH>;
    static const bool attr = [] {
        (void)hipFuncSetAttribute((const void*)ivf_lm_scan<NCH>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::kBytes);
        return true;
    }();
    (void)attr;
    // Products and partial sums the MFMA flushes below 2^-126 lose at most
    // 2^-126 each: 2 dim such terms in a dot, counted twice for L2's -2 dot.
    const float abs_slack = (float)(4.0 * dim * 1.1754943508222875e-38);
    // Far more blocks than fit on the chip (512 at two per CU): the
    // dispatcher hands the next item to whichever CU frees first, which
    // balances items of 1 to 8 tiles and 1 to 16 queries (measured at 1M x
    // 128, nprobe 4 / 32: 2.52M / 824k queries/s with 1024 blocks looping
    // over the items, 2.78M / 887k with 16384).  Blocks past the last item
    // leave at once; larger batches loop.
    static const unsigned grid = [] {
        const char* ev = std::getenv("MANS_IVF_LM_BLOCKS");
        return ev ? (unsigned)std::max(1, std::atoi(ev)) : 16384u;
    }();
    hipLaunchKernelGGL(ivf_lm_scan<NCH>, dim3(grid), dim3(256), S::kBytes, st, la, dim, queries,
                       metric, bc, abs_slack, kc, cand);
    const int cap = flat_cap_for(kc);
    if (cap != kLmMergeCap) return hipErrorInvalidValue;  // kc <= 64 on this path
    hipLaunchKernelGGL(ivf_lm_merge<NCH>, dim3((unsigned)nq), dim3(256),
                       sizeof(uint64_t) * 4 * (size_t)cap, st, la, qtotal, dim, queries, list_ids,
                       metric, kc, cap, (const uint64_t*)cand, fa);
    return hipGetLastError();
}

static bool ivf_list_major_enabled() {
    static const bool on = [] {
        const char* e = std::getenv("MANS_IVF_LIST_MAJOR");
        return !(e && e[0] == '0');
    }();
    return on;
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
    const int nlist_i = (int)ivf->nlist;
    const int64_t pchunk = std::min<int64_t>(nq, 2048);  // queries per key pass
    hipError_t e = slot->aux0.ensure((size_t)pchunk * nlist_i * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = slot->aux1.ensure((size_t)nq * np * sizeof(uint32_t), ctx->fail_alloc);
    if (e != hipSuccess) return hip_fail(e, "IVF probe workspace");
    ctx->time_begin(slot, st);
    for (int64_t q0 = 0; q0 < nq && e == hipSuccess; q0 += pchunk) {
        const int64_t m = std::min<int64_t>(pchunk, nq - q0);
        const dim3 grid((unsigned)((nlist_i + 255) / 256), (unsigned)((m + kCoarseQ - 1) / kCoarseQ));
        hipLaunchKernelGGL(ivf_coarse_keys, grid, dim3(256), 0, st, d_q + q0 * dim, m, dim, (const float*)ivf->cent_t.p,
                           (const float*)ivf->cent->norms.p, nlist_i, (int)metric, (float*)slot->aux0.p);
        if (np <= kProbeWaveMax)
            hipLaunchKernelGGL(ivf_probe_select_waves, dim3((unsigned)m), dim3(256), 0, st,
                               (const float*)slot->aux0.p, nlist_i, np,
                               (uint32_t*)slot->aux1.p + q0 * np);
        else
            hipLaunchKernelGGL(ivf_probe_select, dim3((unsigned)m), dim3(256),
                               nlist_i <= kProbeLdsSlots ? sizeof(uint64_t) * nlist_i : 0, st,
                               (const float*)slot->aux0.p, nlist_i, np,
                               (uint32_t*)slot->aux1.p + q0 * np);
        e = hipGetLastError();
    }
    ctx->time_end(slot, st, "ivf_probe");
    if (e != hipSuccess) return hip_fail(e, "IVF probes");
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
    if (nq >= kLmMinBatch && nch <= kLmMaxNch && kc <= 64 && ivf_list_major_enabled()) {
        // First round list-major; the queries whose proof fails continue
        // below with a larger candidate count.
        const int nlist = (int)ivf->nlist;
        const int64_t pairs = nq * np;
        const int64_t lists_bound = nq * ((int64_t)np + max_rows / kLmRows + 1);
        size_t off = 0;
        auto take = [&](size_t bytes) {
            const size_t at = off;
            off += (bytes + 15) / 16 * 16;
            return at;
        };
        const size_t o_lcount = take((size_t)nlist * 4), o_lstart = take((size_t)(nlist + 1) * 4);
        const size_t o_item = take((size_t)(nlist + 1) * 4), o_pairs = take((size_t)pairs * 4);
        const size_t o_qchunk = take((size_t)pairs * 4), o_qcount = take((size_t)nq * 4);
        const size_t o_qbase = take((size_t)(nq + 1) * 8), o_qtotal = take((size_t)nq * 8);
        const size_t o_qbound = take((size_t)nq * 4);
        // Work items: at most one per (query, chunk of a probed list) plus
        // one per (list, chunk) for the partial query groups.
        const int64_t items_bound = lists_bound + ivf->n / kLmRows + nlist;
        const size_t o_items = take((size_t)items_bound * sizeof(int2));
        e = slot->aux2.ensure(off, ctx->fail_alloc);
        if (e == hipSuccess)
            e = slot->cand.ensure((size_t)lists_bound * kc * sizeof(uint64_t), ctx->fail_alloc);
        if (e == hipSuccess) e = slot->status_h.ensure((size_t)nq);
        if (e != hipSuccess) return hip_fail(e, "IVF list-major workspace");
        char* base = (char*)slot->aux2.p;
        int32_t* lcount = (int32_t*)(base + o_lcount);
        LmArgs la;
        la.packed = (const float*)ivf->packed.p;
        la.packed_norms = (const float*)ivf->packed_norms.p;
        la.offsets = (const int64_t*)ivf->offsets.p;
        la.probes = d_probes;
        la.lstart = (const int32_t*)(base + o_lstart);
        la.lpairs = (const int32_t*)(base + o_pairs);
        la.item_off = (const int32_t*)(base + o_item);
        la.items = (const int2*)(base + o_items);
        la.qchunk = (const int32_t*)(base + o_qchunk);
        la.qbase = (const int64_t*)(base + o_qbase);
        la.qbound = (uint32_t*)(base + o_qbound);
        la.np = np;
        la.nlist = nlist;
        const int64_t* qtotal = (const int64_t*)(base + o_qtotal);
        e = hipMemsetAsync(lcount, 0, (size_t)nlist * 4, st);
        const unsigned pblocks = (unsigned)((pairs + 255) / 256);
        if (e == hipSuccess) {
            hipLaunchKernelGGL(ivf_lm_count, dim3(pblocks), dim3(256), 0, st, d_probes, pairs, lcount);
            hipLaunchKernelGGL(ivf_lm_lists, dim3(1), dim3(1024), 0, st, lcount,
                               (const int64_t*)ivf->offsets.p, nlist, (int32_t*)la.lstart,
                               (int32_t*)la.item_off);
            hipLaunchKernelGGL(ivf_lm_fill, dim3(pblocks), dim3(256), 0, st, d_probes, pairs,
                               la.lstart, lcount, (int32_t*)la.lpairs);
            hipLaunchKernelGGL(ivf_lm_items, dim3((unsigned)((nlist + 3) / 4)), dim3(256), 0, st,
                               la.item_off, la.lstart, (const int64_t*)ivf->offsets.p, nlist,
                               (int2*)la.items);
            hipLaunchKernelGGL(ivf_lm_qplan, dim3((unsigned)((nq + 3) / 4)), dim3(256), 0, st,
                               d_probes, np, nq, (const int64_t*)ivf->offsets.p,
                               (int32_t*)la.qchunk, (int32_t*)(base + o_qcount),
                               (int64_t*)qtotal, la.qbound);
            hipLaunchKernelGGL(ivf_lm_qscan, dim3(1), dim3(1024), 0, st,
                               (const int32_t*)(base + o_qcount), nq, (int64_t*)la.qbase);
            e = hipGetLastError();
        }
        FlatArgs fa = {};
        fa.out_dist = d_dist;
        fa.out_ids = d_ids;
        fa.status = (uint8_t*)slot->status_h.p;  // pinned: read after the stream syncs
        fa.k = keff;
        fa.k_stride = (int)k;
        const BoundCoef bc = make_bounds(dim);
        uint64_t* cand = (uint64_t*)slot->cand.p;
        const float* lq = d_q;
        const uint32_t* lids = (const uint32_t*)ivf->list_ids.p;
        ctx->time_begin(slot, st);
        if (e == hipSuccess) {
            switch (nch) {
            case 1: e = launch_lm<1>(la, qtotal, nq, dim, lq, lids, (int)metric, bc, kc, cand, fa, st); break;
            case 2: e = launch_lm<2>(la, qtotal, nq, dim, lq, lids, (int)metric, bc, kc, cand, fa, st); break;
            case 3: e = launch_lm<3>(la, qtotal, nq, dim, lq, lids, (int)metric, bc, kc, cand, fa, st); break;
            default: e = launch_lm<4>(la, qtotal, nq, dim, lq, lids, (int)metric, bc, kc, cand, fa, st); break;
            }
        }
        ctx->time_end(slot, st, "ivf_lm");
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "IVF list-major scan");
        const uint8_t* sh = (const uint8_t*)slot->status_h.p;
        for (int64_t i = 0; i < nq; ++i)
            if (sh[i]) pending.push_back((uint32_t)i);
        if (pending.empty()) {
            ctx->time_end(slot, st, "ivf_scan");
            return MANS_OK;
        }
        npend = (int64_t)pending.size();
        kc *= 4;
        ctx->proof_retries += npend;
    }
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
    if (e == hipSuccess)
        e = ivf->cent_t.ensure((size_t)ivf->nlist * dim * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess && ivf->nlist > 0) {
        const int64_t cells = ivf->nlist * dim;
        hipLaunchKernelGGL(ivf_transpose, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, st,
                           (const float*)cent->rows.p, ivf->nlist, (int)dim, (float*)ivf->cent_t.p);
        e = hipGetLastError();
    }
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
