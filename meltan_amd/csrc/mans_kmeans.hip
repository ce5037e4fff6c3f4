// k-means on gfx950 with the rules of KMeans.cluster (KMeans.swift:53-257),
// for IVF-flat centroids (IVFFlatSearch.buildPartition,
// IVFFlatSearch.swift:517-551) and IVF-PQ training (_IVFPQIndex.train,
// IVFPQIndex.swift:54-104; ProductQuantizer.train,
// ProductQuantizer.swift:10-85).
//
//  - Assignment (KMeans.swift:196-215): each row's argmin over the
//    centroids of SIMDDistance.distance as a sequential sum, strict < so the
//    first centroid wins ties; one thread per row, the row in registers,
//    the centroid values uniform across the wave.
//  - Stop (KMeans.swift:168-171, 230-233): a problem ends at its first pass
//    that changes no assignment, before any update; the previous
//    assignments start at -1.
//  - Update (KMeans.swift:224-250, single-worker order): each centroid is
//    the Float sum of its rows taken in row order, times 1 / Float(count);
//    an empty cluster keeps its centroid.  One block per centroid collects
//    the matching rows 256 at a time in row order (an ordered compaction)
//    and adds them one dimension per thread, so every (centroid, dimension)
//    sum is the same sequence of additions as the reference's.
//  - Initial centroids: rows 0, s, 2s, ... with s = max(1, n / k), a
//    deterministic stand-in for the k-means++ seeding (KMeans.swift:259-328),
//    which draws from Swift's stdlib RNG.
//
// Several problems that share n, dim and k (the subspaces of a product
// quantizer) run in the same launches, blockIdx.y selecting the problem.
#include <algorithm>
#include <cstring>
#include <vector>

#include "mans_hip.h"
#include "mans_ivf.hpp"
#include "mans_runtime.hpp"

namespace mans {

namespace {

// SIMDDistance.distance with the row in registers (the order of
// simd_distance).
template <int DIM>
__device__ __forceinline__ float reg_distance(const float (&x)[DIM], float xn,
                                              const float* __restrict__ cr, int metric) {
    if (metric == kMetricL2) {
        float s = 0.0f;
#pragma unroll
        for (int d = 0; d < DIM; ++d) {
            const float t = x[d] - cr[d];
            s += t * t;
        }
        return s;
    }
    float dot = 0.0f;
#pragma unroll
    for (int d = 0; d < DIM; ++d) dot += x[d] * cr[d];
    if (metric == kMetricIP) return -dot;
    float nb = 0.0f;
#pragma unroll
    for (int d = 0; d < DIM; ++d) nb += cr[d] * cr[d];
    const float denom = sqrtf(xn) * sqrtf(nb);
    return denom < 1e-10f ? 1.0f : 1.0f - dot / denom;
}

// Assignment pass over problem blockIdx.y (skipped unless active[p]):
// assign[p * n + r] = argmin_c distance(row r, centroid c); changed[p] is
// set when an assignment differs from the previous pass.  DIM 0: any dim,
// the row read from memory per centroid.
template <int DIM>
__global__ __launch_bounds__(256) void kmeans_assign(const float* __restrict__ rows, int64_t n,
                                                     int64_t ld, int dim, int64_t prob_off,
                                                     const float* __restrict__ cent, int k,
                                                     int metric, int32_t* __restrict__ assign,
                                                     const uint32_t* __restrict__ active,
                                                     uint32_t* __restrict__ changed) {
    const int p = blockIdx.y;
    if (!active[p]) return;
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool valid = r < n;
    const float* xr = rows + p * prob_off + (valid ? r : 0) * ld;
    const float* cp = cent + (int64_t)p * k * dim;
    int best = 0;
    float bestd = kFltMax;
    if constexpr (DIM > 0) {
        float x[DIM];
#pragma unroll
        for (int d = 0; d < DIM; ++d) x[d] = xr[d];
        float xn = 0.0f;
        if (metric == kMetricCosine) {
#pragma unroll
            for (int d = 0; d < DIM; ++d) xn += x[d] * x[d];
        }
        for (int c = 0; c < k; ++c) {
            const float dist = reg_distance<DIM>(x, xn, cp + (int64_t)c * DIM, metric);
            if (dist < bestd) {
                bestd = dist;
                best = c;
            }
        }
    } else {
        for (int c = 0; c < k; ++c) {
            const float dist = simd_distance(xr, cp + (int64_t)c * dim, dim, metric);
            if (dist < bestd) {
                bestd = dist;
                best = c;
            }
        }
    }
    bool diff = false;
    if (valid) {
        int32_t* a = assign + (int64_t)p * n + r;
        diff = *a != best;
        *a = best;
    }
    if (__ballot(diff) != 0 && (threadIdx.x & 63) == 0) atomicOr(&changed[p], 1u);
}

// Update pass: block (c, p) recomputes centroid c of problem p (when
// update[p]) as the Float sum of its rows in row order times
// 1 / Float(count).  dynamic LDS: dim floats.
__global__ __launch_bounds__(256) void kmeans_update(const float* __restrict__ rows, int64_t n,
                                                     int64_t ld, int dim, int64_t prob_off,
                                                     const int32_t* __restrict__ assign,
                                                     float* __restrict__ cent, int k,
                                                     const uint32_t* __restrict__ update) {
    extern __shared__ float acc[];
    __shared__ int32_t list[256];
    __shared__ int s_wcnt[4];
    const int c = blockIdx.x, p = blockIdx.y;
    if (!update[p]) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* base = rows + p * prob_off;
    const int32_t* ap = assign + (int64_t)p * n;
    for (int d = tid; d < dim; d += 256) acc[d] = 0.0f;
    int64_t count = 0;
    for (int64_t r0 = 0; r0 < n; r0 += 256) {
        const int64_t r = r0 + tid;
        const bool match = r < n && ap[r] == c;
        const uint64_t bal = __ballot(match);
        if (lane == 0) s_wcnt[wave] = __popcll(bal);
        __syncthreads();
        int off = 0;
        for (int w = 0; w < wave; ++w) off += s_wcnt[w];
        const int nmatch = s_wcnt[0] + s_wcnt[1] + s_wcnt[2] + s_wcnt[3];
        if (match) list[off + __popcll(bal & lanemask_lt())] = (int32_t)tid;
        __syncthreads();
        for (int d = tid; d < dim; d += 256) {
            float a = acc[d];
            for (int j = 0; j < nmatch; ++j) a += base[(r0 + list[j]) * ld + d];
            acc[d] = a;
        }
        count += nmatch;
        __syncthreads();
    }
    if (count == 0) return;
    const float scale = 1.0f / (float)count;
    float* out = cent + ((int64_t)p * k + c) * dim;
    for (int d = tid; d < dim; d += 256) out[d] = acc[d] * scale;
}

// Initial centroids: centroid c of problem p is row (c * stride) % n.
__global__ void kmeans_init(const float* __restrict__ rows, int64_t n, int64_t ld, int dim,
                            int64_t prob_off, int64_t k, int64_t stride, float* __restrict__ cent) {
    const int p = blockIdx.y;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= k * dim) return;
    const int64_t c = t / dim;
    const int d = (int)(t - c * dim);
    cent[(int64_t)p * k * dim + t] = rows[p * prob_off + ((c * stride) % n) * ld + d];
}

// dst[i] = rows[idx[i]], `dim` floats each.
__global__ void gather_rows(const float* __restrict__ rows, int dim, const int64_t* __restrict__ idx,
                            int64_t count, float* __restrict__ dst) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= count * dim) return;
    const int64_t i = t / dim;
    const int d = (int)(t - i * dim);
    dst[t] = rows[idx[i] * dim + d];
}

// res[r] = rows[r] - cent[assign[r]], elementwise in Float
// (IVFPQIndex.swift:366-368).
__global__ void residuals_kernel(const float* __restrict__ rows, int64_t n, int dim,
                                 const float* __restrict__ cent, const int32_t* __restrict__ assign,
                                 float* __restrict__ res) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n * dim) return;
    const int64_t r = t / dim;
    const int d = (int)(t - r * dim);
    res[t] = rows[t] - cent[(int64_t)assign[r] * dim + d];
}

template <int DIM>
void launch_assign(dim3 grid, hipStream_t st, const float* rows, int64_t n, int64_t ld, int dim,
                   int64_t prob_off, const float* cent, int k, int metric, int32_t* assign,
                   const uint32_t* active, uint32_t* changed) {
    hipLaunchKernelGGL(kmeans_assign<DIM>, grid, dim3(256), 0, st, rows, n, ld, dim, prob_off, cent,
                       k, metric, assign, active, changed);
}

}  // namespace

int kmeans_run(mans_ctx* ctx, hipStream_t st, const float* rows, int64_t n, int64_t ld, int dim,
               int64_t prob_off, int nprob, int64_t k, int64_t iters, int metric, float* d_cent,
               int32_t* d_assign) {
    if (n <= 0 || k <= 0 || k > n || nprob <= 0 || nprob > 65535 || k > 0x7FFFFFFF)
        return fail(MANS_SEARCH_FAILED, "k-means: need 1 <= k <= n and 1..65535 problems");
    if ((int64_t)dim * 4 > 160 * 1024) return fail(MANS_SEARCH_FAILED, "k-means: dim too large");
    DevBuf flags;
    hipError_t e = flags.ensure(2 * (size_t)nprob * sizeof(uint32_t), ctx->fail_alloc);
    if (e != hipSuccess) return hip_fail(e, "k-means workspace");
    uint32_t* d_active = (uint32_t*)flags.p;
    uint32_t* d_changed = d_active + nprob;
    const int64_t stride = n / k > 1 ? n / k : 1;
    {
        const int64_t cells = k * dim;
        hipLaunchKernelGGL(kmeans_init, dim3((unsigned)((cells + 255) / 256), (unsigned)nprob),
                           dim3(256), 0, st, rows, n, ld, dim, prob_off, k, stride, d_cent);
        e = hipGetLastError();
    }
    if (e == hipSuccess)
        e = hipMemsetAsync(d_assign, 0xFF, (size_t)nprob * n * sizeof(int32_t), st);
    std::vector<uint32_t> active((size_t)nprob, 1u), changed((size_t)nprob, 0u);
    const dim3 agrid((unsigned)((n + 255) / 256), (unsigned)nprob);
    for (int64_t it = 0; it < iters && e == hipSuccess; ++it) {
        e = hipMemcpyAsync(d_active, active.data(), nprob * sizeof(uint32_t), hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemsetAsync(d_changed, 0, nprob * sizeof(uint32_t), st);
        if (e != hipSuccess) break;
        switch (dim) {
        case 2: launch_assign<2>(agrid, st, rows, n, ld, dim, prob_off, d_cent, (int)k, metric, d_assign, d_active, d_changed); break;
        case 4: launch_assign<4>(agrid, st, rows, n, ld, dim, prob_off, d_cent, (int)k, metric, d_assign, d_active, d_changed); break;
        case 8: launch_assign<8>(agrid, st, rows, n, ld, dim, prob_off, d_cent, (int)k, metric, d_assign, d_active, d_changed); break;
        case 16: launch_assign<16>(agrid, st, rows, n, ld, dim, prob_off, d_cent, (int)k, metric, d_assign, d_active, d_changed); break;
        case 32: launch_assign<32>(agrid, st, rows, n, ld, dim, prob_off, d_cent, (int)k, metric, d_assign, d_active, d_changed); break;
        case 64: launch_assign<64>(agrid, st, rows, n, ld, dim, prob_off, d_cent, (int)k, metric, d_assign, d_active, d_changed); break;
        case 96: launch_assign<96>(agrid, st, rows, n, ld, dim, prob_off, d_cent, (int)k, metric, d_assign, d_active, d_changed); break;
        case 128: launch_assign<128>(agrid, st, rows, n, ld, dim, prob_off, d_cent, (int)k, metric, d_assign, d_active, d_changed); break;
        default: launch_assign<0>(agrid, st, rows, n, ld, dim, prob_off, d_cent, (int)k, metric, d_assign, d_active, d_changed);
        }
        e = hipGetLastError();
        if (e == hipSuccess)
            e = hipMemcpyAsync(changed.data(), d_changed, nprob * sizeof(uint32_t), hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) break;
        bool any = false;
        for (int p = 0; p < nprob; ++p) {
            if (active[p] && !changed[p]) active[p] = 0;  // converged: no update
            any = any || active[p];
        }
        if (!any) break;
        e = hipMemcpyAsync(d_active, active.data(), nprob * sizeof(uint32_t), hipMemcpyHostToDevice, st);
        if (e == hipSuccess) {
            hipLaunchKernelGGL(kmeans_update, dim3((unsigned)k, (unsigned)nprob), dim3(256),
                               sizeof(float) * (size_t)dim, st, rows, n, ld, dim, prob_off,
                               (const int32_t*)d_assign, d_cent, (int)k, (const uint32_t*)d_active);
            e = hipGetLastError();
        }
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? MANS_OK : hip_fail(e, "k-means");
}

}  // namespace mans

using namespace mans;

extern "C" {

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
    DevBuf d_cent, d_assign;
    hipError_t e = d_cent.ensure((size_t)k * dim * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = d_assign.ensure((size_t)n * sizeof(int32_t), ctx->fail_alloc);
    if (e != hipSuccess) return hip_fail(e, "k-means workspace");
    int rc = kmeans_run(ctx, st, (const float*)corpus->rows.p, n, dim, (int)dim, 0, 1, k, iters,
                        (int)metric, (float*)d_cent.p, (int32_t*)d_assign.p);
    if (rc != MANS_OK) return rc;
    e = hipMemcpyAsync(out_centroids, d_cent.p, (size_t)k * dim * sizeof(float), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? MANS_OK : hip_fail(e, "k-means download");
}

int mans_ivf_flat_train(mans_ctx* ctx, const mans_corpus* corpus, int64_t nlist, uint32_t metric,
                        float* out_centroids, int64_t* out_nlist) {
    if (!ctx || !corpus || !out_centroids)
        return fail(MANS_SEARCH_FAILED, "mans_ivf_flat_train: NULL argument");
    if (metric > 2) return fail(MANS_SEARCH_FAILED, "IVF-flat does not support this metric");
    const int64_t n = corpus->n, dim = corpus->dim;
    if (n < 1) return fail(MANS_SEARCH_FAILED, "IVF-flat build requires count > 0");
    // The sample of IVFFlatSearch.swift:528-543.
    const int64_t lists = std::min<int64_t>(std::max<int64_t>(1, nlist), n);
    const int64_t count =
        std::min<int64_t>(n, std::max<int64_t>(lists, std::min<int64_t>(4096, std::max(lists * 16, lists))));
    const int64_t stride = std::max<int64_t>(1, n / count);
    std::vector<int64_t> idx;
    idx.reserve((size_t)count);
    for (int64_t cursor = 0; (int64_t)idx.size() < count && cursor < n; cursor += stride)
        idx.push_back(cursor);
    while ((int64_t)idx.size() < count) idx.push_back((int64_t)idx.size() % n);
    DeviceGuard dg(ctx->device);
    SlotLease lease(ctx);
    if (!lease.slot) return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    hipStream_t st = lease.slot->stream;
    DevBuf d_idx, d_sample, d_cent, d_assign;
    hipError_t e = d_idx.ensure((size_t)count * sizeof(int64_t), ctx->fail_alloc);
    if (e == hipSuccess) e = d_sample.ensure((size_t)count * dim * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = d_cent.ensure((size_t)lists * dim * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = d_assign.ensure((size_t)count * sizeof(int32_t), ctx->fail_alloc);
    if (e == hipSuccess)
        e = hipMemcpyAsync(d_idx.p, idx.data(), (size_t)count * sizeof(int64_t), hipMemcpyHostToDevice, st);
    if (e == hipSuccess) {
        const int64_t cells = count * dim;
        hipLaunchKernelGGL(gather_rows, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, st,
                           (const float*)corpus->rows.p, (int)dim, (const int64_t*)d_idx.p, count,
                           (float*)d_sample.p);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return hip_fail(e, "IVF-flat training sample");
    int rc = kmeans_run(ctx, st, (const float*)d_sample.p, count, dim, (int)dim, 0, 1, lists, 8,
                        (int)metric, (float*)d_cent.p, (int32_t*)d_assign.p);
    if (rc != MANS_OK) return rc;
    e = hipMemcpyAsync(out_centroids, d_cent.p, (size_t)lists * dim * sizeof(float), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "IVF-flat centroids download");
    if (out_nlist) *out_nlist = lists;
    return MANS_OK;
}

int mans_ivfpq_train(mans_ctx* ctx, const mans_corpus* train, int64_t nlist, int64_t m, int64_t iters,
                     uint32_t metric, float* out_coarse, float* out_codebooks) {
    if (!ctx || !train || !out_coarse || !out_codebooks)
        return fail(MANS_SEARCH_FAILED, "mans_ivfpq_train: NULL argument");
    const int64_t n = train->n, dim = train->dim;
    if (metric > 2) return fail(MANS_SEARCH_FAILED, "IVF-PQ does not support this metric");
    if (n < 256) return fail(MANS_SEARCH_FAILED, "Need at least 256 vectors for PQ training");
    if (nlist < 1 || nlist > n)
        return fail(MANS_SEARCH_FAILED, "Need at least nlist vectors for the coarse quantizer");
    if (m < 1 || dim % m != 0)
        return fail(MANS_SEARCH_FAILED, "Vector dimension must be divisible by numSubspaces");
    const int64_t dsub = dim / m;
    iters = std::max<int64_t>(1, iters);  // IVFPQConfiguration clamps trainingIterations to >= 1
    DeviceGuard dg(ctx->device);
    SlotLease lease(ctx);
    if (!lease.slot) return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    hipStream_t st = lease.slot->stream;
    DevBuf d_coarse, d_assign, d_res, d_books, d_sub_assign;
    hipError_t e = d_coarse.ensure((size_t)nlist * dim * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = d_assign.ensure((size_t)n * sizeof(int32_t), ctx->fail_alloc);
    if (e == hipSuccess) e = d_res.ensure((size_t)n * dim * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = d_books.ensure((size_t)m * 256 * dsub * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = d_sub_assign.ensure((size_t)m * n * sizeof(int32_t), ctx->fail_alloc);
    if (e != hipSuccess) return hip_fail(e, "IVF-PQ training workspace");
    const float* rows = (const float*)train->rows.p;
    int rc = kmeans_run(ctx, st, rows, n, dim, (int)dim, 0, 1, nlist, iters, (int)metric,
                        (float*)d_coarse.p, (int32_t*)d_assign.p);
    if (rc != MANS_OK) return rc;
    {
        const int64_t cells = n * dim;
        hipLaunchKernelGGL(residuals_kernel, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, st,
                           rows, n, (int)dim, (const float*)d_coarse.p, (const int32_t*)d_assign.p,
                           (float*)d_res.p);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return hip_fail(e, "IVF-PQ residuals");
    rc = kmeans_run(ctx, st, (const float*)d_res.p, n, dim, (int)dsub, dsub, (int)m, 256, iters,
                    kMetricL2, (float*)d_books.p, (int32_t*)d_sub_assign.p);
    if (rc != MANS_OK) return rc;
    e = hipMemcpyAsync(out_coarse, d_coarse.p, (size_t)nlist * dim * sizeof(float), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(out_codebooks, d_books.p, (size_t)m * 256 * dsub * sizeof(float),
                           hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? MANS_OK : hip_fail(e, "IVF-PQ training download");
}

}  // extern "C"
