// Kernels shared by the IVF-flat and IVF-PQ files: the per-query plan of
// probed segments and the work-item map over them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mans_device.hpp"

struct mans_ctx;

namespace mans {

// One wave per query of the launch: its probed lists' packed starts and
// concatenated starts, its candidate count and its number of work items.
__global__ __launch_bounds__(256) void ivf_plan(const uint32_t* __restrict__ probes, int np,
                                                const uint32_t* __restrict__ qidx, int64_t nq,
                                                const int64_t* __restrict__ offsets, int64_t chunk,
                                                int64_t* __restrict__ seg, int64_t* __restrict__ total,
                                                int32_t* __restrict__ nitems);

// One block: exclusive scan of the per-query item counts, then the item ->
// query map.  item_off[nq] holds the number of items.
__global__ __launch_bounds__(1024) void ivf_items(const int32_t* __restrict__ nitems, int64_t nq,
                                                   int32_t* __restrict__ item_off,
                                                   int32_t* __restrict__ item_q);

// SIMDDistance.distance (SIMDDistance.swift:17-80) as sequential sums.
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

// k-means (KMeans.cluster, KMeans.swift:53-257) for `nprob` independent
// problems that share n, dim and k -- the subspaces of a product quantizer,
// or one problem: problem p's row r is the dim floats at
// rows + p * prob_off + r * ld.  d_cent receives nprob x k x dim centroids
// and d_assign nprob x n assignments of the last assignment pass.  Each
// problem stops at its first pass that changes no assignment.
int kmeans_run(mans_ctx* ctx, hipStream_t st, const float* rows, int64_t n, int64_t ld, int dim,
               int64_t prob_off, int nprob, int64_t k, int64_t iters, int metric, float* d_cent,
               int32_t* d_assign);

}  // namespace mans
