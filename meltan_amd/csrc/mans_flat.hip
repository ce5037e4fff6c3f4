// Exact flat scan on gfx950: FlatGPUSearch.batchSearch / ParallelFlatScan.search
// (FlatGPUSearch.swift:103-181, ParallelFlatScan.swift:96-155) in one launch.
//
//  1. Streaming pass (flat_scan_f4): 16 lanes per row, 128-bit loads, fused
//     multiply-adds in any order, a 16-lane DPP reduction, then a provable
//     lower bound on the exact distance (the "key").  Each wave keeps its
//     best kc keys in LDS (WaveTopK); wave 0 folds the block's 4 lists and
//     writes kc slots.
//  2. Merge: the last block of each group of kGroupBlocks blocks to arrive
//     (per-query counters, one atomic per block) merges the group's lists;
//     the last group to arrive merges the group lists.  That block then
//     recomputes the kc candidates' distances in the scalar order of
//     dots.c:40-47 with the host formulas (bit-identical to the CPU path),
//     sorts them by (distance, id) and writes k.  The query passes the proof
//     when the kc-th key is >= the k-th exact distance: every row left out
//     has a key >= the kc-th key, so an exact distance >= every row returned.
//  3. The host re-runs queries that fail the proof with a larger kc, and
//     past the largest kc with flat_scan_rows (exact distances as keys).
//
// The lower bound: any summation order of d products has error at most
// gamma_d * sum|q_i v_i| <= gamma_d * |q| |v|, gamma_d = d u / (1 - d u),
// u = 2^-24 (Higham, Accuracy and Stability of Numerical Algorithms, 3.1).
// Both the fast dot and the sequential dot obey it, so their difference is
// at most twice that; the per-metric constants also absorb the rounding of
// the finalising operations and of the fast query norm.
#include <algorithm>
#include <cstdlib>

#include "mans_device.hpp"
#include "mans_internal.hpp"

namespace mans {

struct BoundCoef {
    float eps_cos;  // absolute slack on cosine distance
    float c_l2;     // slack = c_l2 * (qn + vn + 2 sqrt(qn vn))
    float c_ip;     // slack = c_ip * sqrt(qn vn)
};

__device__ __forceinline__ float lower_key(float f, float qn, float vn, int metric,
                                           const BoundCoef& bc) {
    if (metric == kMetricIP) {
        float s = sqrtf(qn * vn);
        return -f - s * bc.c_ip;
    }
    if (metric == kMetricL2) {
        float s = sqrtf(qn * vn);
        float dd = qn - 2.0f * f + vn;
        dd = dd > 0.0f ? dd : 0.0f;
        return dd - (qn + vn + 2.0f * s) * bc.c_l2;
    }
    if (vn == 0.0f) return 1.0f - bc.eps_cos;  // both paths give exactly 1
    float s = sqrtf(qn * vn);
    if (s < 1.001e-10f) return -1.0f;  // near the 1e-10 branch of the formula
    return (1.0f - f / s) - bc.eps_cos;
}

// Per-launch outputs and merge bookkeeping (indexed by blockIdx.y).
struct FlatArgs {
    uint64_t* cand;      // [nq][nblk][kc]  block lists
    uint64_t* gcand;     // [nq][ngroups][kc]  group lists
    uint32_t* counters;  // [nq][ngroups + 1], zero between launches
    float* out_dist;     // [nq_total][k_stride], indexed by the query id
    uint32_t* out_ids;
    uint8_t* status;     // [nq]: 0 proven, 1 re-run with a larger kc
    int k;               // results per query (<= kc)
    int k_stride;
    int group_blocks;
    int ngroups;
};

// Lists passed between blocks are written and read with device-scope
// atomic stores/loads: they go to the device coherence point, which each
// XCD's L2 does not hide.  This avoids device-scope fences, which on a
// multi-XCD part write back and invalidate the whole L2 of the XCD.
__device__ __forceinline__ void store_shared_slot(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_shared_slot(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// All threads call this after their store_shared_slot writes; returns true
// (in every thread) in the block that arrives last at `counter` (expected
// arrivals: `total`).  The workgroup release waits until this block's
// device-scope stores are complete, the barrier makes that true for every
// wave, and only then is the arrival counted, so the last block to arrive
// finds every list at the coherence point.
__device__ __forceinline__ bool block_arrive_last(uint32_t* counter, uint32_t total) {
    __shared__ int last;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               total - 1;
    __syncthreads();
    return last;
}

// Block-wide selection of the kc smallest over `nl` lists of kc slots in
// global memory; result sorted in lds[0, kc) (wave 0's buffer).
__device__ __forceinline__ void block_select_lists(const uint64_t* src, int nl, uint64_t* lds, int cap, int kc,
                                   WaveTopK& sel) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, nt = blockDim.x;
    const int nw = nt >> 6;
    sel.init(lds + wave * cap, cap, kc);
    const int64_t total = (int64_t)nl * kc;
    constexpr int kAhead = 4;
    for (int64_t base = (int64_t)wave * 64; base < total; base += (int64_t)nt * kAhead) {
        uint64_t v[kAhead];
#pragma unroll
        for (int u = 0; u < kAhead; ++u) {
            int64_t i = base + (int64_t)u * nt + lane;
            v[u] = i < total ? load_shared_slot(src + i) : kEmptySlot;
        }
#pragma unroll
        for (int u = 0; u < kAhead; ++u) {
            bool ok = v[u] != kEmptySlot;
            sel.offer(ok, ok ? slot_key(v[u]) : 0.0f, slot_id(v[u]));
        }
    }
    sel.finish();
    __syncthreads();
    if (wave == 0) {
        for (int w = 1; w < nw; ++w) sel.offer_slots(lds + w * cap, kc);
        sel.finish();
    }
    __syncthreads();
}

// Wave 0 folds waves 1..3 of the block into its selector (block's kc best).
__device__ __forceinline__ void block_fold(WaveTopK& sel, uint64_t* lds, int cap) {
    __syncthreads();
    if ((threadIdx.x >> 6) == 0) {
        const int nw = blockDim.x >> 6;
        for (int w = 1; w < nw; ++w) sel.offer_slots(lds + w * cap, sel.kc);
        sel.finish();
    }
    __syncthreads();
}

// Sequential dot in the order of dots.c:40-47 for a row held by a 16-lane
// DPP row: lane lr holds float4 chunks lr + 16 j (j < NCH) of the row and
// of the query.  The running sum visits the chunks in index order, each
// chunk's four products in order, and moves from the lane owning chunk c to
// the lane owning chunk c + 1.  Every lane of the group returns the total.
template <int NCH>
__device__ __forceinline__ float chain_dot(const f4v* a, const f4v* b, int dim4) {
    const int lane = __lane_id(), lr = lane & 15, row0 = lane & ~15;
    float acc = 0.0f;
    int last = 0;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
#pragma unroll
        for (int o = 0; o < 16; ++o) {
            const int c = o + 16 * j;
            if (c < dim4) {
                float t = acc + a[j].x * b[j].x;
                t = t + a[j].y * b[j].y;
                t = t + a[j].z * b[j].z;
                t = t + a[j].w * b[j].w;
                acc = lr == o ? t : acc;
                last = o;
                // row_ror:1 -- lane i takes lane i - 1 of its 16-lane row
                if (c + 1 < dim4)
                    acc = __int_as_float(
                        __builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x121, 0xF, 0xF, false));
            }
        }
    }
    return __shfl(acc, row0 | last);
}

// The last block of a query: exact rescore of the kc candidates held in
// lds[0, kc), sort, outputs and proof status.  qv: the query chunks.
template <int NCH>
__device__ __forceinline__ void final_rescore_f4(const f4v* qv, const float* __restrict__ rows,
                                 const float* __restrict__ norms, int64_t n, int dim, int metric,
                                 uint32_t q, uint64_t* lds, int kc, const FlatArgs& fa) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = lane >> 4, lr = lane & 15, dim4 = dim >> 2;
    __shared__ int ncand_sh;
    uint64_t* top = lds;
    uint64_t* res = lds + kc;  // kc slots (cap >= 2 kc)
    if (tid == 0) {
        int c = 0;
        while (c < kc && top[c] != kEmptySlot) ++c;
        ncand_sh = c;
    }
    __syncthreads();
    const int ncand = ncand_sh;
    for (int i = tid; i < kc; i += blockDim.x) res[i] = kEmptySlot;
    __syncthreads();
    // One candidate row per 16-lane group per pass.  (Interleaving several
    // chains per group would overlap their latencies but raises the kernel's
    // register count, which costs the streaming pass more occupancy.)
    const float qn = metric == kMetricIP ? 0.0f : chain_dot<NCH>(qv, qv, dim4);
    const int groups = (blockDim.x >> 4);
    for (int base = 0; base < ncand; base += groups) {
        const int s0 = base + wave * 4 + grp;
        const bool v0 = s0 < ncand;
        const uint32_t id0 = v0 ? slot_id(top[s0]) : 0u;
        f4v a0[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            int idx = lr + 16 * c;
            a0[c] = (v0 && idx < dim4) ? *reinterpret_cast<const f4v*>(rows + (int64_t)id0 * dim + 4 * idx)
                                       : f4v{0.f, 0.f, 0.f, 0.f};
        }
        const float dot0 = chain_dot<NCH>(a0, qv, dim4);
        if (lr == 0 && v0)
            res[s0] = pack_slot(
                host_distance(dot0, qn, metric == kMetricIP ? 0.0f : norms[id0], metric), id0);
    }
    __syncthreads();
    if (wave == 0) wave_bitonic_sort(res, kc);
    __syncthreads();
    const int kout = fa.k < ncand ? fa.k : ncand;
    for (int i = tid; i < fa.k_stride; i += blockDim.x) {
        float dv = kFltMax;
        uint32_t id = kEmptyId;
        if (i < kout) {
            id = slot_id(res[i]);
            dv = slot_key(res[i]);
        }
        fa.out_dist[(int64_t)q * fa.k_stride + i] = dv;
        fa.out_ids[(int64_t)q * fa.k_stride + i] = id;
    }
    if (tid == 0) {
        const float cutoff = ncand > 0 ? slot_key(top[ncand - 1]) : 0.0f;
        bool all_rows = (int64_t)ncand >= n;
        bool ok = all_rows || (kout > 0 && cutoff >= slot_key(res[kout - 1]));
        fa.status[blockIdx.y] = ok ? 0 : 1;
    }
}

// Exact-key final step: the candidates' keys already are their exact
// distances, so the sorted kc list is the answer (the proof holds).
__device__ __forceinline__ void final_exact_keys(uint64_t* lds, int kc, int64_t n, uint32_t q, const FlatArgs& fa) {
    const int tid = threadIdx.x;
    __shared__ int ncand_sh;
    if (tid == 0) {
        int c = 0;
        while (c < kc && lds[c] != kEmptySlot) ++c;
        ncand_sh = c;
    }
    __syncthreads();
    const int ncand = ncand_sh;
    const int kout = fa.k < ncand ? fa.k : ncand;
    for (int i = tid; i < fa.k_stride; i += blockDim.x) {
        float dv = kFltMax;
        uint32_t id = kEmptyId;
        if (i < kout) {
            id = slot_id(lds[i]);
            dv = slot_key(lds[i]);
        }
        fa.out_dist[(int64_t)q * fa.k_stride + i] = dv;
        fa.out_ids[(int64_t)q * fa.k_stride + i] = id;
    }
    if (tid == 0) fa.status[blockIdx.y] = 0;
}

// Steps 2: block list out, group merge, query merge.  Returns true in the
// block that holds the query's kc best in lds[0, kc) afterwards.
__device__ __forceinline__ bool flat_block_epilogue(WaveTopK& sel, uint64_t* lds, int cap, int kc,
                                    const FlatArgs& fa) {
    block_fold(sel, lds, cap);
    const int tid = threadIdx.x;
    const int nblk = gridDim.x;
    const int g = blockIdx.x / fa.group_blocks;
    const int gsize = min(fa.group_blocks, nblk - g * fa.group_blocks);
    uint64_t* cand_q = fa.cand + (int64_t)blockIdx.y * nblk * kc;
    uint64_t* gcand_q = fa.gcand + (int64_t)blockIdx.y * fa.ngroups * kc;
    uint32_t* cnt_q = fa.counters + (int64_t)blockIdx.y * (fa.ngroups + 1);
    if (tid < 64)
        for (int i = tid; i < kc; i += 64)
            store_shared_slot(&cand_q[(int64_t)blockIdx.x * kc + i],
                              i < sel.count ? sel.buf[i] : kEmptySlot);
    if (!block_arrive_last(&cnt_q[g], (uint32_t)gsize)) return false;
    if (tid == 0)  // every block of the group has arrived
        __hip_atomic_store(&cnt_q[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    block_select_lists(cand_q + (int64_t)g * fa.group_blocks * kc, gsize, lds, cap, kc, sel);
    if (tid < 64)
        for (int i = tid; i < kc; i += 64)
            store_shared_slot(&gcand_q[(int64_t)g * kc + i], i < sel.count ? sel.buf[i] : kEmptySlot);
    if (!block_arrive_last(&cnt_q[fa.ngroups], (uint32_t)fa.ngroups)) return false;
    if (tid == 0)
        __hip_atomic_store(&cnt_q[fa.ngroups], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    block_select_lists(gcand_q, fa.ngroups, lds, cap, kc, sel);
    return true;
}

// grid: (nblk, nq_launch); block 256 = 4 waves; dynamic LDS: 4 * cap slots.
template <int NCH>
__global__ __launch_bounds__(256) void flat_scan_f4(
    const float* __restrict__ rows, const float* __restrict__ norms, int64_t n, int dim,
    const float* __restrict__ queries, const uint32_t* __restrict__ qidx, int metric,
    BoundCoef bc, int kc, int cap, int64_t rows_per_block, FlatArgs fa) {
    extern __shared__ uint64_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = lane >> 4, lr = lane & 15;
    const uint32_t q = qidx ? qidx[blockIdx.y] : blockIdx.y;
    const int dim4 = dim >> 2;
    const float* qp = queries + (int64_t)q * dim;

    f4v qv[NCH];
    float qsq = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        int idx = lr + 16 * c;
        qv[c] = idx < dim4 ? *reinterpret_cast<const f4v*>(qp + 4 * idx) : f4v{0.f, 0.f, 0.f, 0.f};
        qsq = fmaf(qv[c].x, qv[c].x, qsq);
        qsq = fmaf(qv[c].y, qv[c].y, qsq);
        qsq = fmaf(qv[c].z, qv[c].z, qsq);
        qsq = fmaf(qv[c].w, qv[c].w, qsq);
    }
    const float qn = row16_sum(qsq);

    WaveTopK sel;
    sel.init(lds + wave * cap, cap, kc);

    const int64_t start = (int64_t)blockIdx.x * rows_per_block;
    const int64_t end = start + rows_per_block < n ? start + rows_per_block : n;
    for (int64_t base = start; base < end; base += 32) {
        const int64_t r0 = base + wave * 4 + grp;
        const int64_t r1 = r0 + 16;
        const bool v0 = r0 < end, v1 = r1 < end;
        const float* p0 = rows + r0 * dim;
        const float* p1 = rows + r1 * dim;
        f4v a[NCH], b[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            int idx = lr + 16 * c;
            bool in = idx < dim4;
            a[c] = (v0 && in) ? load_stream(p0 + 4 * idx) : f4v{0.f, 0.f, 0.f, 0.f};
            b[c] = (v1 && in) ? load_stream(p1 + 4 * idx) : f4v{0.f, 0.f, 0.f, 0.f};
        }
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            s0 = fmaf(a[c].x, qv[c].x, s0);
            s0 = fmaf(a[c].y, qv[c].y, s0);
            s0 = fmaf(a[c].z, qv[c].z, s0);
            s0 = fmaf(a[c].w, qv[c].w, s0);
            s1 = fmaf(b[c].x, qv[c].x, s1);
            s1 = fmaf(b[c].y, qv[c].y, s1);
            s1 = fmaf(b[c].z, qv[c].z, s1);
            s1 = fmaf(b[c].w, qv[c].w, s1);
        }
        s0 = row16_sum(s0);
        s1 = row16_sum(s1);
        float k0 = 0.0f, k1 = 0.0f;
        if (lr == 0) {
            if (v0) k0 = lower_key(s0, qn, norms[r0], metric, bc);
            if (v1) k1 = lower_key(s1, qn, norms[r1], metric, bc);
        }
        sel.offer(lr == 0 && v0, k0, (uint32_t)r0);
        sel.offer(lr == 0 && v1, k1, (uint32_t)r1);
    }
    sel.finish();
    if (!flat_block_epilogue(sel, lds, cap, kc, fa)) return;
    final_rescore_f4<NCH>(qv, rows, norms, n, dim, metric, q, lds, kc, fa);
}

// Exact-key variant: one thread per row, distances in the scalar dots.c
// order with the host formulas.  Used for dims the float4 path does not
// cover, for unaligned queries and as the terminal round of the proof loop.
// dynamic LDS: 4 * cap slots + dim floats.
__global__ __launch_bounds__(256) void flat_scan_rows(
    const float* __restrict__ rows, const float* __restrict__ norms, int64_t n, int dim,
    const float* __restrict__ queries, const uint32_t* __restrict__ qidx, int metric, int kc,
    int cap, int64_t rows_per_block, FlatArgs fa) {
    extern __shared__ uint64_t lds[];
    float* qs = reinterpret_cast<float*>(lds + 4 * cap);
    __shared__ float qn_sh;
    const int tid = threadIdx.x, wave = tid >> 6;
    const uint32_t q = qidx ? qidx[blockIdx.y] : blockIdx.y;
    const float* qp = queries + (int64_t)q * dim;
    for (int d = tid; d < dim; d += 256) qs[d] = qp[d];
    __syncthreads();
    if (tid == 0) qn_sh = (metric == kMetricIP) ? 0.0f : exact_dot(qs, qs, dim);
    __syncthreads();
    const float qn = qn_sh;

    WaveTopK sel;
    sel.init(lds + wave * cap, cap, kc);
    const int64_t start = (int64_t)blockIdx.x * rows_per_block;
    const int64_t end = start + rows_per_block < n ? start + rows_per_block : n;
    for (int64_t base = start; base < end; base += 256) {
        const int64_t r = base + tid;
        const bool v = r < end;
        float key = 0.0f;
        if (v) {
            float dot = exact_dot(rows + r * dim, qs, dim);
            key = host_distance(dot, qn, metric == kMetricIP ? 0.0f : norms[r], metric);
        }
        sel.offer(v, key, (uint32_t)r);
    }
    sel.finish();
    if (!flat_block_epilogue(sel, lds, cap, kc, fa)) return;
    final_exact_keys(lds, kc, n, q, fa);
}

// Squared norms in the scalar order of dots.c:40-47, one thread per row;
// rows are staged through LDS in 32-column tiles so global reads coalesce.
__global__ __launch_bounds__(256) void row_norms_kernel(const float* __restrict__ rows, int64_t n,
                                                        int dim, float* __restrict__ out) {
    __shared__ float tile[256 * 33];
    const int tid = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * 256;
    float acc = 0.0f;
    for (int c0 = 0; c0 < dim; c0 += 32) {
        const int width = dim - c0 < 32 ? dim - c0 : 32;
        for (int i = tid; i < 256 * 32; i += 256) {
            int r = i >> 5, c = i & 31;
            int64_t gr = row0 + r;
            tile[r * 33 + c] = (gr < n && c < width) ? rows[gr * dim + c0 + c] : 0.0f;
        }
        __syncthreads();
        for (int c = 0; c < width; ++c) {
            float v = tile[tid * 33 + c];
            acc = acc + v * v;
        }
        __syncthreads();
    }
    if (row0 + tid < n) out[row0 + tid] = acc;
}

// ---------------------------------------------------------------------------

static BoundCoef make_bounds(int dim) {
    const double u = 1.0 / 16777216.0;
    const double g = (double)dim * u / (1.0 - (double)dim * u);
    BoundCoef bc;
    bc.eps_cos = (float)((3.0 * g * (1.0 + 3.0 * g) + 16.0 * u) * 1.0001);
    bc.c_l2 = (float)((4.0 * g + 8.0 * u) * (1.0 + 4.0 * g) * 1.0001);
    bc.c_ip = (float)((2.0 * g + 4.0 * u) * (1.0 + 4.0 * g) * 1.0001);
    return bc;
}

int flat_nch_for_dim(int dim) {
    if (dim % 4 != 0) return 0;
    int dim4 = dim / 4;
    static const int options[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32};
    for (int o : options)
        if (16 * o >= dim4) return o;
    return 0;
}

static int pow2_at_least(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

int flat_cap_for(int kc) { return pow2_at_least(kc + 64 > 2 * kc ? kc + 64 : 2 * kc); }

hipError_t launch_row_norms(const float* rows, int64_t n, int dim, float* out, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(row_norms_kernel, dim3((unsigned)blocks), dim3(256), 0, s, rows, n, dim, out);
    return hipGetLastError();
}

FlatPlan plan_flat(int64_t n, int64_t nq, int kc) {
    FlatPlan p;
    p.kc = kc;
    p.cap = flat_cap_for(kc);
    static const int64_t target = [] {
        const char* e = std::getenv("MANS_FLAT_BLOCKS");
        return e ? std::max<int64_t>(1, std::atoll(e)) : (int64_t)1024;
    }();
    int64_t want_blocks = (target + nq - 1) / nq;
    int64_t max_blocks = (n + 63) / 64;
    if (want_blocks > max_blocks) want_blocks = max_blocks;
    if (want_blocks < 1) want_blocks = 1;
    int64_t rpb = (n + want_blocks - 1) / want_blocks;
    rpb = (rpb + 63) / 64 * 64;  // whole 32-row steps for the 4 waves
    p.rows_per_block = rpb;
    p.nblk = (int)((n + rpb - 1) / rpb);
    p.group_blocks = kGroupBlocks;
    p.ngroups = (p.nblk + kGroupBlocks - 1) / kGroupBlocks;
    return p;
}

template <int NCH>
static void launch_f4(const FlatPlan& p, const float* rows, const float* norms, int64_t n, int dim,
                      const float* queries, const uint32_t* qidx, int64_t nq, int metric,
                      const BoundCoef& bc, const FlatArgs& fa, hipStream_t s) {
    size_t shmem = sizeof(uint64_t) * 4 * (size_t)p.cap;
    hipLaunchKernelGGL(flat_scan_f4<NCH>, dim3(p.nblk, (unsigned)nq), dim3(256), shmem, s, rows,
                       norms, n, dim, queries, qidx, metric, bc, p.kc, p.cap, p.rows_per_block, fa);
}

hipError_t launch_flat_search(const FlatPlan& p, bool exact, const float* rows, const float* norms,
                              int64_t n, int dim, const float* queries, const uint32_t* qidx,
                              int64_t nq, int metric, const FlatBuffers& b, int k, int k_stride,
                              hipStream_t s) {
    FlatArgs fa;
    fa.cand = b.cand;
    fa.gcand = b.gcand;
    fa.counters = b.counters;
    fa.out_dist = b.out_dist;
    fa.out_ids = b.out_ids;
    fa.status = b.status;
    fa.k = k;
    fa.k_stride = k_stride;
    fa.group_blocks = p.group_blocks;
    fa.ngroups = p.ngroups;
    int nch = exact ? 0 : flat_nch_for_dim(dim);
    BoundCoef bc = make_bounds(dim);
    switch (nch) {
    case 1: launch_f4<1>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, fa, s); break;
    case 2: launch_f4<2>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, fa, s); break;
    case 3: launch_f4<3>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, fa, s); break;
    case 4: launch_f4<4>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, fa, s); break;
    case 6: launch_f4<6>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, fa, s); break;
    case 8: launch_f4<8>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, fa, s); break;
    case 12: launch_f4<12>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, fa, s); break;
    case 16: launch_f4<16>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, fa, s); break;
    case 24: launch_f4<24>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, fa, s); break;
    case 32: launch_f4<32>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, fa, s); break;
    default: {
        size_t shmem = sizeof(uint64_t) * 4 * (size_t)p.cap + sizeof(float) * (size_t)dim;
        hipLaunchKernelGGL(flat_scan_rows, dim3(p.nblk, (unsigned)nq), dim3(256), shmem, s, rows,
                           norms, n, dim, queries, qidx, metric, p.kc, p.cap, p.rows_per_block, fa);
    }
    }
    return hipGetLastError();
}

}  // namespace mans
