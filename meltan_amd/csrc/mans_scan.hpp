// Device building blocks shared by the scan kernels (flat fp32, int8):
// lower-bound keys, the cross-block list merge, the exact rescore in the
// dots.c order and the proof status.
#pragma once

#include "mans_device.hpp"
#include "mans_internal.hpp"

namespace mans {

struct BoundCoef {
    float eps_cos;  // absolute slack on cosine distance
    float c_l2;     // slack = c_l2 * (qn + vn + 2 sqrt(qn vn))
    float c_ip;     // slack = c_ip * sqrt(qn vn)
};

// Slack coefficients for dimension `dim`; u: the unit roundoff the fast dot
// products are assumed to meet (gamma_d = d u / (1 - d u)).
inline BoundCoef make_bounds(int dim, double u = 1.0 / 16777216.0) {
    const double g = (double)dim * u / (1.0 - (double)dim * u);
    BoundCoef bc;
    bc.eps_cos = (float)((3.0 * g * (1.0 + 3.0 * g) + 16.0 * u) * 1.0001);
    bc.c_l2 = (float)((4.0 * g + 8.0 * u) * (1.0 + 4.0 * g) * 1.0001);
    bc.c_ip = (float)((2.0 * g + 4.0 * u) * (1.0 + 4.0 * g) * 1.0001);
    return bc;
}

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

// Block-wide selection of the kc smallest of `total` slots in global memory
// (lists written by other blocks); result sorted in lds[0, kc) (wave 0's
// buffer).
__device__ __forceinline__ void block_select_lists(const uint64_t* src, int64_t total, uint64_t* lds,
                                                   int cap, int kc, WaveTopK& sel) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, nt = blockDim.x;
    const int nw = nt >> 6;
    sel.init(lds + wave * cap, cap, kc);
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

// Proof applied by final_rescore_f4 to the rescored candidates.
enum ProofMode : int {
    kProofFlat = 0,    // cutoff key >= k-th exact distance
    kProofMargin = 1,  // BoundedExactScan.swift:108-113: cutoff >= tau + max(1e-7, |tau| 1e-6)
    kProofNone = 2,    // fixed budget: no proof (status 0)
};

// The last block of a query: exact rescore of the kc candidates held in
// lds[0, kc), sort by (distance, id), outputs and proof status.  qv: the
// query chunks.  lds must hold kc + pow2(kc) slots (cap >= 2 kc, 4 caps).
// Candidate ids index `rows`; idmap (nullable) maps them to the ids that are
// reported and that order ties.  n: the number of rows the query could see.
// status_idx: the status slot (default: blockIdx.y).
template <int NCH>
__device__ __forceinline__ void final_rescore_f4(const f4v* qv, const float* __restrict__ rows,
                                 const float* __restrict__ norms, int64_t n, int dim, int metric,
                                 uint32_t q, uint64_t* lds, int kc, const FlatArgs& fa,
                                 float list_cut = kFltMax, int proof = kProofFlat,
                                 const uint32_t* idmap = nullptr, int status_idx = -1) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = lane >> 4, lr = lane & 15, dim4 = dim >> 2;
    __shared__ int ncand_sh;
    uint64_t* top = lds;
    uint64_t* res = lds + kc;
    int sort_n = 32;
    while (sort_n < kc) sort_n <<= 1;
    if (tid == 0) {
        int c = 0;
        while (c < kc && top[c] != kEmptySlot) ++c;
        ncand_sh = c;
    }
    __syncthreads();
    const int ncand = ncand_sh;
    for (int i = tid; i < sort_n; i += blockDim.x) res[i] = kEmptySlot;
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
                host_distance(dot0, qn, metric == kMetricIP ? 0.0f : norms[id0], metric),
                idmap ? idmap[id0] : id0);
    }
    __syncthreads();
    if (wave == 0) wave_bitonic_sort(res, sort_n);
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
        // list_cut: rows that bounded lists turned away have keys >= it.
        float cutoff = ncand > 0 ? slot_key(top[ncand - 1]) : 0.0f;
        cutoff = cutoff < list_cut ? cutoff : list_cut;
        const bool all_rows = (int64_t)ncand >= n;
        bool ok;
        if (proof == kProofNone) {
            ok = true;
        } else if (proof == kProofMargin) {
            // Fewer candidates than k means every row was a candidate.
            const float tau = kout > 0 ? slot_key(res[kout - 1]) : 0.0f;
            double margin = fabs((double)tau) * 1e-6;
            margin = margin < 1e-7 ? 1e-7 : margin;
            ok = all_rows || ncand < fa.k || (double)cutoff >= (double)tau + margin;
        } else {
            ok = all_rows || (kout > 0 && cutoff >= slot_key(res[kout - 1]));
        }
        fa.status[status_idx >= 0 ? status_idx : (int)blockIdx.y] = ok ? 0 : 1;
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
    block_select_lists(cand_q + (int64_t)g * fa.group_blocks * kc, (int64_t)gsize * kc, lds, cap,
                       kc, sel);
    if (tid < 64)
        for (int i = tid; i < kc; i += 64)
            store_shared_slot(&gcand_q[(int64_t)g * kc + i], i < sel.count ? sel.buf[i] : kEmptySlot);
    if (!block_arrive_last(&cnt_q[fa.ngroups], (uint32_t)fa.ngroups)) return false;
    if (tid == 0)
        __hip_atomic_store(&cnt_q[fa.ngroups], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    block_select_lists(gcand_q, (int64_t)fa.ngroups * kc, lds, cap, kc, sel);
    return true;
}

}  // namespace mans
