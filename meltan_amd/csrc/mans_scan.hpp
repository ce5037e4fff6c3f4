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

// Branch-free (all three keys, then a select): a branch here would split
// the scan loop into blocks across which the compiler does not keep the
// next step's loads in flight.
__device__ __forceinline__ float lower_key(float f, float qn, float vn, int metric,
                                           const BoundCoef& bc) {
    const float s = sqrtf(qn * vn);
    const float k_ip = -f - s * bc.c_ip;
    float dd = qn - 2.0f * f + vn;
    dd = dd > 0.0f ? dd : 0.0f;
    const float k_l2 = dd - (qn + vn + 2.0f * s) * bc.c_l2;
    float k_cos = (1.0f - f / s) - bc.eps_cos;
    k_cos = s < 1.001e-10f ? -1.0f : k_cos;            // near the 1e-10 branch of the formula
    k_cos = vn == 0.0f ? 1.0f - bc.eps_cos : k_cos;    // both paths give exactly 1
    return metric == kMetricIP ? k_ip : (metric == kMetricL2 ? k_l2 : k_cos);
}

// lower_key for one metric known at the call (the same expressions as its
// branch there): for callers outside a load-pipelined loop, where a uniform
// branch on the metric costs nothing and the other metrics' square root and
// division are not evaluated.
template <int METRIC>
__device__ __forceinline__ float lower_key_m(float f, float qn, float vn, const BoundCoef& bc) {
    const float s = sqrtf(qn * vn);
    if constexpr (METRIC == kMetricIP) {
        return -f - s * bc.c_ip;
    } else if constexpr (METRIC == kMetricL2) {
        float dd = qn - 2.0f * f + vn;
        dd = dd > 0.0f ? dd : 0.0f;
        return dd - (qn + vn + 2.0f * s) * bc.c_l2;
    } else {
        float k_cos = (1.0f - f / s) - bc.eps_cos;
        k_cos = s < 1.001e-10f ? -1.0f : k_cos;
        k_cos = vn == 0.0f ? 1.0f - bc.eps_cos : k_cos;
        return k_cos;
    }
}

// Loads of the streaming pass: R rows per 16-lane group (rows base + 4 wave
// + grp + 16 j), clamped to the block's last row and, past the row's end,
// replaced by zeros, so that no branch separates the loads.  The scheduling
// barrier keeps every load of the step ahead of the arithmetic that uses it.
template <int NCH, bool FULL, int R>
__device__ __forceinline__ void scan_load(const float* __restrict__ rows,
                                          const float* __restrict__ norms, int dim, int dim4,
                                          int64_t base, int64_t end, int slot, int lr,
                                          f4v (&a)[R][NCH], float (&vn)[R]) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int64_t r = base + slot + 16 * j;
        vn[j] = norms[r < end ? r : end - 1];
    }
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int64_t r = base + slot + 16 * j;
        const float* p = rows + (r < end ? r : end - 1) * dim;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int idx = lr + 16 * c;
            if (FULL) {
                a[j][c] = load_stream(p + 4 * idx);
            } else {
                const bool in = idx < dim4;
                const f4v t = load_stream(p + 4 * (in ? idx : dim4 - 1));
                a[j][c] = in ? t : f4v{0.f, 0.f, 0.f, 0.f};
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Fast dots (two accumulators per row), keys and offers of one step.
template <int NCH, int R, class Sel>
__device__ __forceinline__ void scan_offer(const f4v (&a)[R][NCH], const float (&vn)[R],
                                           const f4v* qv, float qn, int metric, const BoundCoef& bc,
                                           int64_t base, int64_t end, int slot, int lr, Sel& sel) {
    float s[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
        float x = 0.0f, y = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            float& t = (c & 1) ? y : x;
            t = fmaf(a[j][c].x, qv[c].x, t);
            t = fmaf(a[j][c].y, qv[c].y, t);
            t = fmaf(a[j][c].z, qv[c].z, t);
            t = fmaf(a[j][c].w, qv[c].w, t);
        }
        s[j] = row16_sum(x + y);
    }
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int64_t r = base + slot + 16 * j;
        sel.offer(lr == 0 && r < end, lower_key(s[j], qn, vn[j], metric, bc), (uint32_t)r);
    }
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
    // Threshold merge (flat scan, kc <= 64): one head per block list.
    uint64_t* heads = nullptr;    // [nq][nblk]
    int fast = 0;
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

// All threads call this after their store_shared_slot writes (and device-
// scope atomics); returns true (in every thread) in the block that arrives
// last at `counter` (expected arrivals: `total`).  Each wave first waits
// until its vector memory operations are complete (a workgroup-scope
// release fence does not wait for them on this target), the barrier makes
// that true for every wave, and only then is the arrival counted, so the
// last block to arrive finds every list at the coherence point.
__device__ __forceinline__ bool block_arrive_last(uint32_t* counter, uint32_t total) {
    __shared__ int last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
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
template <class Sel>
__device__ __forceinline__ void block_select_lists(const uint64_t* src, int64_t total, uint64_t* lds,
                                                   int cap, int kc, Sel& sel) {
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
template <class Sel>
__device__ __forceinline__ void block_fold(Sel& sel, uint64_t* lds, int cap) {
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

// chain_dot of two rows a0, a1 against the same b, their chains interleaved
// (each row's operations and their order are chain_dot's): a 16-lane group
// keeps two independent dependency chains in flight.
template <int NCH>
__device__ __forceinline__ void chain_dot2(const f4v* a0, const f4v* a1, const f4v* b, int dim4,
                                           float& d0, float& d1) {
    const int lane = __lane_id(), lr = lane & 15, row0 = lane & ~15;
    float acc0 = 0.0f, acc1 = 0.0f;
    int last = 0;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
#pragma unroll
        for (int o = 0; o < 16; ++o) {
            const int c = o + 16 * j;
            if (c < dim4) {
                float t0 = acc0 + a0[j].x * b[j].x;
                float t1 = acc1 + a1[j].x * b[j].x;
                t0 = t0 + a0[j].y * b[j].y;
                t1 = t1 + a1[j].y * b[j].y;
                t0 = t0 + a0[j].z * b[j].z;
                t1 = t1 + a1[j].z * b[j].z;
                t0 = t0 + a0[j].w * b[j].w;
                t1 = t1 + a1[j].w * b[j].w;
                acc0 = lr == o ? t0 : acc0;
                acc1 = lr == o ? t1 : acc1;
                last = o;
                if (c + 1 < dim4) {
                    acc0 = __int_as_float(
                        __builtin_amdgcn_update_dpp(0, __float_as_int(acc0), 0x121, 0xF, 0xF, false));
                    acc1 = __int_as_float(
                        __builtin_amdgcn_update_dpp(0, __float_as_int(acc1), 0x121, 0xF, 0xF, false));
                }
            }
        }
    }
    d0 = __shfl(acc0, row0 | last);
    d1 = __shfl(acc1, row0 | last);
}

// Threshold merge, step 1 (the scan kernel, every block): fold the block's
// four sorted wave lists (lds, stride cap) into its kc best (kc 32 or 64)
// and write them and the block's head (its smallest slot) with plain stores;
// the merge kernel reads them after the scan kernel has completed.  (No
// atomics: device-scope atomics queue behind the scan's memory traffic.)
__device__ __forceinline__ void flat_fast_block_out(const uint64_t* lds, int cap, int kc,
                                                    const FlatArgs& fa) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nblk = gridDim.x;
    __syncthreads();  // the four wave lists are final
    if (wave == 0) {
        const uint64_t v = wave_top_of_four(lds, cap, kc);
        uint64_t* cand_q = fa.cand + (int64_t)blockIdx.y * nblk * kc;
        if (lane < kc) cand_q[(int64_t)blockIdx.x * kc + lane] = v;
        if (lane == 0) fa.heads[(int64_t)blockIdx.y * nblk + blockIdx.x] = v;
    }
}

// Threshold merge, step 2 (one block of 256 threads per query): the kc best
// of the nblk block lists (cand_q, kc slots each) and their heads.  The heads
// are spread over 2 kc buckets (list b -> bucket b % 2 kc) and T is the kc-th
// smallest bucket minimum: the minima are heads of distinct lists, so at
// least kc slots are <= T and the query's kc best are the kc smallest slots
// <= T; only lists whose head is <= T hold such slots.  Those slots are
// gathered in LDS and sorted.  If more than kFastListCap lists or
// kFastCandCap slots qualify (many equal keys), every list is selected over
// instead.  Result: the kc best ascending in lds[0, kc) (kEmptySlot past the
// last candidate).
template <class Sel>
__device__ __forceinline__ void flat_fast_merge_lists(uint64_t* lds, int cap, int kc, int nblk,
                                                      const uint64_t* __restrict__ cand_q,
                                                      const uint64_t* __restrict__ heads_q,
                                                      Sel& sel) {
    __shared__ uint64_t bucket_sh[2 * kFastMaxKc];
    __shared__ uint64_t thr_sh;
    __shared__ int nlist_sh, ncand_sh;
    __shared__ uint16_t qlist[kFastListCap];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nb = 2 * kc;
    if (tid < nb) bucket_sh[tid] = kEmptySlot;
    if (tid == 0) {
        nlist_sh = 0;
        ncand_sh = 0;
    }
    constexpr int kHeads = 4;  // heads per thread and round
    uint64_t hv[kHeads];
#pragma unroll
    for (int i = 0; i < kHeads; ++i) {
        const int b = tid + 256 * i;
        hv[i] = b < nblk ? heads_q[b] : kEmptySlot;
    }
    __syncthreads();
    for (int h0 = 0; h0 < nblk; h0 += 256 * kHeads) {
        if (h0 > 0) {
#pragma unroll
            for (int i = 0; i < kHeads; ++i) {
                const int b = h0 + tid + 256 * i;
                hv[i] = b < nblk ? heads_q[b] : kEmptySlot;
            }
        }
#pragma unroll
        for (int i = 0; i < kHeads; ++i)
            if (hv[i] != kEmptySlot)
                atomicMin((unsigned long long*)&bucket_sh[(h0 + tid + 256 * i) % nb],
                          (unsigned long long)hv[i]);
    }
    __syncthreads();
    if (wave == 0) {
        uint64_t t;
        if (kc == 32) {
            uint64_t v[1];
            v[0] = bucket_sh[lane];
            wave_sort_regs<1>(v);
            t = shfl64(v[0], 31);
        } else {
            uint64_t v[2];
            v[0] = bucket_sh[lane];
            v[1] = bucket_sh[64 + lane];
            wave_sort_regs<2>(v);
            t = shfl64(v[0], 63);
        }
        if (lane == 0) thr_sh = t;  // kEmptySlot: fewer than kc lists, all qualify
    }
    __syncthreads();
    const uint64_t T = thr_sh;
    for (int h0 = 0; h0 < nblk; h0 += 256 * kHeads) {
        if (h0 > 0) {
#pragma unroll
            for (int i = 0; i < kHeads; ++i) {
                const int b = h0 + tid + 256 * i;
                hv[i] = b < nblk ? heads_q[b] : kEmptySlot;
            }
        }
#pragma unroll
        for (int i = 0; i < kHeads; ++i) {
            const bool pass = hv[i] != kEmptySlot && hv[i] <= T;
            const uint64_t m = __ballot(pass);
            if (m == 0) continue;
            int base = 0;
            if (lane == 0) base = atomicAdd(&nlist_sh, __popcll(m));
            base = __shfl(base, 0);
            const int pos = base + __popcll(m & lanemask_lt());
            if (pass && pos < kFastListCap) qlist[pos] = (uint16_t)(h0 + tid + 256 * i);
        }
    }
    __syncthreads();
    const int nl = nlist_sh;
    if (nl > kFastListCap) {  // more qualifying lists than the queue holds
        block_select_lists(cand_q, (int64_t)nblk * kc, lds, cap, kc, sel);
        return;
    }
    const int total = nl * kc;
    const int lkc = kc == 32 ? 5 : 6;
    constexpr int kAhead = 8;
    for (int e0 = 0; e0 < total; e0 += 256 * kAhead) {
        uint64_t sv[kAhead];
#pragma unroll
        for (int u = 0; u < kAhead; ++u) {
            const int e = e0 + 256 * u + tid;
            sv[u] = e < total ? cand_q[(int64_t)qlist[e >> lkc] * kc + (e & (kc - 1))] : kEmptySlot;
        }
#pragma unroll
        for (int u = 0; u < kAhead; ++u) {
            const bool pass = sv[u] != kEmptySlot && sv[u] <= T;
            const uint64_t m = __ballot(pass);
            if (m == 0) continue;
            int base = 0;
            if (lane == 0) base = atomicAdd(&ncand_sh, __popcll(m));
            base = __shfl(base, 0);
            const int pos = base + __popcll(m & lanemask_lt());
            if (pass && pos < kFastCandCap) lds[pos] = sv[u];
        }
    }
    __syncthreads();
    const int nc = ncand_sh;
    if (nc > kFastCandCap) {
        block_select_lists(cand_q, (int64_t)nblk * kc, lds, cap, kc, sel);
        return;
    }
    int size = 64;
    while (size < nc) size <<= 1;
    for (int i = nc + tid; i < size; i += 256) lds[i] = kEmptySlot;
    __syncthreads();
    if (wave == 0) wave_bitonic_sort<512>(lds, size);  // up to kFastCandCap slots in registers
    __syncthreads();
}

// LDS the threshold merge's rescore needs beyond lds[0, 128): the query
// (up to 384 floats) and 32 staged rows of up to 384 floats, each padded by
// 4 floats so that the lanes' 16-byte reads of one column spread over the
// banks.
constexpr int kRescoreRows = 32;
constexpr int kRescoreMaxDim = 384;
constexpr int kRescoreStride = kRescoreMaxDim + 4;
constexpr size_t kFastLdsBytes =
    128 * sizeof(uint64_t) + (kRescoreMaxDim + kRescoreRows * kRescoreStride) * sizeof(float);

// Exact rescore for the threshold merge (kc <= 64, candidates ascending in
// lds[0, kc), dim <= 64 NCH <= 384).  The whole block loads 32 candidate
// rows at once into LDS (every load in flight together, one barrier); then
// lane c of wave 0 runs candidate c's whole dot product in the dots.c order
// and lane 32 the query's own q.q.  Two passes for kc = 64.  Wave 0 then
// sorts the results; outputs and the proof as final_rescore_f4 (flat proof).
template <int NCH, bool FULL>
__device__ __forceinline__ void final_rescore_fast(const float* __restrict__ qp,
                                                   const float* __restrict__ rows,
                                                   const float* __restrict__ norms, int64_t n,
                                                   int dim, int metric, uint32_t q, uint64_t* lds,
                                                   int kc, const FlatArgs& fa, int status_idx) {
    static_assert(16 * NCH * 4 <= kRescoreMaxDim, "rows longer than the staging area");
    constexpr int kRow4 = 16 * NCH;                    // float4s per row, padded
    constexpr int kPer = kRescoreRows * kRow4 / 256;   // float4s each thread stages
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int dim4 = FULL ? kRow4 : (dim >> 2);
    const uint64_t* top = lds;
    uint64_t* res = lds + 64;
    float* qs = reinterpret_cast<float*>(lds + 128);
    float* stage = qs + kRescoreMaxDim;
    const int ncand = __popcll(__ballot(lane < kc && top[lane] != kEmptySlot));
    for (int i = tid; i < dim4; i += blockDim.x)
        *reinterpret_cast<f4v*>(qs + 4 * i) = *reinterpret_cast<const f4v*>(qp + 4 * i);
    float qn = 0.0f;
    for (int pass = 0; pass * kRescoreRows < ncand; ++pass) {
        const int cl = pass * kRescoreRows + lane;  // the candidate lane `lane` rescores
        // The candidate's norm, in flight with its row.
        const float vn_c = wave == 0 && lane < kRescoreRows && cl < ncand && metric != kMetricIP
                               ? norms[slot_id(top[cl])]
                               : 0.0f;
        f4v v[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int e = tid + 256 * j;
            const int r = e / kRow4, c4 = e - r * kRow4;
            const int c = pass * kRescoreRows + r;
            const bool in = c < ncand && (FULL || c4 < dim4);
            const uint32_t id = c < ncand ? slot_id(top[c]) : 0u;
            const f4v t = *reinterpret_cast<const f4v*>(rows + (int64_t)id * dim + (in ? 4 * c4 : 0));
            v[j] = in ? t : f4v{0.f, 0.f, 0.f, 0.f};
        }
        if (pass > 0) __syncthreads();  // the previous pass has read the stage
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int e = tid + 256 * j;
            const int r = e / kRow4, c4 = e - r * kRow4;
            *reinterpret_cast<f4v*>(stage + r * kRescoreStride + 4 * c4) = v[j];
        }
        __syncthreads();
        if (wave == 0) {
            float acc = 0.0f;
            if (lane <= kRescoreRows) {
                const float* xr = lane < kRescoreRows ? stage + lane * kRescoreStride : qs;
                for (int i = 0; i < dim4; ++i) {
                    const f4v x = *reinterpret_cast<const f4v*>(xr + 4 * i);
                    const f4v y = *reinterpret_cast<const f4v*>(qs + 4 * i);
                    acc = acc + x.x * y.x;
                    acc = acc + x.y * y.y;
                    acc = acc + x.z * y.z;
                    acc = acc + x.w * y.w;
                }
            }
            if (pass == 0) qn = metric == kMetricIP ? 0.0f : __shfl(acc, kRescoreRows);
            if (lane < kRescoreRows) {
                uint64_t rs = kEmptySlot;
                if (cl < ncand) {
                    const uint32_t cid = slot_id(top[cl]);
                    rs = pack_slot(host_distance(acc, qn, vn_c, metric), cid);
                }
                res[cl] = rs;
            }
        }
    }
    __syncthreads();
    if (wave == 0) {
        uint64_t w[1];
        w[0] = lane < ncand ? res[lane] : kEmptySlot;
        wave_sort_regs<1>(w);
        res[lane] = w[0];
    }
    __syncthreads();
    const int kout = fa.k < ncand ? fa.k : ncand;
    for (int i = tid; i < fa.k_stride; i += blockDim.x) {
        float dv = kFltMax;
        uint32_t oid = kEmptyId;
        if (i < kout) {
            oid = slot_id(res[i]);
            dv = slot_key(res[i]);
        }
        fa.out_dist[(int64_t)q * fa.k_stride + i] = dv;
        fa.out_ids[(int64_t)q * fa.k_stride + i] = oid;
    }
    if (tid == 0) {
        const float cutoff = ncand > 0 ? slot_key(top[ncand - 1]) : 0.0f;
        const bool ok = (int64_t)ncand >= n || (kout > 0 && cutoff >= slot_key(res[kout - 1]));
        fa.status[status_idx] = ok ? 0 : 1;
    }
}

// Proof applied by final_rescore_f4 to the rescored candidates.
enum ProofMode : int {
    kProofFlat = 0,    // cutoff key >= k-th exact distance
    kProofMargin = 1,  // BoundedExactScan.swift:108-113: cutoff >= tau + max(1e-7, |tau| 1e-6)
    kProofNone = 2,    // fixed budget: no proof (status 0)
};

// Status of a query after a launch: 0 done, 1 proof failed (grow the
// candidate count), kStatusReselect: the bounded lists could not show that
// the candidates are the kc smallest keys (select again at the same kc with
// the streaming scan).
constexpr uint8_t kStatusReselect = 2;

// The last block of a query: exact rescore of the kc candidates held in
// lds[0, kc), sort by (distance, id), outputs and proof status.  qv: the
// query chunks.  lds must hold kc + pow2(kc) slots (cap >= 2 kc, 4 caps).
// Candidate ids index `rows`; idmap (nullable) maps them to the ids that are
// reported and that order ties.  n: the number of rows the query could see.
// status_idx: the status slot (default: blockIdx.y).
// sel_cut: the smallest largest slot over bounded lists that turned rows
// away (kEmptySlot: none did).  Such a row's slot is above sel_cut, so the
// candidates are the exact kc smallest slots only when the kc-th is <=
// sel_cut; otherwise the status is kStatusReselect and nothing else holds.
template <int NCH>
__device__ __forceinline__ void final_rescore_f4(const f4v* qv, const float* __restrict__ rows,
                                 const float* __restrict__ norms, int64_t n, int dim, int metric,
                                 uint32_t q, uint64_t* lds, int kc, const FlatArgs& fa,
                                 float list_cut = kFltMax, int proof = kProofFlat,
                                 const uint32_t* idmap = nullptr, int status_idx = -1,
                                 uint64_t sel_cut = kEmptySlot) {
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
        const bool sel_exact = sel_cut == kEmptySlot || (ncand == kc && top[kc - 1] <= sel_cut);
        fa.status[status_idx >= 0 ? status_idx : (int)blockIdx.y] =
            !sel_exact ? kStatusReselect : (ok ? 0 : 1);
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

// Block-wide minimum (MAX = false) or maximum of one value per thread
// (shuffles within each wave, then one value per wave through LDS; 64-bit
// LDS atomics would serialise every thread).  blockDim.x <= 1024.
template <bool MAX>
__device__ __forceinline__ uint64_t block_reduce_u64(uint64_t v) {
    __shared__ uint64_t part[16];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint64_t t = lane_xor64(v, o);
        v = MAX ? (t > v ? t : v) : (t < v ? t : v);
    }
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();  // part[] may still be read from a previous call
    if ((threadIdx.x & 63) == 0) part[wave] = v;
    __syncthreads();
    v = part[0];
    for (int w = 1; w < nw; ++w) v = MAX ? (part[w] > v ? part[w] : v) : (part[w] < v ? part[w] : v);
    return v;
}

// Whole-block radix select over `total` distinct slots read through
// get(i): returns a cut U with exactly min(need, total) slots <= U, and
// the largest of those in *kth (kEmptySlot when total <= need: every slot
// is taken).  Most significant 8-bit digit first: each pass counts the
// slots that share the digits chosen so far by their next digit, and stops
// as soon as the digit bin that holds the need-th slot holds no more than
// the slots still needed.  hist: 256 words of LDS.
template <class Get>
__device__ __forceinline__ uint64_t block_radix_cut(Get&& get, int64_t total, int need,
                                                    uint32_t* hist, uint64_t* kth) {
    const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63;
    __shared__ uint64_t s_prefix;
    __shared__ int s_need, s_done;
    if (total <= need) {
        *kth = kEmptySlot;
        return kEmptySlot;
    }
    // Digits above the highest one where the smallest and largest slots
    // differ are common to all slots: the passes start below them.
    uint64_t lo = ~0ull, hi = 0;
    for (int64_t i = tid; i < total; i += nt) {
        const uint64_t s = get(i);
        lo = s < lo ? s : lo;
        hi = s > hi ? s : hi;
    }
    const uint64_t s_min = block_reduce_u64<false>(lo);
    const uint64_t s_max = block_reduce_u64<true>(hi);
    const uint64_t diff = s_min ^ s_max;  // nonzero: the slots are distinct
    const int top_shift = diff ? (63 - __clzll((long long)diff)) / 8 * 8 : 0;
    uint64_t mask = top_shift == 56 ? 0ull : ~0ull << (top_shift + 8);
    uint64_t prefix = s_min & mask;
    for (int shift = top_shift; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += nt) hist[i] = 0;
        __syncthreads();
        for (int64_t i = tid; i < total; i += nt) {
            const uint64_t s = get(i);
            if ((s & mask) == prefix) atomicAdd(&hist[(s >> shift) & 255], 1u);
        }
        __syncthreads();
        if (tid < 64) {
            // Lane l owns bins 4 l .. 4 l + 3; an inclusive scan over the
            // lanes gives each lane the count below its first bin.
            const uint32_t c0 = hist[4 * lane], c1 = hist[4 * lane + 1];
            const uint32_t c2 = hist[4 * lane + 2], c3 = hist[4 * lane + 3];
            const uint32_t own = c0 + c1 + c2 + c3;
            uint32_t incl = own;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_up(incl, o);
                incl += lane >= o ? t : 0u;
            }
            uint32_t before = incl - own;
            const uint32_t c[4] = {c0, c1, c2, c3};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (before < (uint32_t)need && (uint32_t)need <= before + c[j]) {
                    s_prefix = prefix | ((uint64_t)(4 * lane + j) << shift);
                    s_need = need - (int)before;
                    s_done = c[j] == (uint32_t)(need - (int)before);
                }
                before += c[j];
            }
        }
        __syncthreads();
        prefix = s_prefix;
        need = s_need;
        mask |= 0xFFull << shift;
        const bool done = s_done;
        __syncthreads();  // s_* are written again by the next pass
        if (done) break;
    }
    const uint64_t cut = prefix | ~mask;
    uint64_t m = 0;
    for (int64_t i = tid; i < total; i += nt) {
        const uint64_t s = get(i);
        m = s <= cut && s > m ? s : m;
    }
    *kth = block_reduce_u64<true>(m);
    return cut;
}

// Starts bringing the candidate rows (ids in top[0, ncand)) into the L2
// without holding registers: one 4-byte global-to-LDS load per 128-byte
// line, each wave's into the same 256 bytes of `sink` (contents unused;
// the loads are complete once a later load of the same thread is).
__device__ __forceinline__ void prefetch_rows(const float* __restrict__ rows, const uint64_t* top,
                                              int ncand, int dim, void* sink) {
    const int lines = (dim * 4 + 127) / 128;
    const int total = ncand * lines;
    for (int i = threadIdx.x; i < total; i += blockDim.x) {
        const int r = i / lines, l = i - r * lines;
        const float* p = rows + (int64_t)slot_id(top[r]) * dim + 32 * l;
        __builtin_amdgcn_global_load_lds(p, (__attribute__((address_space(3))) void*)sink, 4, 0, 0);
    }
}

// Exact rescore of up to 64 M (<= blockDim.x = 256) candidates (ascending
// in top[0, ncand)), one candidate per thread: thread t runs candidate t's
// whole dot product in the dots.c order.  The rows reach LDS in pieces of
// kWidePiece floats, loaded by the whole block (W pieces in flight, M
// float4 loads per thread and piece) and written one piece ahead of the
// threads that read them.  qp: the query (read with scalar loads); qn: its
// sequential q.q.  res: 256 slots (it may be the sink of prefetch_rows);
// stage: 2 * 64 M * kWideStride floats.  Outputs, proof, list_cut and
// sel_cut as final_rescore_f4 (status at blockIdx.y).  dim % 4 == 0.
constexpr int kWidePiece = 16;
constexpr int kWideStride = 20;  // floats per staged row piece (bank spread)
template <int M, int W>
__device__ __forceinline__ void final_rescore_wide_mw(const float* __restrict__ qp, float qn,
                                                      const float* __restrict__ rows,
                                                      const float* __restrict__ norms, int64_t n,
                                                      int dim, int metric, uint32_t q,
                                                      const uint64_t* top, int ncand, int kc,
                                                      uint64_t* res, float* stage, const FlatArgs& fa,
                                                      int proof, uint64_t sel_cut, float list_cut) {
    const int tid = threadIdx.x;
    const int npieces = (dim + kWidePiece - 1) / kWidePiece;
    const int lr = tid >> 2, u = tid & 3;  // stages float4 u of rows lr + 64 m
    const float* rp[M];
    bool rv[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const int c = lr + 64 * m;
        rv[m] = c < ncand;
        rp[m] = rows + (int64_t)(rv[m] ? slot_id(top[c]) : 0u) * dim;
    }
    auto load_piece = [&](int pc, f4v (&v)[M]) {
        const int off = kWidePiece * pc + 4 * u;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const bool in = rv[m] && off < dim;
            const f4v t = *reinterpret_cast<const f4v*>(rp[m] + (in ? off : 0));
            v[m] = in ? t : f4v{0.f, 0.f, 0.f, 0.f};
        }
    };
    f4v v[W][M];
#pragma unroll
    for (int w = 0; w < W; ++w)
        if (w < npieces) load_piece(w, v[w]);
    float acc = 0.0f;
    for (int pc0 = 0; pc0 < npieces; pc0 += W) {
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const int pc = pc0 + w;
            if (pc >= npieces) break;
            float* buf = stage + (pc & 1) * 64 * M * kWideStride;
#pragma unroll
            for (int m = 0; m < M; ++m)
                *reinterpret_cast<f4v*>(buf + (lr + 64 * m) * kWideStride + 4 * u) = v[w][m];
            if (pc + W < npieces) load_piece(pc + W, v[w]);
            __syncthreads();
            if (tid < ncand) {
                const float* xr = buf + tid * kWideStride;
                const float* yr = qp + kWidePiece * pc;  // uniform: scalar loads
                const int rem = dim - kWidePiece * pc;
#pragma unroll
                for (int i = 0; i < kWidePiece / 4; ++i) {
                    if (4 * i >= rem) break;
                    const f4v x = *reinterpret_cast<const f4v*>(xr + 4 * i);
                    const f4v y = *reinterpret_cast<const f4v*>(yr + 4 * i);
                    acc = acc + x.x * y.x;
                    acc = acc + x.y * y.y;
                    acc = acc + x.z * y.z;
                    acc = acc + x.w * y.w;
                }
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // prefetches into res have landed
    __syncthreads();
    int sort_n = 64;
    while (sort_n < ncand) sort_n <<= 1;
    if (tid < sort_n) {
        uint64_t rs = kEmptySlot;
        if (tid < ncand) {
            const uint32_t cid = slot_id(top[tid]);
            rs = pack_slot(host_distance(acc, qn, metric == kMetricIP ? 0.0f : norms[cid], metric),
                           cid);
        }
        res[tid] = rs;
    }
    __syncthreads();
    if (tid < 64) wave_bitonic_sort(res, sort_n);
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
            const float tau = kout > 0 ? slot_key(res[kout - 1]) : 0.0f;
            double margin = fabs((double)tau) * 1e-6;
            margin = margin < 1e-7 ? 1e-7 : margin;
            ok = all_rows || ncand < fa.k || (double)cutoff >= (double)tau + margin;
        } else {
            ok = all_rows || (kout > 0 && cutoff >= slot_key(res[kout - 1]));
        }
        const bool sel_exact = sel_cut == kEmptySlot || (ncand == kc && top[kc - 1] <= sel_cut);
        fa.status[blockIdx.y] = !sel_exact ? kStatusReselect : (ok ? 0 : 1);
    }
}

// final_rescore_wide_mw with eight float4 loads per thread in flight (8
// pieces for up to 64 candidates, 4 for 128, 3 for 192, 2 for 256; deeper
// windows spill).
__device__ __forceinline__ void final_rescore_wide(const float* __restrict__ qp, float qn,
                                                   const float* __restrict__ rows,
                                                   const float* __restrict__ norms, int64_t n,
                                                   int dim, int metric, uint32_t q,
                                                   const uint64_t* top, int ncand, int kc,
                                                   uint64_t* res, float* stage, const FlatArgs& fa,
                                                   int proof, uint64_t sel_cut,
                                                   float list_cut = kFltMax) {
    if (ncand <= 64)
        final_rescore_wide_mw<1, 8>(qp, qn, rows, norms, n, dim, metric, q, top, ncand, kc, res, stage, fa, proof, sel_cut, list_cut);
    else if (ncand <= 128)
        final_rescore_wide_mw<2, 4>(qp, qn, rows, norms, n, dim, metric, q, top, ncand, kc, res, stage, fa, proof, sel_cut, list_cut);
    else if (ncand <= 192)
        final_rescore_wide_mw<3, 3>(qp, qn, rows, norms, n, dim, metric, q, top, ncand, kc, res, stage, fa, proof, sel_cut, list_cut);
    else
        final_rescore_wide_mw<4, 2>(qp, qn, rows, norms, n, dim, metric, q, top, ncand, kc, res, stage, fa, proof, sel_cut, list_cut);
}

// The kc-th smallest of `total` slots at src (written by an earlier launch;
// empty slots, kEmptySlot, are the largest values): kEmptySlot when fewer
// than kc are not empty.  Up to kKthLdsSlots slots are read once into
// lds; more are read from memory on every radix pass.
constexpr int kKthLdsSlots = 4096;
__device__ __forceinline__ uint64_t block_kth_slot(const uint64_t* __restrict__ src, int64_t total,
                                                   int kc, uint64_t* lds) {
    __shared__ uint32_t hist[256];
    const bool in_lds = total <= kKthLdsSlots;
    if (in_lds)
        for (int64_t i = threadIdx.x; i < total; i += blockDim.x) lds[i] = src[i];
    __syncthreads();
    uint64_t kth;
    block_radix_cut([&](int64_t i) { return in_lds ? lds[i] : src[i]; }, total, kc, hist, &kth);
    return kth;
}

}  // namespace mans
