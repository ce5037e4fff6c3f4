// Exact flat scan on gfx950: FlatGPUSearch.batchSearch / ParallelFlatScan.search
// (FlatGPUSearch.swift:103-181, ParallelFlatScan.swift:96-155).
//
//  1. Streaming pass (flat_scan_f4): 16 lanes per row, 128-bit loads, fused
//     multiply-adds in any order, a 16-lane DPP reduction, then a provable
//     lower bound on the exact distance (the "key").  Each wave keeps its
//     best kc keys in LDS (WaveTopK); wave 0 folds the block's 4 lists and
//     writes kc slots.
//  2. Merge.  Fast path (kc <= 64, dim <= 384): a second kernel
//     (flat_fast_merge, one block per query) merges the block lists by a
//     threshold taken from the lists' heads and rescores the kc candidates
//     with one lane per candidate.  Otherwise the last block of each group
//     of kGroupBlocks blocks to arrive (per-query counters, one atomic per
//     block) merges the group's lists, the last group to arrive merges the
//     group lists and rescores.  Either way the kc candidates' distances
//     are recomputed in the scalar order of dots.c:40-47 with the host
//     formulas (bit-identical to the CPU path), sorted by (distance, id) and
//     k are written.  The query passes the proof when the kc-th key is >=
//     the k-th exact distance: every row left out has a key >= the kc-th
//     key, so an exact distance >= every row returned.
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
#include "mans_scan.hpp"

namespace mans {

// grid: (nblk, nq_launch); block 256 = 4 waves; dynamic LDS: 4 * cap slots
// (kFastLdsBytes with FAST).  FULL: dim == 64 NCH (no partial chunks).
// PF: one row per group per step with the next step's row loaded while the
// current one is reduced; otherwise two rows per group per step.  FAST
// (kc <= 64, cap 128, PF): the threshold merge and lane-per-candidate
// rescore (flat_fast_merge) finish the query.  rows_per_block sets the
// grid's block count; the rows go to blocks in strided 32-row tiles.
template <int NCH, bool FULL, bool PF, bool FAST>
__global__ __launch_bounds__(256) void flat_scan_f4(
    const float* __restrict__ rows, const float* __restrict__ norms, int64_t n, int dim,
    const float* __restrict__ queries, const uint32_t* __restrict__ qidx, int metric,
    BoundCoef bc, int kc, int cap, int64_t rows_per_block, FlatArgs fa) {
    extern __shared__ uint64_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = lane >> 4, lr = lane & 15;
    const int slot = wave * 4 + grp;
    const uint32_t q = qidx ? qidx[blockIdx.y] : blockIdx.y;
    const int dim4 = FULL ? 16 * NCH : (dim >> 2);
    const float* qp = queries + (int64_t)q * dim;

    f4v qv[NCH];
    float qsq = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        int idx = lr + 16 * c;
        qv[c] = (FULL || idx < dim4) ? *reinterpret_cast<const f4v*>(qp + 4 * idx)
                                     : f4v{0.f, 0.f, 0.f, 0.f};
        qsq = fmaf(qv[c].x, qv[c].x, qsq);
        qsq = fmaf(qv[c].y, qv[c].y, qsq);
        qsq = fmaf(qv[c].z, qv[c].z, qsq);
        qsq = fmaf(qv[c].w, qv[c].w, qsq);
    }
    const float qn = row16_sum(qsq);

    WaveTopKT<FAST ? 128 : 0> sel;
    sel.init(lds + wave * cap, cap, kc);

    // Block b takes the 32-row tiles b, b + nblk, b + 2 nblk, ...: the
    // blocks in flight read one moving window of the corpus, which keeps
    // the HBM pages they open close together.
    const int64_t stride = 32 * (int64_t)gridDim.x;
    const int64_t first = 32 * (int64_t)blockIdx.x;
    if constexpr (PF) {
        f4v a[1][NCH], b[1][NCH];
        float va[1], vb[1];
        scan_load<NCH, FULL, 1>(rows, norms, dim, dim4, first, n, slot, lr, a, va);
        for (int64_t base = first; base < n; base += stride) {
            scan_load<NCH, FULL, 1>(rows, norms, dim, dim4, base + 16, n, slot, lr, b, vb);
            scan_offer<NCH, 1>(a, va, qv, qn, metric, bc, base, n, slot, lr, sel);
            scan_load<NCH, FULL, 1>(rows, norms, dim, dim4, base + stride, n, slot, lr, a, va);
            scan_offer<NCH, 1>(b, vb, qv, qn, metric, bc, base + 16, n, slot, lr, sel);
        }
    } else {
        static_assert(!FAST, "the fast kernel prefetches");
        for (int64_t base = first; base < n; base += stride) {
            f4v a[2][NCH];
            float va[2];
            scan_load<NCH, FULL, 2>(rows, norms, dim, dim4, base, n, slot, lr, a, va);
            scan_offer<NCH, 2>(a, va, qv, qn, metric, bc, base, n, slot, lr, sel);
        }
    }
    sel.finish();
    if constexpr (FAST) {
        flat_fast_block_out(lds, cap, kc, fa);  // flat_fast_merge finishes the query
    } else {
        if (!flat_block_epilogue(sel, lds, cap, kc, fa)) return;
        final_rescore_f4<NCH>(qv, rows, norms, n, dim, metric, q, lds, kc, fa);
    }
}

// Threshold merge and exact rescore of the fast scan: one block per query
// (grid: nq_launch), after flat_scan_f4<..., FAST> has written the block
// lists and heads.  dynamic LDS: kFastLdsBytes.
template <int NCH, bool FULL>
__global__ __launch_bounds__(256) void flat_fast_merge(
    const float* __restrict__ rows, const float* __restrict__ norms, int64_t n, int dim,
    const float* __restrict__ queries, const uint32_t* __restrict__ qidx, int metric, int kc,
    int cap, int nblk, FlatArgs fa) {
    extern __shared__ uint64_t lds[];
    const int y = blockIdx.x;
    const uint32_t q = qidx ? qidx[y] : (uint32_t)y;
    WaveTopKT<128> sel;  // the full selection, if too many slots qualify
    flat_fast_merge_lists(lds, cap, kc, nblk, fa.cand + (int64_t)y * nblk * kc,
                          fa.heads + (int64_t)y * nblk, sel);
    final_rescore_fast<NCH, FULL>(queries + (int64_t)q * dim, rows, norms, n, dim, metric, q, lds,
                                  kc, fa, y);
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

FlatPlan plan_flat(int64_t n, int64_t nq, int kc, int64_t target_blocks) {
    FlatPlan p;
    p.kc = kc;
    p.cap = flat_cap_for(kc);
    static const int64_t flat_target = [] {
        const char* e = std::getenv("MANS_FLAT_BLOCKS");
        return e ? std::max<int64_t>(1, std::atoll(e)) : (int64_t)0;
    }();
    // About 512 blocks per launch for large corpora (two per CU: the merge
    // reads one list per block); for smaller ones about one block per 196
    // rows (at least 256), so a block's fixed costs (list, head, merge
    // inputs) stay small next to its rows.
    const int64_t auto_target = std::min<int64_t>(512, std::max<int64_t>(256, n / 196));
    const int64_t target = target_blocks > 0 ? target_blocks : (flat_target > 0 ? flat_target : auto_target);
    int64_t want_blocks = (target + nq - 1) / nq;
    int64_t max_blocks = (n + 63) / 64;
    if (want_blocks > max_blocks) want_blocks = max_blocks;
    if (want_blocks < 1) want_blocks = 1;
    int64_t rpb = (n + want_blocks - 1) / want_blocks;
    rpb = (rpb + 15) / 16 * 16;
    p.rows_per_block = rpb;
    p.nblk = (int)((n + rpb - 1) / rpb);
    p.group_blocks = kGroupBlocks;
    p.ngroups = (p.nblk + kGroupBlocks - 1) / kGroupBlocks;
    p.fast = kc <= kFastMaxKc && p.cap == 128 && p.nblk <= kFastMaxBlocks;
    return p;
}

template <int NCH>
static void launch_f4(const FlatPlan& p, const float* rows, const float* norms, int64_t n, int dim,
                      const float* queries, const uint32_t* qidx, int64_t nq, int metric,
                      const BoundCoef& bc, const FlatArgs& fa, hipStream_t s) {
    size_t shmem = sizeof(uint64_t) * 4 * (size_t)p.cap;
    constexpr bool kPf = NCH <= 6;  // room for a second row buffer at 4 waves per SIMD
    const dim3 grid(p.nblk, (unsigned)nq);
    if constexpr (kPf) {
        if (fa.fast) {
            if (dim == 64 * NCH) {
                hipLaunchKernelGGL((flat_scan_f4<NCH, true, true, true>), grid, dim3(256), shmem, s,
                                   rows, norms, n, dim, queries, qidx, metric, bc, p.kc, p.cap,
                                   p.rows_per_block, fa);
                hipLaunchKernelGGL((flat_fast_merge<NCH, true>), dim3((unsigned)nq), dim3(256),
                                   kFastLdsBytes, s, rows, norms, n, dim, queries, qidx, metric, p.kc,
                                   p.cap, p.nblk, fa);
            } else {
                hipLaunchKernelGGL((flat_scan_f4<NCH, false, true, true>), grid, dim3(256), shmem, s,
                                   rows, norms, n, dim, queries, qidx, metric, bc, p.kc, p.cap,
                                   p.rows_per_block, fa);
                hipLaunchKernelGGL((flat_fast_merge<NCH, false>), dim3((unsigned)nq), dim3(256),
                                   kFastLdsBytes, s, rows, norms, n, dim, queries, qidx, metric, p.kc,
                                   p.cap, p.nblk, fa);
            }
            return;
        }
    }
    hipLaunchKernelGGL((flat_scan_f4<NCH, false, kPf, false>), grid, dim3(256), shmem, s, rows,
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
    fa.heads = b.heads;
    int nch = exact ? 0 : flat_nch_for_dim(dim);
    fa.fast = p.fast && nch != 0 && nch <= 6 ? 1 : 0;
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
