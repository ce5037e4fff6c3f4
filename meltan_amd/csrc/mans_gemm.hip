// Batched exact flat scan on gfx950: FlatGPUSearch.batchSearch
// (FlatGPUSearch.swift:103-181) for batches of queries, as an fp32 MFMA
// contraction with the top-k selection fused into its epilogue, followed by
// the per-query merge, exact rescore and proof of the streaming scan.
#include <algorithm>
#include <cstdlib>

#include "mans_device.hpp"
#include "mans_internal.hpp"
#include "mans_scan.hpp"

namespace mans {

// Batched queries: the query x row contraction on fp32 MFMA
// (v_mfma_f32_32x32x2_f32) with the selection fused into the epilogue, so
// the nq x n score matrix is never written.
//
// Block: 4 waves and 128 queries (32 per wave) over one segment of rows.
// Rows are the MFMA A operand, 32 per tile, staged through LDS in K-slices
// (double-buffered); queries are the B operand and stay in registers for the
// whole segment (DIM / 2 values per lane).  In the 32 x 32 result a lane
// holds one query (lane % 32) against 16 rows of the tile (row
// 8 (v / 4) + 4 h + v % 4 for accumulator v, h = lane / 32), and keeps the
// C smallest (key, row) slots it has seen in registers, sorted (C = 4 for
// kc <= 32, 8 for kc = 64).  A tile's keys are offered while the next
// tile's MFMAs run.
//
// flat_lists_merge selects each query's kc smallest keys over its 2 nseg
// lists and runs the streaming scan's exact rescore.  A row turned away by a
// full list has a key >= that list's largest key, so the proof's cutoff is
// the smaller of the kc-th merged key and the smallest full-list maximum.
//
// The keys are the streaming scan's lower bounds computed with u = 2^-23
// (twice the fp32 unit roundoff, so any faithfully rounded accumulation
// inside the matrix core is covered) and an absolute term for products and
// partial sums flushed below the smallest normal.
constexpr int kGemmQueries = 128;  // queries per block
constexpr int kGemmRows = 32;      // rows per tile

// Slots per lane list for a candidate count kc.
inline int gemm_list_len(int kc) { return kc <= 32 ? 4 : 8; }

struct GemmArgs {
    int nseg;              // row segments (multiple of 8)
    int nqb;               // query blocks
    int64_t rows_per_seg;  // multiple of kGemmRows
    float abs_slack;
    uint64_t* lists;       // [nq][nseg][2][C]
};

// LDS slices of the row tile: SL MFMA steps (2 SL values of k) per slice,
// SL dividing DIM / 2, a multiple of 4 and at most 96.
template <int DIM>
struct GemmShape {
    static constexpr int NS = DIM / 2;  // MFMA steps per tile
    static constexpr int SL = NS <= 96 ? NS : (NS % 96 == 0 ? 96 : 64);
    static constexpr int NSLICE = NS / SL;
    static constexpr int SK = 2 * SL;   // k values per slice
    static constexpr int SS = SK + 4;   // LDS floats per row: odd float4 count, no bank conflicts
    static constexpr int SLICE_FLOATS = kGemmRows * SS;
    static constexpr int F4_PER_ROW = SK / 4;
    static constexpr int LOADS = kGemmRows * F4_PER_ROW / 256;  // float4 per thread per slice
    static_assert(DIM % 8 == 0 && NS % SL == 0 && SL % 4 == 0, "unsupported dimension");
    static_assert(kGemmRows * F4_PER_ROW % 256 == 0, "slice does not split over 256 threads");
};

template <int DIM>
size_t gemm_lds_bytes() {
    using G = GemmShape<DIM>;
    return sizeof(float) * (2 * G::SLICE_FLOATS + 4 * kGemmRows);
}

// Sorted ascending list of the C smallest slots; inserts s, branch-free.
template <int C>
__device__ __forceinline__ void list_insert(uint64_t (&l)[C], uint64_t s) {
    uint64_t below = l[0];
    l[0] = s < l[0] ? s : l[0];
#pragma unroll
    for (int i = 1; i < C; ++i) {
        const uint64_t cur = l[i];
        const uint64_t m = s > below ? s : below;
        l[i] = m < cur ? m : cur;
        below = cur;
    }
}

// grid: nseg * nqb blocks (1-D); block 256.  Block b serves segment
// 8 (b / (8 nqb)) + b % 8 and query block (b % (8 nqb)) / 8: the query
// blocks of one segment share b % 8, which places them on the same XCD, so
// the segment is read from HBM once into that XCD's L2.
//
// MFMA step s = 4 g + j (j < 4) contracts k = 8 g + 4 h + j, so a lane reads
// the k values of its steps as float4s: rows from LDS (row-major, padded),
// queries once from global memory into registers.  Alternate steps
// accumulate into two chains, so consecutive MFMAs are independent.
template <int DIM, int METRIC, int C>
__global__ __launch_bounds__(256) void flat_gemm_f32(
    const float* __restrict__ rows, const float* __restrict__ norms, int64_t n,
    const float* __restrict__ queries, int64_t nq, BoundCoef bc, GemmArgs ga) {
    using G = GemmShape<DIM>;
    constexpr int NS = G::NS, SL = G::SL, SK = G::SK, NSLICE = G::NSLICE, SS = G::SS;
    extern __shared__ uint64_t lds[];
    float* xs = reinterpret_cast<float*>(lds);  // [2][32][SS]
    float* tva = xs + 2 * G::SLICE_FLOATS;      // [2][32] row norms vn
    float* tvb = tva + 2 * kGemmRows;           // [2][32] sqrt(vn), or 1 / sqrt(vn) for cosine
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, col = lane & 31;

    const int b = blockIdx.x, grp = 8 * ga.nqb;
    const int seg = 8 * (b / grp) + (b % 8);
    const int qb = (b % grp) / 8;

    // Lanes past the batch compute with query 0; their keys are never offered.
    const int64_t qid = (int64_t)qb * kGemmQueries + wave * 32 + col;
    const bool qvalid = qid < nq;
    float qreg[NS];
    float qsq = 0.0f;
    {
        const float* qp = queries + (qvalid ? qid : 0) * DIM + 4 * h;
#pragma unroll
        for (int g = 0; g < NS / 4; ++g) {
            const f4v v = *reinterpret_cast<const f4v*>(qp + 8 * g);
            qreg[4 * g + 0] = v.x;
            qreg[4 * g + 1] = v.y;
            qreg[4 * g + 2] = v.z;
            qreg[4 * g + 3] = v.w;
            qsq = fmaf(v.x, v.x, qsq);
            qsq = fmaf(v.y, v.y, qsq);
            qsq = fmaf(v.z, v.z, qsq);
            qsq = fmaf(v.w, v.w, qsq);
        }
    }
    const float qn = qsq + __shfl_xor(qsq, 32);
    const float sq = sqrtf(qn);
    const float rq = 1.0f / sq;  // inf for qn == 0: such keys take the tiny-product branch
    uint64_t lst[C];
#pragma unroll
    for (int i = 0; i < C; ++i) lst[i] = kEmptySlot;

    const int64_t seg0 = (int64_t)seg * ga.rows_per_seg;
    const int64_t seg1 = seg0 + ga.rows_per_seg < n ? seg0 + ga.rows_per_seg : n;
    const int64_t ntiles = seg1 > seg0 ? (seg1 - seg0 + kGemmRows - 1) / kGemmRows : 0;

    // Rows past the segment's end load the segment's last row (their keys
    // are never offered), so the loads need no branch.
    f4v pre[G::LOADS];
    auto load_slice = [&](int64_t tile, int part) {
#pragma unroll
        for (int u = 0; u < G::LOADS; ++u) {
            const int e = tid + 256 * u;
            const int r = e / G::F4_PER_ROW, i = e % G::F4_PER_ROW;
            int64_t row = seg0 + tile * kGemmRows + r;
            row = row < seg1 ? row : seg1 - 1;
            pre[u] = *reinterpret_cast<const f4v*>(rows + row * DIM + part * SK + 4 * i);
        }
    };
    auto store_slice = [&](int buf) {
        float* dst = xs + buf * G::SLICE_FLOATS;
#pragma unroll
        for (int u = 0; u < G::LOADS; ++u) {
            const int e = tid + 256 * u;
            const int r = e / G::F4_PER_ROW, i = e % G::F4_PER_ROW;
            *reinterpret_cast<f4v*>(dst + r * SS + 4 * i) = pre[u];
        }
    };
    auto load_norms = [&](int64_t tile) {
        if (tid < kGemmRows) {
            int64_t row = seg0 + tile * kGemmRows + tid;
            row = row < seg1 ? row : seg1 - 1;
            const float vn = norms[row];
            const int at = (int)(tile & 1) * kGemmRows + tid;
            tva[at] = vn;
            tvb[at] = METRIC == kMetricCosine ? (vn > 0.0f ? 1.0f / sqrtf(vn) : 0.0f) : sqrtf(vn);
        }
    };
    // Offers tile `tile`'s 16 keys per lane (tile < 0: nothing).
    auto offer = [&](const f16v& f, int64_t tile) {
        const int tb = (int)(tile & 1) * kGemmRows;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = 8 * (v >> 2) + 4 * h + (v & 3);
            const int64_t row = seg0 + tile * kGemmRows + m;
            const bool ok = qvalid && tile >= 0 && row < seg1;
            const float vn = tva[tb + m], wv = tvb[tb + m];
            float key;
            if (METRIC == kMetricIP) {
                key = -f[v] - (sq * wv) * bc.c_ip;
            } else if (METRIC == kMetricL2) {
                float dd = qn - 2.0f * f[v] + vn;
                dd = dd > 0.0f ? dd : 0.0f;
                key = dd - (qn + vn + 2.0f * (sq * wv)) * bc.c_l2;
            } else {
                key = (1.0f - f[v] * (rq * wv)) - bc.eps_cos;
                key = qn * vn < 1.03e-20f ? -1.0f : key;       // near the 1e-10 branch
                key = vn == 0.0f ? 1.0f - bc.eps_cos : key;  // both paths give exactly 1
            }
            key -= ga.abs_slack;
            list_insert<C>(lst, ok ? pack_slot(key, (uint32_t)row) : kEmptySlot);
        }
    };

    if (ntiles > 0) {
        load_slice(0, 0);
        store_slice(0);
    }
    __syncthreads();
    int buf = 0;
    f16v prev = {};
    for (int64_t t = 0; t < ntiles; ++t) {
        load_norms(t);
        f16v acc0 = {}, acc1 = {};
#pragma unroll
        for (int part = 0; part < NSLICE; ++part) {
            // Prefetch the next slice; past the last one, reload the last.
            int64_t ntile = part + 1 < NSLICE ? t : t + 1;
            int npart = part + 1 < NSLICE ? part + 1 : 0;
            if (ntile >= ntiles) {
                ntile = ntiles - 1;
                npart = NSLICE - 1;
            }
            load_slice(ntile, npart);
            const float* xl = xs + buf * G::SLICE_FLOATS + col * SS + 4 * h;
            f4v a = *reinterpret_cast<const f4v*>(xl);
#pragma unroll
            for (int g = 0; g < SL / 4; ++g) {
                // The next group's operand is read before this group's MFMAs.
                const f4v an = g + 1 < SL / 4 ? *reinterpret_cast<const f4v*>(xl + 8 * (g + 1)) : a;
                const int sb = part * SL + 4 * g;
                acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, qreg[sb + 0], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, qreg[sb + 1], acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, qreg[sb + 2], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, qreg[sb + 3], acc1, 0, 0, 0);
                a = an;
            }
            // The previous tile's keys (its norms were stored before the
            // last barrier and are overwritten only after the next one).
            if (part == 0) offer(prev, t - 1);
            // The other buffer was last read before the previous barrier.
            store_slice(buf ^ 1);
            __syncthreads();
            buf ^= 1;
        }
        prev = acc0 + acc1;
    }
    offer(prev, ntiles - 1);
    if (qvalid) {
        uint64_t* out = ga.lists + (((size_t)qid * ga.nseg + seg) * 2 + h) * C;
#pragma unroll
        for (int i = 0; i < C; ++i) out[i] = lst[i];
    }
}

// grid (1, nq): one block per query selects the kc smallest keys over its
// 2 nseg lists, then the exact rescore and proof of the streaming scan.
template <int NCH>
__global__ __launch_bounds__(256) void flat_lists_merge(
    const float* __restrict__ rows, const float* __restrict__ norms, int64_t n, int dim,
    const float* __restrict__ queries, int metric, int kc, int cap, int nlists, int list_len,
    const uint64_t* __restrict__ lists, FlatArgs fa) {
    extern __shared__ uint64_t lds[];
    __shared__ uint32_t cut_bits;
    const int lr = threadIdx.x & 15;
    const uint32_t q = blockIdx.y;
    const int dim4 = dim >> 2;
    const float* qp = queries + (int64_t)q * dim;
    f4v qv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = lr + 16 * c;
        qv[c] = idx < dim4 ? *reinterpret_cast<const f4v*>(qp + 4 * idx) : f4v{0.f, 0.f, 0.f, 0.f};
    }
    const uint64_t* lq = lists + (size_t)q * nlists * list_len;
    if (threadIdx.x == 0) cut_bits = 0xFFFFFFFFu;
    __syncthreads();
    // Smallest largest key over the full lists (ordered key bits).
    uint32_t mine = 0xFFFFFFFFu;
    for (int i = threadIdx.x; i < nlists; i += blockDim.x) {
        const uint64_t last = lq[(size_t)i * list_len + list_len - 1];
        if (last != kEmptySlot) mine = min(mine, (uint32_t)(last >> 32));
    }
    atomicMin(&cut_bits, mine);
    WaveTopK sel;
    block_select_lists(lq, (int64_t)nlists * list_len, lds, cap, kc, sel);  // ends in a barrier
    const float list_cut = cut_bits == 0xFFFFFFFFu ? kFltMax : from_ordered_bits(cut_bits);
    final_rescore_f4<NCH>(qv, rows, norms, n, dim, metric, q, lds, kc, fa, list_cut);
}

// ---------------------------------------------------------------------------

static bool gemm_dim_supported(int dim) {
    switch (dim) {
    case 64: case 96: case 128: case 192: case 256: case 384: return true;
    default: return false;
    }
}

bool plan_gemm(int64_t n, int dim, int64_t nq, int kc, GemmPlan* out) {
    static const int64_t min_batch = [] {
        const char* e = std::getenv("MANS_GEMM_MIN_BATCH");
        return e ? std::max<int64_t>(1, std::atoll(e)) : (int64_t)16;
    }();
    static const int64_t target = [] {
        const char* e = std::getenv("MANS_GEMM_BLOCKS");
        return e ? std::max<int64_t>(8, std::atoll(e)) : (int64_t)1024;
    }();
    if (!gemm_dim_supported(dim) || kc > kGemmMaxKc || nq < min_batch || n < kGemmMinRows)
        return false;
    GemmPlan p;
    p.kc = kc;
    p.cap = flat_cap_for(kc);
    p.nqb = (int)((nq + kGemmQueries - 1) / kGemmQueries);
    // About `target` blocks, a multiple of 8 segments of >= 1024 rows each
    // (the lane lists stay a small fraction of the rows they see).
    int64_t nseg = (target + p.nqb - 1) / p.nqb;
    nseg = (nseg + 7) / 8 * 8;
    int64_t max_seg = n / 1024 / 8 * 8;
    if (nseg > max_seg) nseg = max_seg;
    if (nseg < 8) nseg = 8;
    int64_t rps = (n + nseg - 1) / nseg;
    p.rows_per_seg = (rps + kGemmRows - 1) / kGemmRows * kGemmRows;
    p.nseg = (int)nseg;
    *out = p;
    return true;
}

size_t gemm_lists_bytes(const GemmPlan& p, int64_t nq) {
    return (size_t)nq * (size_t)p.nseg * 2 * gemm_list_len(p.kc) * sizeof(uint64_t);
}

template <int DIM, int C>
static hipError_t launch_gemm_dim_c(const GemmPlan& p, const float* rows, const float* norms,
                                    int64_t n, const float* queries, int64_t nq, int metric,
                                    const GemmArgs& ga, hipStream_t s) {
    const BoundCoef bc = make_bounds(DIM, 1.0 / 8388608.0);
    const dim3 grid((unsigned)(p.nseg * p.nqb));
    const size_t shmem = gemm_lds_bytes<DIM>();
    switch (metric) {
    case kMetricCosine:
        hipLaunchKernelGGL((flat_gemm_f32<DIM, kMetricCosine, C>), grid, dim3(256), shmem, s, rows,
                           norms, n, queries, nq, bc, ga);
        break;
    case kMetricL2:
        hipLaunchKernelGGL((flat_gemm_f32<DIM, kMetricL2, C>), grid, dim3(256), shmem, s, rows,
                           norms, n, queries, nq, bc, ga);
        break;
    case kMetricIP:
        hipLaunchKernelGGL((flat_gemm_f32<DIM, kMetricIP, C>), grid, dim3(256), shmem, s, rows,
                           norms, n, queries, nq, bc, ga);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int DIM>
static hipError_t launch_gemm_dim(const GemmPlan& p, const float* rows, const float* norms,
                                  int64_t n, const float* queries, int64_t nq, int metric,
                                  const GemmArgs& ga, hipStream_t s) {
    return gemm_list_len(p.kc) == 4
               ? launch_gemm_dim_c<DIM, 4>(p, rows, norms, n, queries, nq, metric, ga, s)
               : launch_gemm_dim_c<DIM, 8>(p, rows, norms, n, queries, nq, metric, ga, s);
}

template <int NCH>
static void launch_lists_merge(const GemmPlan& p, const float* rows, const float* norms, int64_t n,
                               int dim, const float* queries, int64_t nq, int metric,
                               const uint64_t* lists, const FlatArgs& fa, hipStream_t s) {
    size_t shmem = sizeof(uint64_t) * 4 * (size_t)p.cap;
    hipLaunchKernelGGL(flat_lists_merge<NCH>, dim3(1, (unsigned)nq), dim3(256), shmem, s, rows,
                       norms, n, dim, queries, metric, p.kc, p.cap, 2 * p.nseg,
                       gemm_list_len(p.kc), lists, fa);
}

hipError_t launch_flat_gemm(const GemmPlan& p, const float* rows, const float* norms, int64_t n,
                            int dim, const float* queries, int64_t nq, int metric,
                            uint64_t* lists, hipStream_t s) {
    GemmArgs ga;
    ga.nseg = p.nseg;
    ga.nqb = p.nqb;
    ga.rows_per_seg = p.rows_per_seg;
    // Products and partial sums flushed below 2^-126 lose at most 2^-126
    // each: 2 dim such terms in a dot, counted twice for L2's -2 dot.
    ga.abs_slack = (float)(4.0 * dim * 1.1754943508222875e-38);
    ga.lists = lists;
    hipError_t e;
    switch (dim) {
    case 64: e = launch_gemm_dim<64>(p, rows, norms, n, queries, nq, metric, ga, s); break;
    case 96: e = launch_gemm_dim<96>(p, rows, norms, n, queries, nq, metric, ga, s); break;
    case 128: e = launch_gemm_dim<128>(p, rows, norms, n, queries, nq, metric, ga, s); break;
    case 192: e = launch_gemm_dim<192>(p, rows, norms, n, queries, nq, metric, ga, s); break;
    case 256: e = launch_gemm_dim<256>(p, rows, norms, n, queries, nq, metric, ga, s); break;
    case 384: e = launch_gemm_dim<384>(p, rows, norms, n, queries, nq, metric, ga, s); break;
    default: return hipErrorInvalidValue;
    }
    return e;
}

hipError_t launch_flat_gemm_merge(const GemmPlan& p, const float* rows, const float* norms,
                                  int64_t n, int dim, const float* queries, int64_t nq, int metric,
                                  const uint64_t* lists, const FlatBuffers& b, int k, int k_stride,
                                  hipStream_t s) {
    FlatArgs fa = {};
    fa.out_dist = b.out_dist;
    fa.out_ids = b.out_ids;
    fa.status = b.status;
    fa.k = k;
    fa.k_stride = k_stride;
    switch (flat_nch_for_dim(dim)) {
    case 1: launch_lists_merge<1>(p, rows, norms, n, dim, queries, nq, metric, lists, fa, s); break;
    case 2: launch_lists_merge<2>(p, rows, norms, n, dim, queries, nq, metric, lists, fa, s); break;
    case 3: launch_lists_merge<3>(p, rows, norms, n, dim, queries, nq, metric, lists, fa, s); break;
    case 4: launch_lists_merge<4>(p, rows, norms, n, dim, queries, nq, metric, lists, fa, s); break;
    case 6: launch_lists_merge<6>(p, rows, norms, n, dim, queries, nq, metric, lists, fa, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mans
