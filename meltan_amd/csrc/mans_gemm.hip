// Batched exact flat scan on gfx950: FlatGPUSearch.batchSearch
// (FlatGPUSearch.swift:103-181) for batches of queries, as an fp32 MFMA
// contraction with the top-k selection fused into its epilogue, followed by
// the per-query merge, exact rescore and proof of the streaming scan.
#include <algorithm>
#include <type_traits>
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

// ---------------------------------------------------------------------------
// Batched queries on bf16 MFMA with fp32-level accuracy (split products).
//
// Every query value x in [2^-50, 2^50] (or 0) is split into bf16 parts
// x = xh + xl + r: xh = bf16(x), xl = bf16(x - xh) (x - xh is exact in
// fp32), both rounded to nearest even, so |x - xh| <= 2^-8 |x| and
// |r| <= 2^-16 |x|.  A row keeps only its high part vh = bf16(v) (same
// rounding) and e_v >= ||v - vh||, the norm of its remainder (summed in
// double, rounded up to fp32).  The contraction sums qh vh and ql vh with
// v_mfma_f32_32x32x16_bf16 into two fp32 accumulators (each product of two
// bf16 values is exact in fp32), added at the end.  Since
//   q.v = (qh + ql) vh + r vh + q (v - vh),
// the sum f satisfies
//   |f - q.v| <= g sum |q_i v_i| + ||q|| e_v,
//   g = 1.024 gamma_d (u = 2^-23) + 1.01 2^-16 + 2^-22
// (the accumulations over (1 + 2^-8)^3 sum |q_i v_i|, |r vh| and the final
// additions; the last term by Cauchy-Schwarz).  The keys are the fp32
// path's lower bounds computed with a unit roundoff u_eff for which
// gamma_d(u_eff) = g (>= every other error term those bounds cover), minus
// the row's remainder term: ||q|| e_v for inner product, 2 ||q|| e_v for
// L2 and e_v / ||v|| for cosine, each times 1 + 2^-12 (which covers the
// roundings of the norms and of the key arithmetic).  Values outside the
// range (huge, tiny, inf, NaN) are flagged when split: a corpus with any
// such value keeps the fp32 contraction, and a flagged query is re-run by
// the streaming scan.
//
// Queries are stored per 8 elements as [8 hi | 8 lo] (32 bytes); rows as
// their dim bf16 high parts (half the fp32 size) plus e_v.
//
// The epilogue admits a key only when it is at or below the lane's
// threshold (its largest slot, or the query's bound): a first launch over
// a sample of rows (the first rows of 64 spread segments) gives each query
// its bound, the kc-th smallest slot of the sampled lists; no slot above it
// is among the query's kc smallest, and the merge's proof cutoff takes it
// into account.

__device__ __forceinline__ uint32_t bf16_rne_bits(float x) {
    const uint32_t b = __float_as_uint(x);
    return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ bool split_in_range(float x) {
    const float a = fabsf(x);
    return a == 0.0f || (a >= 0x1p-50f && a <= 0x1p50f);
}

// One thread per 8 elements of `count` queries of dim (multiple of 8)
// floats; bad[query] gets 1 for a value outside the range.
__global__ void split_queries_kernel(const float* __restrict__ src, int64_t count, int dim,
                                     uint32_t* __restrict__ dst, uint32_t* __restrict__ bad) {
    const int cpr = dim >> 3;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= count * cpr) return;
    const int64_t row = t / cpr;
    const int c = (int)(t - row * cpr);
    const float* s = src + row * dim + 8 * c;
    const f4v a = *reinterpret_cast<const f4v*>(s);
    const f4v b = *reinterpret_cast<const f4v*>(s + 4);
    const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t hi[4], lo[4];
    bool ok = true;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        const uint32_t h0 = bf16_rne_bits(x[i]), h1 = bf16_rne_bits(x[i + 1]);
        const float r0 = x[i] - __uint_as_float(h0 << 16);
        const float r1 = x[i + 1] - __uint_as_float(h1 << 16);
        hi[i / 2] = h0 | (h1 << 16);
        lo[i / 2] = bf16_rne_bits(r0) | (bf16_rne_bits(r1) << 16);
        ok = ok && split_in_range(x[i]) && split_in_range(x[i + 1]);
    }
    uint32_t* d = dst + row * dim + 8 * c;
    *reinterpret_cast<i4v*>(d) = i4v{(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    *reinterpret_cast<i4v*>(d + 4) = i4v{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
    if (!ok) atomicOr(bad + row, 1u);
}

hipError_t launch_split_queries(const float* src, int64_t count, int dim, uint32_t* dst,
                                uint32_t* bad, hipStream_t s) {
    const int64_t threads = count * (dim / 8);
    if (threads <= 0) return hipSuccess;
    hipLaunchKernelGGL(split_queries_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       s, src, count, dim, dst, bad);
    return hipGetLastError();
}

// One wave per row of `count` rows of dim (multiple of 8) floats: hi gets
// the row's bf16 high parts and recs two record planes of `count` float4s:
// {vn, 1 / sqrt(vn), e' / sqrt(vn), 0} (cosine) and {vn, sqrt(vn), e', 0}
// (L2, inner product), with vn the row's squared norm and
// e' >= (1 + 2^-12) ||v - vh|| (summed in double, rounded up); bad[0] gets
// 1 for a value outside the range.
__global__ __launch_bounds__(256) void split_rows_kernel(const float* __restrict__ src,
                                                         const float* __restrict__ norms,
                                                         int64_t count, int dim,
                                                         uint16_t* __restrict__ hi,
                                                         float* __restrict__ recs,
                                                         uint32_t* __restrict__ bad) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= count) return;
    const float* s = src + row * dim;
    double acc = 0.0;
    bool ok = true;
    for (int c = lane; c < dim / 8; c += 64) {
        const f4v a = *reinterpret_cast<const f4v*>(s + 8 * c);
        const f4v b = *reinterpret_cast<const f4v*>(s + 8 * c + 4);
        const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t h[4];
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            const uint32_t h0 = bf16_rne_bits(x[i]), h1 = bf16_rne_bits(x[i + 1]);
            // The remainders are exact in fp32, their squares in double.
            const double r0 = (double)(x[i] - __uint_as_float(h0 << 16));
            const double r1 = (double)(x[i + 1] - __uint_as_float(h1 << 16));
            acc += r0 * r0;
            acc += r1 * r1;
            h[i / 2] = h0 | (h1 << 16);
            ok = ok && split_in_range(x[i]) && split_in_range(x[i + 1]);
        }
        *reinterpret_cast<i4v*>(hi + row * dim + 8 * c) = i4v{(int)h[0], (int)h[1], (int)h[2], (int)h[3]};
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
    if (lane == 0) {
        // The double sum and square root are off by far less than 2^-40;
        // the factor 1 + 2^-12 covers the roundings of the norms and of the
        // key arithmetic that use e'.
        const double e = sqrt(acc) * (1.0 + 0x1p-40) * (1.0 + 0x1p-12);
        float f = (float)e;
        if ((double)f < e) f = __uint_as_float(__float_as_uint(f) + 1u);
        const float vn = norms[row];
        const float ws = sqrtf(vn);
        const float wr = vn > 0.0f ? 1.0f / ws : 0.0f;
        f4v* r4 = reinterpret_cast<f4v*>(recs);
        r4[row] = f4v{vn, wr, f * wr, 0.0f};
        r4[count + row] = f4v{vn, ws, f, 0.0f};
    }
    if (!ok) atomicOr(bad, 1u);
}

hipError_t launch_split_rows(const float* src, const float* norms, int64_t count, int dim,
                             uint16_t* hi, float* recs, uint32_t* bad, hipStream_t s) {
    if (count <= 0) return hipSuccess;
    hipLaunchKernelGGL(split_rows_kernel, dim3((unsigned)((count + 3) / 4)), dim3(256), 0, s, src,
                       norms, count, dim, hi, recs, bad);
    return hipGetLastError();
}

typedef __bf16 bf8v __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// s_waitcnt vmcnt(N) through the builtin, so the compiler's own wait
// insertion knows which loads are complete (expcnt and lgkmcnt at their
// no-wait values).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

constexpr int kBf2Waves = 8;
constexpr int kBf2Slots = 3;     // row tile ring: tile t + 2 loads while tile t is used
constexpr int kBf2RecSlots = 4;  // row record ring
constexpr int kBf2Lists = 4;     // sampled launch: lane lists per query and segment
constexpr int kBf2ListLen = 4;   // sampled launch: slots per lane list
constexpr int kBf2Cap = 64;      // full launch: candidate slots per query and segment
// The full launch's 32 x 32 sums of a query group, query-major: query q's
// 32 rows start at q * kBf2DotStride + (q / 16) * 32 floats (16-byte
// aligned; the key waves' two query halves fall on different banks).
constexpr int kBf2DotStride = 36;
constexpr int kBf2DotGroup = 32 * kBf2DotStride + 32;

// The chunk permutation of row r in a tile whose rows are cpr 16-byte
// chunks: chunk c sits at c ^ bf2_swz(r).  With a row stride of 8 chunks
// mod 16 (128 bytes mod 256), rows r and r + 1 fall in different 128-byte
// halves, so (r / 2) & 7 keeps the 16 rows read by 16 lanes at 16 distinct
// 16-byte bank groups; otherwise r & swz with swz + 1 the largest power of
// two (at most 16) dividing cpr.
template <int CPR>
struct Bf2Swizzle {
    static constexpr int LOWBIT = CPR & -CPR;
    static constexpr int SWZ = (CPR & 15) == 8 ? 7 : (LOWBIT < 16 ? LOWBIT : 16) - 1;
    __device__ static int of(int r) { return (CPR & 15) == 8 ? (r >> 1) & 7 : r & SWZ; }
};

// ---------------------------------------------------------------------------
// Work split: 8 waves serve 128 queries over one segment of rows; wave w
// takes query group w & 3 (32 queries) and half w >> 2 of the k range, so a
// wave keeps only its half of the query's split parts in registers and two
// waves fit on a SIMD.  Per 32-row tile the two halves' sums are exchanged
// through LDS and added (the same IEEE sum in either wave), and each wave
// keys 8 of the 16 rows a lane holds.  The sampled launch (no bounds)
// inserts them into sorted lane lists (4 lists per query and segment: half
// x lane half), lowering each lane's threshold as its list fills; the full
// launch appends keys at or below the query's bound to a candidate buffer
// per query and segment.
//
// Tiles reach LDS by direct global-to-LDS loads (global_load_lds, 16 bytes
// per lane) into a ring of three slots, two tiles ahead; each wave issues
// the same number of row loads per tile (padded) and wave 0 one more, the
// tile's row records.  A slot holds, per k half, 32 rows x CPR swizzled
// 16-byte chunks.
template <int DIM>
struct Bf2Shape {
    static constexpr int NS = DIM / 16;  // MFMA k-steps per row
    static constexpr int NH = NS / 2;    // k-steps per half
    static constexpr int CPR = 2 * NH;   // 16-byte chunks of a row per half
    using Swz = Bf2Swizzle<CPR>;
    static constexpr int HALF_CHUNKS = kGemmRows * CPR;
    static constexpr int TILE_CHUNKS = 2 * HALF_CHUNKS;
    static constexpr int LOADS = (TILE_CHUNKS + 64 * kBf2Waves - 1) / (64 * kBf2Waves);
    static constexpr int SLOT_BYTES = 16 * 64 * kBf2Waves * LOADS;
    static_assert(DIM % 32 == 0, "unsupported dimension");
};

template <int DIM>
constexpr size_t bf2_lds_bytes() {
    return kBf2Slots * (size_t)Bf2Shape<DIM>::SLOT_BYTES + 16 * kBf2RecSlots * kGemmRows +
           16 * 2 * 2 * kBf2Waves * 64;
}

struct Bf2Args {
    int nseg;
    int nqb;
    int64_t rows_per_seg;     // multiple of kGemmRows
    int64_t seg_rows;         // rows scanned from each segment's start
    float abs_slack;
    const uint64_t* qbound;   // full launch: per query
    // Sampled launch: lane lists [nq][nseg][kBf2Lists][kBf2ListLen].  Full launch:
    // candidate buffers [nq][nseg][kBf2Cap], unsorted, padded with
    // kEmptySlot; a buffer that fills up sets bit 2 of qflag[query].
    uint64_t* lists;
    uint32_t* qflag;
};

// The lower-bound key of a row from its dot f with the query (the split
// contraction's sum), the query's qn, sqrt(qn), 1 / sqrt(qn) and cosine
// threshold vn_tiny, and the row's record {vn, w, c, 0}.
template <int METRIC>
__device__ __forceinline__ float bf2_key(float f, float qn, float sq, float rq, float vn_tiny,
                                         const f4v& rec, const BoundCoef& bc, float eps_all,
                                         float abs_slack) {
    const float vn = rec.x, wv = rec.y, vc = rec.z;
    if (METRIC == kMetricIP) return (-f - sq * (wv * bc.c_ip + vc)) - abs_slack;
    if (METRIC == kMetricL2) {
        float dd = qn - 2.0f * f + vn;
        dd = dd > 0.0f ? dd : 0.0f;
        return (dd - ((qn + vn + 2.0f * (sq * wv)) * bc.c_l2 + sq * (2.0f * vc))) - abs_slack;
    }
    // A zero row has wv = vc = 0 and key 1 - eps (both paths give exactly
    // 1); rows with qn vn below 1.03e-20 get -1 (the formula's 1e-10 branch
    // is near).
    const float k = (1.0f - f * (rq * wv)) - (eps_all + vc);
    return vn < vn_tiny ? -1.0f : k;
}

// One wave's work over the block's segment; KP: the wave's k half.
template <int DIM, int METRIC, int C, bool BOUNDED, int KP>
__device__ __forceinline__ void bf2_segment(const uint16_t* __restrict__ hi_rows,
                                                    const f4v* __restrict__ recs, int64_t n,
                                                    const uint32_t* __restrict__ split_q,
                                                    const float* __restrict__ queries, int64_t nq,
                                                    const BoundCoef& bc, const Bf2Args& ga,
                                                    int wave) {
    using G = Bf2Shape<DIM>;
    constexpr int NH = G::NH, CPR = G::CPR;
    extern __shared__ uint64_t lds[];
    uint8_t* ring = reinterpret_cast<uint8_t*>(lds);                       // [slot][half][32][CPR][16]
    f4v* trec = reinterpret_cast<f4v*>(ring + kBf2Slots * G::SLOT_BYTES);  // [rec slot][32]
    f4v* xa = trec + kBf2RecSlots * kGemmRows;  // partner sums [2][wave][64], first four
    f4v* xb = xa + 2 * kBf2Waves * 64;          // and second four
    const int lane = threadIdx.x & 63;
    const int qg = wave & 3;
    const int h = lane >> 5, col = lane & 31;

    const int b = blockIdx.x, grp = 8 * ga.nqb;
    const int seg = 8 * (b / grp) + (b % 8);
    const int qb = (b % grp) / 8;

    const int64_t qid = (int64_t)qb * kGemmQueries + qg * 32 + col;
    const bool qvalid = qid < nq;
    const int64_t qrow = qvalid ? qid : 0;
    bf8v qh[NH], ql[NH];
#pragma unroll
    for (int s = 0; s < NH; ++s) {
        const uint32_t* p = split_q + qrow * DIM + 8 * (2 * (KP * NH + s) + h);
        qh[s] = __builtin_bit_cast(bf8v, *reinterpret_cast<const i4v*>(p));
        ql[s] = __builtin_bit_cast(bf8v, *reinterpret_cast<const i4v*>(p + 4));
    }
    // The query norm in the fp32 path's order (fmaf over float4 chunks).
    float qsq = 0.0f;
    {
        const float* qp = queries + qrow * DIM + 4 * h;
#pragma unroll
        for (int g = 0; g < DIM / 8; ++g) {
            const f4v v = *reinterpret_cast<const f4v*>(qp + 8 * g);
            qsq = fmaf(v.x, v.x, qsq);
            qsq = fmaf(v.y, v.y, qsq);
            qsq = fmaf(v.z, v.z, qsq);
            qsq = fmaf(v.w, v.w, qsq);
        }
    }
    const float qn = qsq + __shfl_xor(qsq, 32);
    const float sq = sqrtf(qn);
    const float rq = 1.0f / sq;
    const float vn_tiny = (1.03e-20f / qn) * 1.0001f;
    const float eps_all = bc.eps_cos + ga.abs_slack;
    uint64_t lst[C];
#pragma unroll
    for (int i = 0; i < C; ++i) lst[i] = kEmptySlot;
    const uint64_t bound = BOUNDED && qvalid ? ga.qbound[qid] : kEmptySlot;
    float thr = !qvalid ? -__int_as_float(0x7F800000)
                        : (bound == kEmptySlot ? __int_as_float(0x7F800000) : slot_key(bound));
    // Full launch: candidates so far in this query's region for this k
    // half (the same in the query's two lanes).
    uint32_t cnt = 0;
    uint64_t* region = ga.lists + ((size_t)qrow * ga.nseg + seg) * kBf2Cap + KP * (kBf2Cap / 2);

    const int64_t seg0 = (int64_t)seg * ga.rows_per_seg;
    const int64_t seg1 = seg0 + ga.seg_rows < n ? seg0 + ga.seg_rows : n;
    const int ntiles = seg1 > seg0 ? (int)((seg1 - seg0 + kGemmRows - 1) / kGemmRows) : 0;

    // Per-lane byte offsets of this lane's chunks within a tile (row r of
    // the tile), the same for every tile; padding positions past the tile
    // load the tile's first chunk.
    uint32_t voff[G::LOADS];
    int vrow[G::LOADS];
#pragma unroll
    for (int u = 0; u < G::LOADS; ++u) {
        int p = (wave * G::LOADS + u) * 64 + lane;
        p = p < G::TILE_CHUNKS ? p : 0;
        const int half = p / G::HALF_CHUNKS, rem = p - half * G::HALF_CHUNKS;
        const int r = rem / CPR, qq = rem - r * CPR;
        const int c = qq ^ G::Swz::of(r);
        vrow[u] = r;
        voff[u] = (uint32_t)(r * DIM * 2 + half * (16 * CPR) + 16 * c);
    }
    const uint8_t* seg_base = reinterpret_cast<const uint8_t*>(hi_rows + seg0 * DIM);
    wait_vmcnt<0>();  // the query parts, before the first tile loads

    // Loads tile t into ring slot `slot` (both k halves) and (wave 0) its
    // records into record slot t % 4.  Rows past the segment's end load its
    // last row.
    auto issue = [&](int t, int slot) {
        if (t >= ntiles) return;
        const int64_t left = seg1 - (seg0 + (int64_t)t * kGemmRows);
        const uint8_t* tb = seg_base + (int64_t)t * (kGemmRows * DIM * 2);
        uint8_t* dst = ring + slot * G::SLOT_BYTES + wave * G::LOADS * 1024;
        if (left >= kGemmRows) {
#pragma unroll
            for (int u = 0; u < G::LOADS; ++u)
                __builtin_amdgcn_global_load_lds(tb + voff[u], (lds_ptr_t)(dst + u * 1024), 16, 0, 0);
        } else {
#pragma unroll
            for (int u = 0; u < G::LOADS; ++u) {
                const int back = vrow[u] < left ? 0 : vrow[u] - (int)left + 1;
                __builtin_amdgcn_global_load_lds(tb + voff[u] - back * (DIM * 2),
                                                 (lds_ptr_t)(dst + u * 1024), 16, 0, 0);
            }
        }
        if (wave == 0) {
            int64_t row = seg0 + (int64_t)t * kGemmRows + (lane & 31);
            row = row < seg1 ? row : seg1 - 1;
            if (lane < kGemmRows)
                __builtin_amdgcn_global_load_lds(recs + row,
                                                 (lds_ptr_t)(trec + (t & (kBf2RecSlots - 1)) * kGemmRows),
                                                 16, 0, 0);
        }
    };
    // Keys of tile t's 8 rows of this lane (rows 8 (v / 4) + 4 h + v % 4
    // for v = 8 KP .. 8 KP + 7): this wave's sums plus the partner's, read
    // from LDS buffer t & 1.
    auto keys = [&](const float (&keep)[8], int t, float (&key)[8]) {
        const int xo = ((t & 1) * kBf2Waves + ((wave + 4) & 7)) * 64 + lane;
        const f4v r0 = xa[xo];
        const f4v r1 = xb[xo];
        const f4v* tr = trec + (t & (kBf2RecSlots - 1)) * kGemmRows;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int v = 8 * KP + i;
            const int m = 8 * (v >> 2) + 4 * h + (v & 3);
            const float fv = keep[i] + (i < 4 ? r0[i] : r1[i - 4]);
            key[i] = bf2_key<METRIC>(fv, qn, sq, rq, vn_tiny, tr[m], bc, eps_all, ga.abs_slack);
        }
    };
    // The full launch appends keys at or below the query's bound to the
    // query's region for this k half (its two lanes, h = 0 and 1, take
    // consecutive slots by ballot; the threshold never changes); the
    // sampled launch inserts into the lane's sorted list and lowers the
    // lane's threshold as the list fills.
    auto offer = [&](const float (&key)[8], int t) {
        float mn = key[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) mn = fminf(mn, key[i]);
        if (BOUNDED) {
            if (__builtin_amdgcn_ballot_w64(mn <= thr) == 0) return;
            const int64_t base = seg0 + (int64_t)t * kGemmRows;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const bool hit = key[i] <= thr;
                const uint64_t m = __builtin_amdgcn_ballot_w64(hit);
                if (m == 0) continue;
                const uint32_t b0 = (uint32_t)(m >> col) & 1u, b1 = (uint32_t)(m >> (col + 32)) & 1u;
                const uint32_t pos = cnt + (h ? b0 : 0u);
                if (hit && pos < (uint32_t)(kBf2Cap / 2)) {
                    const int v = 8 * KP + i;
                    const int mrow = 8 * (v >> 2) + 4 * h + (v & 3);
                    region[pos] = pack_slot(key[i], (uint32_t)(base + mrow));
                }
                cnt += b0 + b1;
            }
            return;
        }
        if (mn <= thr) {
            const int64_t base = seg0 + (int64_t)t * kGemmRows;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (key[i] <= thr) {
                    const int v = 8 * KP + i;
                    const int m = 8 * (v >> 2) + 4 * h + (v & 3);
                    list_insert<C>(lst, pack_slot(key[i], (uint32_t)(base + m)));
                    thr = lst[C - 1] == kEmptySlot ? thr : slot_key(lst[C - 1]);
                }
            }
        }
    };
    // Tile t's sums: the partner half's 8 (rows it keys) go to LDS buffer
    // t & 1, this wave's 8 stay in `keep`.
    auto send = [&](const f16v& part, int t, float (&keep)[8]) {
        constexpr int other = 8 * (1 - KP), my0 = 8 * KP;
        const int xo = ((t & 1) * kBf2Waves + wave) * 64 + lane;
        xa[xo] = f4v{part[other], part[other + 1], part[other + 2], part[other + 3]};
        xb[xo] = f4v{part[other + 4], part[other + 5], part[other + 6], part[other + 7]};
#pragma unroll
        for (int i = 0; i < 8; ++i) keep[i] = part[my0 + i];
    };

    issue(0, 0);
    issue(1, 1);
    float keep[8] = {};
    int cslot = 0, islot = 2;  // t % 3 and (t + 2) % 3
    for (int t = 0; t < ntiles; ++t) {
        // Tile t is in LDS once this wave's loads of it are done (those of
        // tile t + 1 may still be in flight); the barrier publishes every
        // wave's loads and parts and frees slot (t - 1) % 3 for tile t + 2.
        if (t + 1 < ntiles) {
            if (wave == 0) wait_vmcnt<G::LOADS + 1>();
            else wait_vmcnt<G::LOADS>();
        } else {
            wait_vmcnt<0>();
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue(t + 2, islot);
        // Tile t - 1's keys (t + 3 selects its buffers; for t = 0 they are
        // never offered).
        float key[8];
        keys(keep, t + 3, key);
        const uint8_t* xl = ring + cslot * G::SLOT_BYTES + KP * (16 * G::HALF_CHUNKS) + col * CPR * 16;
        const int sw = G::Swz::of(col);
        f16v acc = {};
#pragma unroll
        for (int s = 0; s < NH; ++s) {
            const int c = 2 * s + h;
            const bf8v ah = __builtin_bit_cast(bf8v, *reinterpret_cast<const i4v*>(xl + 16 * (c ^ sw)));
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, qh[s], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, ql[s], acc, 0, 0, 0);
        }
        if (t > 0) offer(key, t - 1);
        send(acc, t, keep);
        cslot = cslot == kBf2Slots - 1 ? 0 : cslot + 1;
        islot = islot == kBf2Slots - 1 ? 0 : islot + 1;
    }
    if (ntiles > 0) {
        __syncthreads();  // the last tile's partner sums
        float key[8];
        keys(keep, ntiles - 1 + 4, key);
        // Rows past the segment's end.
        const int64_t left = seg1 - (seg0 + (int64_t)(ntiles - 1) * kGemmRows);
        if (left < kGemmRows) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int v = 8 * KP + i;
                const int m = 8 * (v >> 2) + 4 * h + (v & 3);
                key[i] = m < left ? key[i] : __int_as_float(0x7F800000);
            }
        }
        offer(key, ntiles - 1);
    }
    if (BOUNDED) {
        // Pads the region with empty slots (lane h takes half of them); a
        // region that filled up (it may have turned keys away) flags its
        // query, which the streaming scan runs again.  The buffer's last
        // slot is filled only then, so the merge's full-list cut stays
        // empty.
        if (qvalid) {
#pragma unroll
            for (int j = 0; j < kBf2Cap / 4; ++j) {
                const uint32_t slot = (uint32_t)(h * (kBf2Cap / 4) + j);
                if (slot >= cnt) region[slot] = kEmptySlot;
            }
            if (h == 0 && cnt >= (uint32_t)(kBf2Cap / 2)) atomicOr(ga.qflag + qid, 2u);
        }
    } else if (qvalid) {
        uint64_t* out = ga.lists + (((size_t)qid * ga.nseg + seg) * kBf2Lists + 2 * KP + h) * C;
#pragma unroll
        for (int i = 0; i < C; ++i) out[i] = lst[i];
    }
}

// grid: nseg * nqb blocks (1-D, XCD mapping as flat_gemm_f32); block 512.
// hi_rows: the rows' bf16 high parts; recs: per row {vn, w, c, 0} of the
// metric (w = sqrt(vn), or 1 / sqrt(vn) for cosine; c the remainder term
// without ||q||: e' for inner product and L2, e' / ||v|| for cosine);
// split_q: the queries' split parts.
template <int DIM, int METRIC, int C, bool BOUNDED>
__global__ __launch_bounds__(512, 1) void flat_gemm_bf16x2(
    const uint16_t* __restrict__ hi_rows, const f4v* __restrict__ recs, int64_t n,
    const uint32_t* __restrict__ split_q, const float* __restrict__ queries, int64_t nq,
    BoundCoef bc, Bf2Args ga) {
    // The k half is uniform over a wave: a scalar branch.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (wave < 4)
        bf2_segment<DIM, METRIC, C, BOUNDED, 0>(hi_rows, recs, n, split_q, queries, nq, bc, ga, wave);
    else
        bf2_segment<DIM, METRIC, C, BOUNDED, 1>(hi_rows, recs, n, split_q, queries, nq, bc, ga, wave);
}

// grid (1, nq), block 256: bound[q] = a slot with the key B and the largest
// id, B the largest exact distance (host formulas, dots.c order) among the
// k rows with the smallest keys in the query's sampled lists.  The k-th
// smallest exact distance over all rows is at most B, so rows with keys
// above B are not among the k nearest: the full launch admits only keys at
// or below B.  kEmptySlot when the lists hold fewer than k rows.  Each
// 16-lane group rescores rows with chain_dot (the merge's dots.c order).
template <int NCH>
__global__ __launch_bounds__(256) void lists_exact_bound(
    int k, int64_t per_query, const uint64_t* __restrict__ lists, const float* __restrict__ rows,
    const float* __restrict__ norms, int dim, const float* __restrict__ queries, int metric,
    uint64_t* __restrict__ bound) {
    extern __shared__ uint64_t lds[];
    __shared__ uint32_t s_ids[kGemmMaxKc];
    __shared__ int s_cnt;
    __shared__ uint32_t s_max;
    const int tid = threadIdx.x, lr = tid & 15, grp = tid >> 4;
    const uint32_t q = blockIdx.y;
    const uint64_t* src = lists + (size_t)q * per_query;
    const uint64_t kth = block_kth_slot(src, per_query, k, lds);
    if (kth == kEmptySlot) {
        if (tid == 0) bound[q] = kEmptySlot;
        return;
    }
    if (tid == 0) {
        s_cnt = 0;
        s_max = 0;
    }
    __syncthreads();
    // The lists hold each row at most once: exactly k slots are <= kth.
    const bool in_lds = per_query <= kKthLdsSlots;
    for (int64_t i = tid; i < per_query; i += blockDim.x) {
        const uint64_t s = in_lds ? lds[i] : src[i];
        if (s <= kth) s_ids[atomicAdd(&s_cnt, 1)] = slot_id(s);
    }
    __syncthreads();
    const int dim4 = dim >> 2;
    const float* qp = queries + (size_t)q * dim;
    f4v qv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = lr + 16 * c;
        qv[c] = idx < dim4 ? *reinterpret_cast<const f4v*>(qp + 4 * idx) : f4v{0.f, 0.f, 0.f, 0.f};
    }
    const float qn = metric == kMetricIP ? 0.0f : chain_dot<NCH>(qv, qv, dim4);
    const int cnt = s_cnt;
    for (int j = grp; j < cnt; j += 16) {
        const uint32_t id = s_ids[j];
        const float* rp = rows + (size_t)id * dim;
        f4v rv[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int idx = lr + 16 * c;
            rv[c] = idx < dim4 ? *reinterpret_cast<const f4v*>(rp + 4 * idx) : f4v{0.f, 0.f, 0.f, 0.f};
        }
        const float dot = chain_dot<NCH>(qv, rv, dim4);
        if (lr == 0) atomicMax(&s_max, ordered_bits(host_distance(dot, qn, norms[id], metric)));
    }
    __syncthreads();
    if (tid == 0) bound[q] = ((uint64_t)s_max << 32) | 0xFFFFFFFFull;
}

// grid (1, nq): one block per query selects the kc smallest keys over its
// 2 nseg lists, then the exact rescore and proof of the streaming scan.
template <int NCH>
__global__ __launch_bounds__(256) void flat_lists_merge(
    const float* __restrict__ rows, const float* __restrict__ norms, int64_t n, int dim,
    const float* __restrict__ queries, int metric, int kc, int cap, int nlists, int list_len,
    const uint64_t* __restrict__ lists, const uint64_t* __restrict__ qbound,
    const uint32_t* __restrict__ qbad, FlatArgs fa) {
    extern __shared__ uint64_t lds[];
    const int tid = threadIdx.x, lr = tid & 15;
    const uint32_t q = blockIdx.y;
    const int dim4 = dim >> 2;
    const float* qp = queries + (int64_t)q * dim;
    f4v qv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = lr + 16 * c;
        qv[c] = idx < dim4 ? *reinterpret_cast<const f4v*>(qp + 4 * idx) : f4v{0.f, 0.f, 0.f, 0.f};
    }
    // q.q in the dots.c order (every lane of a 16-lane group gets it).
    const float qn = metric == kMetricIP ? 0.0f : chain_dot<NCH>(qv, qv, dim4);
    const uint64_t* lq = lists + (size_t)q * nlists * list_len;
    const int64_t total = (int64_t)nlists * list_len;
    uint64_t* top = lds;         // 256 slots
    uint64_t* res = lds + 256;   // 256 slots
    uint64_t* cand = lds + 512;  // the lists' slots, then the rescore stage
    // Smallest largest slot over the full lists: its key bounds the rows
    // the lists turned away.
    uint64_t mine = kEmptySlot;
    for (int i = tid; i < nlists; i += blockDim.x) {
        const uint64_t last = lq[(size_t)i * list_len + list_len - 1];
        mine = last < mine ? last : mine;
    }
    const uint64_t full_cut = block_reduce_u64<false>(mine);
    const bool in_lds = total <= kKthLdsSlots;
    __shared__ uint32_t hist[256];
    __shared__ int ntop, nkept;
    if (tid == 0) {
        ntop = 0;
        nkept = 0;
    }
    __syncthreads();
    // The non-empty slots, compacted into LDS when they fit (in any order).
    if (in_lds)
        for (int64_t i = tid; i < total; i += blockDim.x) {
            const uint64_t s = lq[i];
            if (s != kEmptySlot) cand[atomicAdd(&nkept, 1)] = s;
        }
    __syncthreads();
    const int64_t nslots = in_lds ? (int64_t)nkept : total;
    // The kc smallest slots (empty slots are the largest values and are
    // never taken).
    auto get = [&](int64_t i) { return in_lds ? cand[i] : lq[i]; };
    uint64_t kth;
    const uint64_t sel = block_radix_cut(get, nslots, kc, hist, &kth);
    for (int64_t i = tid; i < nslots; i += blockDim.x) {
        const uint64_t s = get(i);
        if (s != kEmptySlot && s <= sel) {
            const int p = atomicAdd(&ntop, 1);
            if (p < 256) top[p] = s;
        }
    }
    __syncthreads();
    const int ncand = ntop < kc ? ntop : kc;
    prefetch_rows(rows, top, ncand, dim, res);
    int sort_n = 64;
    while (sort_n < kc) sort_n <<= 1;
    for (int i = ncand + tid; i < sort_n; i += blockDim.x) top[i] = kEmptySlot;
    __syncthreads();
    if (tid < 64) wave_bitonic_sort(top, sort_n);
    __syncthreads();
    float list_cut = full_cut == kEmptySlot ? kFltMax : slot_key(full_cut);
    // Rows above the query's bound were never admitted: their keys are >= it.
    if (qbound && qbound[q] != kEmptySlot) list_cut = fminf(list_cut, slot_key(qbound[q]));
    final_rescore_wide(qp, qn, rows, norms, n, dim, metric, q, top, ncand, kc, res,
                       reinterpret_cast<float*>(cand), fa, kProofFlat, kEmptySlot, list_cut);
    // A query with values outside the split range has no valid keys here,
    // and one whose candidate buffer filled up may miss rows: the streaming
    // scan runs it again.
    if (tid == 0 && qbad && qbad[q]) fa.status[q] = 1;
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
        return e ? std::max<int64_t>(8, std::atoll(e)) : (int64_t)512;
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
    // Bounding launch of the split-bf16 contraction: up to 32 segments
    // spread over the rows, about a thirty-second of the rows in all.
    p.s_nseg = (int)std::min<int64_t>(nseg, 32);
    const int64_t srps = (n + p.s_nseg - 1) / p.s_nseg;
    p.s_rows_per_seg = (srps + kGemmRows - 1) / kGemmRows * kGemmRows;
    int64_t srows = (n / 32 / p.s_nseg + kGemmRows - 1) / kGemmRows * kGemmRows;
    srows = std::max<int64_t>(srows, kGemmRows);
    p.s_seg_rows = std::min(srows, p.s_rows_per_seg);
    *out = p;
    return true;
}

size_t gemm_lists_bytes(const GemmPlan& p, int64_t nq) {
    // The split-bf16 path (lps 4): the full launch's candidate buffers,
    // which also hold the sampled launch's lane lists (s_nseg <= nseg).
    const size_t per = p.lps == 4 ? (size_t)kBf2Cap : (size_t)p.lps * gemm_list_len(p.kc);
    return (size_t)nq * (size_t)p.nseg * per * sizeof(uint64_t);
}

// Unit roundoff for make_bounds that covers the split-bf16 dot error
// without the rows' remainder term: one accumulation chain of 2 d products
// (d / 2 k values, two products each, per half, then the halves added: at
// most d + 1 roundings per product), so
// g = 1.024 gamma_{d+1}(2^-23) + 1.01 2^-16 + 2^-22 (gamma_d(u_eff) = g).
static double bf2_unit_roundoff(int dim) {
    const double u23 = 1.0 / 8388608.0;
    const double gd = (dim + 1) * u23 / (1.0 - (dim + 1) * u23);
    const double g = 1.024 * gd + 1.01 / 65536.0 + 1.0 / 4194304.0;
    return g / ((double)dim * (1.0 + g));
}

struct Bf2Inputs {
    const uint16_t* hi_rows;
    const f4v* recs;
    int64_t n;
    const uint32_t* split_q;
    const float* queries;
    int64_t nq;
};

template <int DIM, int C>
static void launch_bf2_dim_c(const GemmPlan& p, bool sampled, const Bf2Inputs& in, int metric,
                             const Bf2Args& ga, hipStream_t s) {
    const BoundCoef bc = make_bounds(DIM, bf2_unit_roundoff(DIM));
    const dim3 grid((unsigned)(ga.nseg * p.nqb));
    const dim3 block(64 * kBf2Waves);
    const size_t shm = bf2_lds_bytes<DIM>();
    static bool attr = [] {
        const int a = (int)bf2_lds_bytes<DIM>();
        (void)hipFuncSetAttribute((const void*)flat_gemm_bf16x2<DIM, kMetricCosine, C, false>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, a);
        (void)hipFuncSetAttribute((const void*)flat_gemm_bf16x2<DIM, kMetricL2, C, false>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, a);
        (void)hipFuncSetAttribute((const void*)flat_gemm_bf16x2<DIM, kMetricIP, C, false>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, a);
        (void)hipFuncSetAttribute((const void*)flat_gemm_bf16x2<DIM, kMetricCosine, C, true>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, a);
        (void)hipFuncSetAttribute((const void*)flat_gemm_bf16x2<DIM, kMetricL2, C, true>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, a);
        (void)hipFuncSetAttribute((const void*)flat_gemm_bf16x2<DIM, kMetricIP, C, true>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, a);
        return true;
    }();
    (void)attr;
#define MANS_BF2_LAUNCH(M, B)                                                                      \
    hipLaunchKernelGGL((flat_gemm_bf16x2<DIM, M, C, B>), grid, block, shm, s, in.hi_rows, in.recs, \
                       in.n, in.split_q, in.queries, in.nq, bc, ga)
    if (sampled) {
        switch (metric) {
        case kMetricCosine: MANS_BF2_LAUNCH(kMetricCosine, false); break;
        case kMetricL2: MANS_BF2_LAUNCH(kMetricL2, false); break;
        default: MANS_BF2_LAUNCH(kMetricIP, false); break;
        }
    } else {
        switch (metric) {
        case kMetricCosine: MANS_BF2_LAUNCH(kMetricCosine, true); break;
        case kMetricL2: MANS_BF2_LAUNCH(kMetricL2, true); break;
        default: MANS_BF2_LAUNCH(kMetricIP, true); break;
        }
    }
#undef MANS_BF2_LAUNCH
}

hipError_t launch_flat_bf2(const GemmPlan& p, bool sampled, const uint16_t* hi_rows,
                           const float* recs, int64_t n, int dim, const uint32_t* split_q,
                           const float* queries, int64_t nq, int metric, const uint64_t* qbound,
                           uint64_t* lists, uint32_t* qflag, hipStream_t s) {
    // The sampled launch keeps kBf2ListLen-slot lane lists (its bound needs
    // only the k <= 32 best rows); the full one kBf2Cap-slot candidate
    // buffers (a half per k half), of which the merge keeps kGemmMaxKc.
    static_assert(kBf2Lists * kBf2ListLen <= kBf2Cap, "sampled lists fit the buffers");
    Bf2Args ga;
    ga.nseg = sampled ? p.s_nseg : p.nseg;
    ga.nqb = p.nqb;
    ga.rows_per_seg = sampled ? p.s_rows_per_seg : p.rows_per_seg;
    ga.seg_rows = sampled ? p.s_seg_rows : p.rows_per_seg;
    // Products and partial sums flushed below 2^-126 (fewer than 6 dim of
    // them per dot), counted twice for L2's -2 dot.
    ga.abs_slack = (float)(12.0 * dim * 1.1754943508222875e-38);
    ga.qbound = qbound;
    ga.lists = lists;
    ga.qflag = qflag;
    // The records of the metric: [n] for cosine, then [n] for L2 and inner
    // product.
    const f4v* r4 = reinterpret_cast<const f4v*>(recs) + (metric == kMetricCosine ? 0 : n);
    const Bf2Inputs in{hi_rows, r4, n, split_q, queries, nq};
    constexpr int C = kBf2ListLen;
    switch (dim) {
    case 64: launch_bf2_dim_c<64, C>(p, sampled, in, metric, ga, s); break;
    case 96: launch_bf2_dim_c<96, C>(p, sampled, in, metric, ga, s); break;
    case 128: launch_bf2_dim_c<128, C>(p, sampled, in, metric, ga, s); break;
    case 192: launch_bf2_dim_c<192, C>(p, sampled, in, metric, ga, s); break;
    case 256: launch_bf2_dim_c<256, C>(p, sampled, in, metric, ga, s); break;
    case 384: launch_bf2_dim_c<384, C>(p, sampled, in, metric, ga, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_bf2_bounds(const GemmPlan& p, int64_t nq, int k, const uint64_t* lists,
                             const float* rows, const float* norms, int dim, const float* queries,
                             int metric, uint64_t* bound, hipStream_t s) {
    const int64_t per_query = (int64_t)p.s_nseg * kBf2Lists * kBf2ListLen;
    const size_t shmem = per_query <= kKthLdsSlots ? sizeof(uint64_t) * (size_t)per_query : 0;
    const dim3 grid(1, (unsigned)nq);
#define MANS_BOUND_CASE(N)                                                                       \
    hipLaunchKernelGGL(lists_exact_bound<N>, grid, dim3(256), shmem, s, k, per_query, lists, rows, \
                       norms, dim, queries, metric, bound)
    switch (flat_nch_for_dim(dim)) {
    case 1: MANS_BOUND_CASE(1); break;
    case 2: MANS_BOUND_CASE(2); break;
    case 3: MANS_BOUND_CASE(3); break;
    case 4: MANS_BOUND_CASE(4); break;
    case 6: MANS_BOUND_CASE(6); break;
    default: return hipErrorInvalidValue;
    }
#undef MANS_BOUND_CASE
    return hipGetLastError();
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
                               const uint64_t* lists, const uint64_t* qbound,
                               const uint32_t* qbad, const FlatArgs& fa, hipStream_t s) {
    // The split-bf16 path (qbound set) leaves one candidate buffer per
    // segment; the fp32 contraction lps sorted lane lists per segment.
    const int nlists = qbound ? p.nseg : p.lps * p.nseg;
    const int list_len = qbound ? kBf2Cap : gemm_list_len(p.kc);
    const int64_t total = (int64_t)nlists * list_len;
    static_assert(kGemmMaxKc <= 64, "the merge's rescore stages one group of 64 rows");
    const size_t stage = sizeof(float) * 2 * 64 * kWideStride;
    const size_t slots = total <= kKthLdsSlots ? sizeof(uint64_t) * (size_t)total : 0;
    const size_t shmem = sizeof(uint64_t) * 512 + std::max(stage, slots);
    hipLaunchKernelGGL(flat_lists_merge<NCH>, dim3(1, (unsigned)nq), dim3(256), shmem, s, rows,
                       norms, n, dim, queries, metric, p.kc, p.cap, nlists, list_len, lists,
                       qbound, qbad, fa);
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
                                  const uint64_t* lists, const uint64_t* qbound,
                                  const uint32_t* qbad, const FlatBuffers& b, int k, int k_stride,
                                  hipStream_t s) {
    FlatArgs fa = {};
    fa.out_dist = b.out_dist;
    fa.out_ids = b.out_ids;
    fa.status = b.status;
    fa.k = k;
    fa.k_stride = k_stride;
    switch (flat_nch_for_dim(dim)) {
    case 1: launch_lists_merge<1>(p, rows, norms, n, dim, queries, nq, metric, lists, qbound, qbad, fa, s); break;
    case 2: launch_lists_merge<2>(p, rows, norms, n, dim, queries, nq, metric, lists, qbound, qbad, fa, s); break;
    case 3: launch_lists_merge<3>(p, rows, norms, n, dim, queries, nq, metric, lists, qbound, qbad, fa, s); break;
    case 4: launch_lists_merge<4>(p, rows, norms, n, dim, queries, nq, metric, lists, qbound, qbad, fa, s); break;
    case 6: launch_lists_merge<6>(p, rows, norms, n, dim, queries, nq, metric, lists, qbound, qbad, fa, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mans
