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
// Every value x in [2^-50, 2^50] (or 0) is split once into bf16 parts
// x = xh + xl + r: xh = bf16(x), xl = bf16(x - xh) (x - xh is exact in
// fp32), both rounded to nearest even, so |x - xh| <= 2^-8 |x| and
// |r| <= 2^-16 |x|.  The contraction sums qh vh, qh vl and ql vh with
// v_mfma_f32_32x32x16_bf16 into three fp32 accumulators (each product of
// two bf16 values is exact in fp32), combined as hh + (hl + lh).  The
// omitted terms ql vl + (qh + ql) rv + rq (vh + vl) + rq rv are at most
// 3.01 2^-16 |q_i v_i| per element, the accumulations add at most
// gamma_d (u = 2^-23) (1 + 2^-7 + 2^-7) sum |q_i v_i| and the two final
// additions 2^-22 of it, so
//   |f - q.v| <= g sum |q_i v_i|,  g = 1.024 gamma_d + 3.01 2^-16 + 2^-22,
// and the keys are the fp32 path's lower bounds computed with a unit
// roundoff u_eff for which gamma_d(u_eff) = g (>= every other error term
// those bounds cover).  Values outside the range (huge, tiny, inf, NaN)
// are flagged when split: a corpus with any such value keeps the fp32
// contraction, and a flagged query is re-run by the streaming scan.
//
// The split parts are stored per 8 elements as [8 hi | 8 lo] (32 bytes),
// so a row keeps its fp32 size and one 16-element MFMA step of a lane is
// two 16-byte reads.
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

// One thread per 8 elements of `count` rows of dim (multiple of 8) floats;
// bad[row] (per_row) or bad[0] gets 1 for a value outside the range.
__global__ void split_bf16_kernel(const float* __restrict__ src, int64_t count, int dim,
                                  uint32_t* __restrict__ dst, uint32_t* __restrict__ bad,
                                  int per_row) {
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
    if (!ok) atomicOr(bad + (per_row ? row : 0), 1u);
}

hipError_t launch_split_bf16(const float* src, int64_t count, int dim, uint32_t* dst,
                             uint32_t* bad, bool per_row, hipStream_t s) {
    const int64_t threads = count * (dim / 8);
    if (threads <= 0) return hipSuccess;
    hipLaunchKernelGGL(split_bf16_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                       src, count, dim, dst, bad, per_row ? 1 : 0);
    return hipGetLastError();
}

typedef __bf16 bf8v __attribute__((ext_vector_type(8)));

// Work split.  A block of 8 waves serves 128 queries over one segment of
// rows: wave w takes query group w & 3 (32 queries) and half w >> 2 of the
// k range, so a wave keeps only its half of the query's split parts in
// registers and two waves fit on a SIMD (one hides the other's latencies).
// Per 32-row tile the two halves' sums (hh + (hl + lh) over each half) are
// exchanged through LDS and added (the same IEEE sum in either wave), and
// each wave keys 8 of the 16 rows a lane holds, keeping its own lane lists
// (4 lists per query and segment: half x lane half).
//
// Tiles reach LDS by direct global-to-LDS loads (global_load_lds, 16 bytes
// per lane) into a ring of two tile slots: tile t + 1 loads while tile t is
// contracted, without holding registers.  A slot holds, per k half, 32 rows
// x CPR 16-byte chunks unpadded; chunk c of row r sits at c ^ (r & SWZ), so
// the 32 lanes of a half-wave reading one chunk of 32 rows hit distinct
// banks.
constexpr int kBf3Waves = 8;
constexpr int kBf3Slots = 2;
constexpr int kBf3Lists = 4;  // lane lists per query and segment

template <int DIM>
struct Bf3Shape {
    static constexpr int NS = DIM / 16;  // MFMA k-steps per row
    static constexpr int NH = NS / 2;    // k-steps per half
    static constexpr int CPR = 4 * NH;   // 16-byte chunks of a row per half
    static constexpr int LOWBIT = CPR & -CPR;
    static constexpr int SWZ = (LOWBIT < 16 ? LOWBIT : 16) - 1;
    static constexpr int HALF_CHUNKS = kGemmRows * CPR;
    static constexpr int TILE_CHUNKS = 2 * HALF_CHUNKS;
    static constexpr int TILE_BYTES = 16 * TILE_CHUNKS;
    static constexpr int WAVE_INSTS = (TILE_CHUNKS + 64 * kBf3Waves - 1) / (64 * kBf3Waves);
    static_assert(DIM % 32 == 0, "unsupported dimension");
};

template <int DIM>
size_t bf3_lds_bytes() {
    return kBf3Slots * (size_t)Bf3Shape<DIM>::TILE_BYTES +
           sizeof(float) * (2 * kBf3Waves * 64 * 8 + kBf3Slots * kGemmRows + 4 * kGemmRows);
}

struct Bf3Args {
    int nseg;
    int nqb;
    int64_t rows_per_seg;     // multiple of kGemmRows
    int64_t seg_rows;         // rows scanned from each segment's start
    float abs_slack;
    const uint64_t* qbound;   // per query (BOUNDED)
    uint64_t* lists;          // [nq][nseg][kBf3Lists][C]
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// grid: nseg * nqb blocks (1-D, XCD mapping as flat_gemm_f32); block 512.
// split_rows / split_q: the split parts of the rows and of the queries.
template <int DIM, int METRIC, int C, bool BOUNDED>
__global__ __launch_bounds__(512, 1) void flat_gemm_bf16x3(
    const uint32_t* __restrict__ split_rows, const float* __restrict__ norms, int64_t n,
    const uint32_t* __restrict__ split_q, const float* __restrict__ queries, int64_t nq,
    BoundCoef bc, Bf3Args ga) {
    using G = Bf3Shape<DIM>;
    constexpr int NH = G::NH, CPR = G::CPR, SWZ = G::SWZ;
    extern __shared__ uint64_t lds[];
    uint8_t* ring = reinterpret_cast<uint8_t*>(lds);                      // [slot][half][32][CPR][16]
    float* xch = reinterpret_cast<float*>(ring + kBf3Slots * G::TILE_BYTES);  // [2][wave][64][8]
    float* tvn = xch + 2 * kBf3Waves * 64 * 8;  // [slot][32] raw vn
    float* tva = tvn + kBf3Slots * kGemmRows;  // [2][32] vn (NaN past the segment)
    float* tvb = tva + 2 * kGemmRows;          // [2][32] sqrt(vn), or 1 / sqrt(vn) for cosine
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int qg = wave & 3, kp = wave >> 2;
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
        const uint32_t* p = split_q + qrow * DIM + 8 * (2 * (kp * NH + s) + h);
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
    // Cosine rows with qn vn below 1.03e-20 get the key -1 (the formula's
    // 1e-10 branch is near); vn below this threshold covers every such row.
    const float vn_tiny = (1.03e-20f / qn) * 1.0001f;
    const float eps_all = bc.eps_cos + ga.abs_slack;
    uint64_t lst[C];
#pragma unroll
    for (int i = 0; i < C; ++i) lst[i] = kEmptySlot;
    const uint64_t bound = !qvalid ? 0ull : (BOUNDED ? ga.qbound[qid] : kEmptySlot);
    float thr = !qvalid ? -__int_as_float(0x7F800000)
                        : (bound == kEmptySlot ? __int_as_float(0x7F800000) : slot_key(bound));

    const int64_t seg0 = (int64_t)seg * ga.rows_per_seg;
    const int64_t seg1 = seg0 + ga.seg_rows < n ? seg0 + ga.seg_rows : n;
    const int64_t ntiles = seg1 > seg0 ? (seg1 - seg0 + kGemmRows - 1) / kGemmRows : 0;

    // Loads tile t into slot t % 2 (both k halves), and its row norms.  Rows
    // past the segment's end load its last row.
    auto issue = [&](int64_t t) {
        if (t >= ntiles) return;
        uint8_t* base = ring + (int)(t % kBf3Slots) * G::TILE_BYTES;
#pragma unroll
        for (int u = 0; u < G::WAVE_INSTS; ++u) {
            const int inst = wave * G::WAVE_INSTS + u;
            const int p = inst * 64 + lane;
            if (G::TILE_CHUNKS % (64 * kBf3Waves) == 0 || p < G::TILE_CHUNKS) {
                const int half = p / G::HALF_CHUNKS, rem = p - half * G::HALF_CHUNKS;
                const int r = rem / CPR, qq = rem - r * CPR;
                const int c = qq ^ (r & SWZ);
                int64_t row = seg0 + t * kGemmRows + r;
                row = row < seg1 ? row : seg1 - 1;
                const uint8_t* src = reinterpret_cast<const uint8_t*>(split_rows + row * DIM) +
                                     half * (16 * CPR) + 16 * c;
                __builtin_amdgcn_global_load_lds(src, (lds_ptr_t)(base + inst * 1024), 16, 0, 0);
            }
        }
        if (wave == 0 && lane < kGemmRows) {
            int64_t row = seg0 + t * kGemmRows + lane;
            row = row < seg1 ? row : seg1 - 1;
            __builtin_amdgcn_global_load_lds(norms + row,
                                             (lds_ptr_t)(tvn + (int)(t % kBf3Slots) * kGemmRows),
                                             4, 0, 0);
        }
    };

    // Tile t's sums: the partner half's 8 (rows it keys) go to LDS buffer
    // t & 1, this wave's 8 stay in `keep`.  After the next barrier the
    // partner's 8 for this wave are read back, added (the same IEEE sum in
    // either wave) and keyed: rows 8 (v / 4) + 4 h + v % 4 for
    // v = 8 KP .. 8 KP + 7, branch-free, then the insertion path only for a
    // lane with a key at or below its threshold.
    auto send = [&](const f16v& part, int64_t t, float (&keep)[8], auto kpc) {
        constexpr int KP = decltype(kpc)::value;
        constexpr int other = 8 * (1 - KP), my0 = 8 * KP;
        float* mine = xch + (((int)(t & 1) * kBf3Waves + wave) * 64 + lane) * 8;
        *reinterpret_cast<f4v*>(mine) = f4v{part[other], part[other + 1], part[other + 2], part[other + 3]};
        *reinterpret_cast<f4v*>(mine + 4) =
            f4v{part[other + 4], part[other + 5], part[other + 6], part[other + 7]};
#pragma unroll
        for (int i = 0; i < 8; ++i) keep[i] = part[my0 + i];
    };
    auto receive_and_offer = [&](const float (&keep)[8], int64_t t, auto kpc) {
        constexpr int KP = decltype(kpc)::value;
        constexpr int my0 = 8 * KP;
        const float* theirs = xch + (((int)(t & 1) * kBf3Waves + ((wave + 4) & 7)) * 64 + lane) * 8;
        const f4v r0 = *reinterpret_cast<const f4v*>(theirs);
        const f4v r1 = *reinterpret_cast<const f4v*>(theirs + 4);
        float f[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[i] = keep[i] + r0[i];
            f[4 + i] = keep[4 + i] + r1[i];
        }
        const int tb = (int)(t & 1) * kGemmRows;
        float key[8];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const int m0 = 8 * ((my0 >> 2) + g) + 4 * h;
            const f4v vna = *reinterpret_cast<const f4v*>(tva + tb + m0);
            const f4v wva = *reinterpret_cast<const f4v*>(tvb + tb + m0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float fv = f[4 * g + j], vn = vna[j], wv = wva[j];
                float k;
                if (METRIC == kMetricIP) {
                    k = (-fv - (sq * wv) * bc.c_ip) - ga.abs_slack;
                } else if (METRIC == kMetricL2) {
                    float dd = qn - 2.0f * fv + vn;
                    dd = dd > 0.0f ? dd : 0.0f;
                    k = (dd - (qn + vn + 2.0f * (sq * wv)) * bc.c_l2) - ga.abs_slack;
                } else {
                    // A zero row has wv = 0 and key 1 - eps (both paths give
                    // exactly 1); past the segment vn and wv are NaN.
                    k = (1.0f - fv * (rq * wv)) - eps_all;
                    k = vn < vn_tiny ? -1.0f : k;
                }
                key[4 * g + j] = k;
            }
        }
        float mn = key[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) mn = fminf(mn, key[i]);
        if (mn <= thr) {
            const int64_t base = seg0 + t * kGemmRows;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (key[i] <= thr) {
                    const int v = my0 + i;
                    const int m = 8 * (v >> 2) + 4 * h + (v & 3);
                    const uint64_t slot = pack_slot(key[i], (uint32_t)(base + m));
                    if (slot <= bound) {
                        list_insert<C>(lst, slot);
                        const uint64_t top = lst[C - 1] < bound ? lst[C - 1] : bound;
                        thr = top == kEmptySlot ? thr : slot_key(top);
                    }
                }
            }
        }
    };

    issue(0);
    float keep[8] = {};
    for (int64_t t = 0; t < ntiles; ++t) {
        // Tile t is in LDS once this wave's loads are done; the barrier
        // publishes every wave's part (and the previous tile's sums and
        // norms) and frees the other slot (tile t - 1).
        wait_vmcnt<0>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue(t + 1);
        if (wave == 0 && lane < kGemmRows) {
            const int64_t row = seg0 + t * kGemmRows + lane;
            const float vn = tvn[(int)(t % kBf3Slots) * kGemmRows + lane];
            const bool in = row < seg1;
            const float nan = __int_as_float(0x7FC00000);
            const int at = (int)(t & 1) * kGemmRows + lane;
            tva[at] = in ? vn : nan;
            tvb[at] = !in ? nan
                          : (METRIC == kMetricCosine ? (vn > 0.0f ? 1.0f / sqrtf(vn) : 0.0f)
                                                     : sqrtf(vn));
        }
        const uint8_t* xl = ring + (int)(t % kBf3Slots) * G::TILE_BYTES +
                            kp * (16 * G::HALF_CHUNKS) + col * CPR * 16;
        const int sw = col & SWZ;
        f16v hh = {}, hl = {}, lh = {};
#pragma unroll
        for (int s = 0; s < NH; ++s) {
            const int c = 4 * s + 2 * h;
            const bf8v ah = __builtin_bit_cast(bf8v, *reinterpret_cast<const i4v*>(xl + 16 * (c ^ sw)));
            const bf8v al = __builtin_bit_cast(bf8v, *reinterpret_cast<const i4v*>(xl + 16 * ((c + 1) ^ sw)));
            hh = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, qh[s], hh, 0, 0, 0);
            hl = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, ql[s], hl, 0, 0, 0);
            lh = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, qh[s], lh, 0, 0, 0);
        }
        const f16v part = hh + (hl + lh);
        // The k half as a constant (kp is uniform over the wave, so these
        // are scalar branches): the previous tile's keys (its partner sums
        // were published by this tile's barrier), then this tile's send.
        if (kp == 0) {
            if (t > 0) receive_and_offer(keep, t - 1, std::integral_constant<int, 0>());
            send(part, t, keep, std::integral_constant<int, 0>());
        } else {
            if (t > 0) receive_and_offer(keep, t - 1, std::integral_constant<int, 1>());
            send(part, t, keep, std::integral_constant<int, 1>());
        }
    }
    if (ntiles > 0) {
        __syncthreads();  // the last tile's partner sums and norms
        if (kp == 0) receive_and_offer(keep, ntiles - 1, std::integral_constant<int, 0>());
        else receive_and_offer(keep, ntiles - 1, std::integral_constant<int, 1>());
    }
    if (qvalid) {
        uint64_t* out = ga.lists + (((size_t)qid * ga.nseg + seg) * kBf3Lists + 2 * kp + h) * C;
#pragma unroll
        for (int i = 0; i < C; ++i) out[i] = lst[i];
    }
}

// grid (1, nq): bound[q] = the kc-th smallest slot of the query's sampled
// lists (kEmptySlot when they hold fewer than kc).
__global__ __launch_bounds__(256) void lists_kth_slot(int kc, int64_t per_query,
                                                      const uint64_t* __restrict__ lists,
                                                      uint64_t* __restrict__ bound) {
    extern __shared__ uint64_t lds[];
    const uint32_t q = blockIdx.y;
    const uint64_t kth = block_kth_slot(lists + (size_t)q * per_query, per_query, kc, lds);
    if (threadIdx.x == 0) bound[q] = kth;
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
    if (in_lds)
        for (int64_t i = tid; i < total; i += blockDim.x) cand[i] = lq[i];
    __shared__ uint32_t hist[256];
    __shared__ int ntop;
    if (tid == 0) ntop = 0;
    __syncthreads();
    // The kc smallest slots (empty slots are the largest values and are
    // never taken).
    auto get = [&](int64_t i) { return in_lds ? cand[i] : lq[i]; };
    uint64_t kth;
    const uint64_t sel = block_radix_cut(get, total, kc, hist, &kth);
    for (int64_t i = tid; i < total; i += blockDim.x) {
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
    // A query with values outside the split range has no valid keys here:
    // the streaming scan runs it again.
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
    // Bounding launch of the split-bf16 contraction: up to 64 segments
    // spread over the rows, about a thirty-second of the rows in all.
    p.s_nseg = (int)std::min<int64_t>(nseg, 64);
    const int64_t srps = (n + p.s_nseg - 1) / p.s_nseg;
    p.s_rows_per_seg = (srps + kGemmRows - 1) / kGemmRows * kGemmRows;
    int64_t srows = (n / 32 / p.s_nseg + kGemmRows - 1) / kGemmRows * kGemmRows;
    srows = std::max<int64_t>(srows, kGemmRows);
    p.s_seg_rows = std::min(srows, p.s_rows_per_seg);
    *out = p;
    return true;
}

size_t gemm_lists_bytes(const GemmPlan& p, int64_t nq) {
    return (size_t)nq * (size_t)p.nseg * p.lps * gemm_list_len(p.kc) * sizeof(uint64_t);
}

// Unit roundoff for make_bounds that covers the split-bf16 dot error
// g = 1.024 gamma_d(2^-23) + 3.01 2^-16 + 2^-21 (gamma_d(u_eff) = g).
static double bf3_unit_roundoff(int dim) {
    const double u23 = 1.0 / 8388608.0;
    const double gd = dim * u23 / (1.0 - dim * u23);
    const double g = 1.024 * gd + 3.01 / 65536.0 + 1.0 / 2097152.0;
    return g / ((double)dim * (1.0 + g));
}

template <int DIM, int C, bool BOUNDED>
static void launch_bf3_dim_c(const GemmPlan& p, const uint32_t* split_rows, const float* norms,
                             int64_t n, const uint32_t* split_q, const float* queries, int64_t nq,
                             int metric, const Bf3Args& ga, hipStream_t s) {
    const BoundCoef bc = make_bounds(DIM, bf3_unit_roundoff(DIM));
    const dim3 grid((unsigned)(ga.nseg * p.nqb));
    const size_t shmem = bf3_lds_bytes<DIM>();
    static bool attr = [] {
        (void)hipFuncSetAttribute((const void*)flat_gemm_bf16x3<DIM, kMetricCosine, C, BOUNDED>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)bf3_lds_bytes<DIM>());
        (void)hipFuncSetAttribute((const void*)flat_gemm_bf16x3<DIM, kMetricL2, C, BOUNDED>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)bf3_lds_bytes<DIM>());
        (void)hipFuncSetAttribute((const void*)flat_gemm_bf16x3<DIM, kMetricIP, C, BOUNDED>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)bf3_lds_bytes<DIM>());
        return true;
    }();
    (void)attr;
    const dim3 block(64 * kBf3Waves);
    switch (metric) {
    case kMetricCosine:
        hipLaunchKernelGGL((flat_gemm_bf16x3<DIM, kMetricCosine, C, BOUNDED>), grid, block, shmem,
                           s, split_rows, norms, n, split_q, queries, nq, bc, ga);
        break;
    case kMetricL2:
        hipLaunchKernelGGL((flat_gemm_bf16x3<DIM, kMetricL2, C, BOUNDED>), grid, block, shmem, s,
                           split_rows, norms, n, split_q, queries, nq, bc, ga);
        break;
    default:
        hipLaunchKernelGGL((flat_gemm_bf16x3<DIM, kMetricIP, C, BOUNDED>), grid, block, shmem, s,
                           split_rows, norms, n, split_q, queries, nq, bc, ga);
        break;
    }
}

template <int DIM>
static void launch_bf3_dim(const GemmPlan& p, bool bounded, const uint32_t* split_rows,
                           const float* norms, int64_t n, const uint32_t* split_q,
                           const float* queries, int64_t nq, int metric, const Bf3Args& ga,
                           hipStream_t s) {
    if (gemm_list_len(p.kc) == 4) {
        if (bounded) launch_bf3_dim_c<DIM, 4, true>(p, split_rows, norms, n, split_q, queries, nq, metric, ga, s);
        else launch_bf3_dim_c<DIM, 4, false>(p, split_rows, norms, n, split_q, queries, nq, metric, ga, s);
    } else {
        if (bounded) launch_bf3_dim_c<DIM, 8, true>(p, split_rows, norms, n, split_q, queries, nq, metric, ga, s);
        else launch_bf3_dim_c<DIM, 8, false>(p, split_rows, norms, n, split_q, queries, nq, metric, ga, s);
    }
}

hipError_t launch_flat_bf3(const GemmPlan& p, bool sampled, const uint32_t* split_rows,
                           const float* norms, int64_t n, int dim, const uint32_t* split_q,
                           const float* queries, int64_t nq, int metric, const uint64_t* qbound,
                           uint64_t* lists, hipStream_t s) {
    Bf3Args ga;
    ga.nseg = sampled ? p.s_nseg : p.nseg;
    ga.nqb = p.nqb;
    ga.rows_per_seg = sampled ? p.s_rows_per_seg : p.rows_per_seg;
    ga.seg_rows = sampled ? p.s_seg_rows : p.rows_per_seg;
    // Products and partial sums of three chains flushed below 2^-126,
    // counted twice for L2's -2 dot.
    ga.abs_slack = (float)(12.0 * dim * 1.1754943508222875e-38);
    ga.qbound = qbound;
    ga.lists = lists;
    const bool bounded = !sampled;
    switch (dim) {
    case 64: launch_bf3_dim<64>(p, bounded, split_rows, norms, n, split_q, queries, nq, metric, ga, s); break;
    case 96: launch_bf3_dim<96>(p, bounded, split_rows, norms, n, split_q, queries, nq, metric, ga, s); break;
    case 128: launch_bf3_dim<128>(p, bounded, split_rows, norms, n, split_q, queries, nq, metric, ga, s); break;
    case 192: launch_bf3_dim<192>(p, bounded, split_rows, norms, n, split_q, queries, nq, metric, ga, s); break;
    case 256: launch_bf3_dim<256>(p, bounded, split_rows, norms, n, split_q, queries, nq, metric, ga, s); break;
    case 384: launch_bf3_dim<384>(p, bounded, split_rows, norms, n, split_q, queries, nq, metric, ga, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_bf3_bounds(const GemmPlan& p, int64_t nq, const uint64_t* lists, uint64_t* bound,
                             hipStream_t s) {
    const int64_t per_query = (int64_t)p.s_nseg * kBf3Lists * gemm_list_len(p.kc);
    hipLaunchKernelGGL(lists_kth_slot, dim3(1, (unsigned)nq), dim3(256),
                       per_query <= kKthLdsSlots ? sizeof(uint64_t) * (size_t)per_query : 0, s, p.kc,
                       per_query, lists, bound);
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
    const int64_t total = (int64_t)p.lps * p.nseg * gemm_list_len(p.kc);
    static_assert(kGemmMaxKc <= 64, "the merge's rescore stages one group of 64 rows");
    const size_t stage = sizeof(float) * 2 * 64 * kWideStride;
    const size_t slots = total <= kKthLdsSlots ? sizeof(uint64_t) * (size_t)total : 0;
    const size_t shmem = sizeof(uint64_t) * 512 + std::max(stage, slots);
    hipLaunchKernelGGL(flat_lists_merge<NCH>, dim3(1, (unsigned)nq), dim3(256), shmem, s, rows,
                       norms, n, dim, queries, metric, p.kc, p.cap, p.lps * p.nseg,
                       gemm_list_len(p.kc), lists, qbound, qbad, fa);
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
