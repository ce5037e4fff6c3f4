// int8 prefilter + exact fp32 rerank on gfx950: BoundedExactScan.search
// (BoundedExactScan.swift:30-122) over the codes of Int8CodeBuffer.fill
// (Int8CodeCache.swift:64-99).
//
//  1. int8_build_codes: one wave per row, bit-exact with Int8CodeBuffer.fill
//     (the row max is order-free, the codes elementwise, the absolute sum an
//     exact integer sum; normSq is the row norm, computed once in the dots.c
//     order).  Rows are stored with a stride rounded up to 16 bytes (zero
//     padding adds nothing to an integer dot).
//  2. int8_query_prep: the query quantisation of BoundedExactScan.swift:52-94
//     in double precision, the sequential query norm and the key coefficients.
//  3. int8_scan: 8 lanes per row, 128-bit code loads, v_dot4_i32_i8, the
//     reference's lower-bound key formulas evaluated in the same operation
//     order and precision (float, double for L2), a per-wave WaveTopK of the
//     `budget` smallest keys, the cross-block merge of the flat scan, and the
//     final block's exact rescore in the dots.c order, sorted by (distance,
//     id), with the reference's margin proof (or none, for a fixed budget).
//  4. The host grows the budget 4x for queries whose proof fails
//     (BoundedExactScan.swift:115-118).  Past the largest on-device budget a
//     proof-checked search returns the exact flat scan's result, which is
//     what a proven reference round returns.
#include <algorithm>
#include <map>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "mans_hip.h"
#include "mans_runtime.hpp"
#include "mans_scan.hpp"

namespace mans {

constexpr int kInt8MaxBudget = 1024;       // largest kc the on-device selection keeps
constexpr int64_t kInt8MinRows = 16384;    // BoundedExactScan.minVectorCount
constexpr int kInt8MaxDim = 512;           // float4 rescore chunks: NCH <= 8

struct Int8QueryCoef {
    float qs;      // Float(queryScale): qsDot == qsW
    float qsqh;    // qsF * qabsHalfF
    float cfd;     // cosFDot == cosFW
    float cfh;     // cosFH
    float qn;      // sequential query norm
    float pad;
    double qn_d;   // Double(queryNormSq)
};

static inline int int8_stride(int64_t dim) { return (int)((dim + 15) / 16 * 16); }

// One wave per row (Int8CodeCache.swift:71-98).
__global__ __launch_bounds__(256) void int8_build_codes(
    const float* __restrict__ rows, const float* __restrict__ norms, int64_t first, int64_t count,
    int dim, int stride, int8_t* __restrict__ codes, float* __restrict__ u, float* __restrict__ w,
    float* __restrict__ normsq, float* __restrict__ invsqrt) {
    const int lane = threadIdx.x & 63;
    const int64_t r = first + (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= first + count) return;  // the whole wave leaves together
    const float* row = rows + r * dim;
    float m = 0.0f;
    for (int d = lane; d < dim; d += 64) {
        const float a = fabsf(row[d]);
        m = a > m ? a : m;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float t = __shfl_xor(m, o);
        m = t > m ? t : m;
    }
    const float scale = m > 0.0f ? m / 127.0f : 1.0f;
    const float inverse = 1.0f / scale;
    int asum = 0;
    for (int d = lane; d < stride; d += 64) {
        int c = 0;
        if (d < dim) {
            const float scaled = row[d] * inverse;
            c = (int)(scaled >= 0.0f ? scaled + 0.5f : scaled - 0.5f);
            c = c > 127 ? 127 : (c < -127 ? -127 : c);
        }
        codes[r * stride + d] = (int8_t)c;
        asum += c < 0 ? -c : c;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) asum += __shfl_xor(asum, o);
    if (lane == 0) {
        const float ebase = ((float)asum / 2.0f + (float)dim / 4.0f) * (1.0f + 1e-6f) + 16.0f;
        const float ns = norms[r];
        u[r] = scale;
        w[r] = scale * ebase;
        normsq[r] = ns;
        invsqrt[r] = ns > 1e-20f ? 1.0f / sqrtf(ns) : 0.0f;
    }
}

// The query quantisation of BoundedExactScan.swift:52-94 by one block:
// its codes (stride bytes, zero past dim) to `codes`, its coefficients to
// *coef (written by thread 0: visible to the block after a barrier).  qsh:
// dim floats of LDS, 16-byte aligned (overwritten); dim % 4 == 0.
__device__ __forceinline__ void int8_prep_block(const float* __restrict__ qp, int dim, int stride,
                                                float* qsh, int8_t* codes, Int8QueryCoef* coef) {
    __shared__ uint32_t max_bits;
    __shared__ int abs_sum;
    const int tid = threadIdx.x;
    if (tid == 0) {
        max_bits = 0u;
        abs_sum = 0;
    }
    __syncthreads();
    float m = 0.0f;
    for (int d = tid; d < dim; d += blockDim.x) {
        const float v = qp[d];
        qsh[d] = v;
        const float a = fabsf(v);
        m = a > m ? a : m;
    }
    atomicMax(&max_bits, __float_as_uint(m));  // non-negative floats order as integers
    __syncthreads();
    const float max_abs = __uint_as_float(max_bits);
    const double qscale = max_abs > 0.0f ? (double)max_abs / 127.0 : 1.0;
    int a = 0;
    for (int d = tid; d < stride; d += blockDim.x) {
        int c = 0;
        if (d < dim) {
            const double scaled = (double)qsh[d] / qscale;
            c = (int)(scaled >= 0.0 ? scaled + 0.5 : scaled - 0.5);
            c = c > 127 ? 127 : (c < -127 ? -127 : c);
        }
        codes[d] = (int8_t)c;
        a += c < 0 ? -c : c;
    }
    atomicAdd(&abs_sum, a);
    __syncthreads();
    // The squares in parallel (each rounded, as in the sequential loop),
    // then thread 0's running sum over them in order.
    for (int d = tid; d < dim; d += blockDim.x) qsh[d] = qsh[d] * qsh[d];
    __syncthreads();
    if (tid == 0) {
        float qn = 0.0f;  // the sequential norm of FlatGPUSearch.swift:532-535
        const f4v* sq = reinterpret_cast<const f4v*>(qsh);
#pragma unroll 8
        for (int i = 0; i < (dim >> 2); ++i) {
            const f4v v = sq[i];
            qn = qn + v.x;
            qn = qn + v.y;
            qn = qn + v.z;
            qn = qn + v.w;
        }
        const float qs = (float)qscale;
        const float qabs_half = (float)abs_sum / 2.0f;
        const float inv = qn > 1e-20f ? 1.0f / sqrtf(qn) : 0.0f;
        Int8QueryCoef c;
        c.qs = qs;
        c.qsqh = qs * qabs_half;
        c.cfd = qs * inv;
        c.cfh = qs * qabs_half * inv;
        c.qn = qn;
        c.pad = 0.0f;
        c.qn_d = (double)qn;
        *coef = c;
    }
}

// One block per query.  dynamic LDS: dim floats.
__global__ __launch_bounds__(256) void int8_query_prep(const float* __restrict__ queries, int dim,
                                                       int stride, int8_t* __restrict__ qcodes,
                                                       Int8QueryCoef* __restrict__ coefs) {
    extern __shared__ float qsh[];
    const int64_t q = blockIdx.x;
    int8_prep_block(queries + q * dim, dim, stride, qsh, qcodes + q * stride, coefs + q);
}

// Lower-bound key of one row, BoundedExactScan.swift:178-228, in the
// reference's operation order and precision.
__device__ __forceinline__ float int8_key(int metric, const Int8QueryCoef& c, float dot, float u,
                                          float w, float vn, float invsqrt) {
    if (metric == kMetricIP) return -(c.qs * u * dot + c.qsqh * u + c.qs * w);
    if (metric == kMetricL2) {
        const float two_qs = 2.0f * c.qs, two_qsqh = 2.0f * c.qsqh;
        const double key = c.qn_d + (double)vn - (double)(two_qs * u * dot) -
                           (double)(two_qsqh * u) - (double)(two_qs * w);
        return (float)key;
    }
    const float inner = c.cfd * u * dot + c.cfh * u + c.cfd * w;
    return 1.0f - inner * invsqrt;
}

__device__ __forceinline__ int dot16_i8(const i4v& a, const i4v& b, int acc) {
    acc = __builtin_amdgcn_sdot4(a.x, b.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a.y, b.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, b.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, b.w, acc, false);
    return acc;
}

// Exact integer sum over the 8 lanes of a row group (lanes 8 g .. 8 g + 7).
__device__ __forceinline__ int sum8(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    v += __shfl_xor(v, 4);
    return v;
}

// Sampled bounds of the streaming scan.  A launch that scans the first
// scan_rows rows of each block's range writes each block's smallest slot
// to block_min_out ([query][block]) and stops; the kc-th smallest of a
// query's block minima is its bound (kc blocks hold a sampled row at or
// below it, so no row above it is among the kc smallest).  The full launch
// then admits no key above it (qbound).
struct I8ScanBounds {
    int64_t scan_rows = INT64_MAX;
    const uint64_t* qbound = nullptr;
    uint64_t* block_min_out = nullptr;
    // Sampled launch over every query: its last block per query writes the
    // bound_kc-th smallest block minimum to qbound_out.
    uint64_t* qbound_out = nullptr;
    int bound_kc = 0;
    // Non-null: the launch quantises the queries itself (dim <= kI8MaxDim)
    // and stores the codes and coefficients here.
    int8_t* prep_codes_out = nullptr;
    Int8QueryCoef* prep_coefs_out = nullptr;
};
constexpr int kI8MaxDim = 512;  // NCH <= 8: 16 lanes x 8 float4 chunks

struct Int8Planes {
    const int8_t* codes;
    const float* u;
    const float* w;
    const float* normsq;
    const float* invsqrt;
    int stride;
};

// The streaming pass of one block over rows [start, end): each 8-lane group
// takes kI8StreamRows rows per step (rows base + 8 kI8StreamRows wave + g8
// + 8 j), and
// the next step's codes are loaded while the current step's are reduced and
// keyed, so a wave has two steps of codes in flight.  Every lane calls
// offer(valid, key, row) once per step: lane l8 = j < kI8StreamRows keys
// row j.
constexpr int kI8StreamRows = 4;
template <int NC8, class Offer>
__device__ __forceinline__ void int8_stream(const Int8Planes& pl, const i4v (&qc)[NC8], int metric,
                                            const Int8QueryCoef& coef, int64_t start, int64_t end,
                                            Offer&& offer) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g8 = lane >> 3, l8 = lane & 7;
    const int nchunk = pl.stride >> 4;
    constexpr int64_t kStep = 4 * 8 * kI8StreamRows;  // rows per block step
    struct Step {
        i4v a[kI8StreamRows][NC8];
        float pu[kI8StreamRows], pw[kI8StreamRows], pn[kI8StreamRows];
    };
    auto load = [&](int64_t base, Step& st) {
#pragma unroll
        for (int j = 0; j < kI8StreamRows; ++j) {
            const int64_t r = base + wave * 8 * kI8StreamRows + g8 + 8 * j;
            // Plane values of clamped rows, so every load is unconditional.
            const int64_t cr = r < end ? r : start;
            st.pu[j] = pl.u[cr];
            st.pw[j] = pl.w[cr];
            st.pn[j] = metric == kMetricL2 ? pl.normsq[cr] : pl.invsqrt[cr];
            // Chunks past the row's end re-read its last chunk; the query's
            // codes there are zero, so they add nothing (and the load needs
            // no branch).
            const i4v* src = reinterpret_cast<const i4v*>(pl.codes + cr * pl.stride);
#pragma unroll
            for (int c = 0; c < NC8; ++c) {
                const int idx = l8 + 8 * c;
                st.a[j][c] = __builtin_nontemporal_load(src + (idx < nchunk ? idx : nchunk - 1));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // Every lane of a group ends with the group's dot of each row.
    auto consume = [&](int64_t base, const Step& st) {
        int sj = 0;
        float uj = 0.0f, wj = 0.0f, nj = 0.0f;
#pragma unroll
        for (int j = 0; j < kI8StreamRows; ++j) {
            int s = 0;
#pragma unroll
            for (int c = 0; c < NC8; ++c) s = dot16_i8(st.a[j][c], qc[c], s);
            s = sum8(s);
            const bool mine = l8 == j;
            sj = mine ? s : sj;
            uj = mine ? st.pu[j] : uj;
            wj = mine ? st.pw[j] : wj;
            nj = mine ? st.pn[j] : nj;
        }
        const int64_t rj = base + wave * 8 * kI8StreamRows + g8 + 8 * (l8 < kI8StreamRows ? l8 : 0);
        const bool vj = l8 < kI8StreamRows && rj < end;
        offer(vj, int8_key(metric, coef, (float)sj, uj, wj, nj, nj), (uint32_t)rj);
    };
    if (start >= end) return;
    Step sa, sb;
    load(start, sa);
    for (int64_t base = start; base < end; base += 2 * kStep) {
        load(base + kStep, sb);
        consume(base, sa);
        load(base + 2 * kStep, sa);
        consume(base + kStep, sb);
    }
}

// The query's codes as the B side of dot16_i8: lane l8 holds 16-byte chunks
// l8 + 8 c (zero past the row's end).
template <int NC8>
__device__ __forceinline__ void int8_query_chunks(const int8_t* qcodes, uint32_t q, int stride,
                                                  i4v (&qc)[NC8]) {
    const int l8 = threadIdx.x & 7, nchunk = stride >> 4;
#pragma unroll
    for (int c = 0; c < NC8; ++c) {
        const int idx = l8 + 8 * c;
        qc[c] = idx < nchunk ? *reinterpret_cast<const i4v*>(qcodes + (int64_t)q * stride + 16 * idx)
                             : i4v{0, 0, 0, 0};
    }
}

// grid (nblk, nq_launch); block 256; dynamic LDS: 4 * cap slots (and, for a
// sampled launch, at least nblk slots).
// NCH: float4 chunks per lane for the rescore (16 lanes per row); the int8
// rows use (NCH + 1) / 2 16-byte chunks per lane with 8 lanes per row.
template <int NCH>
__global__ __launch_bounds__(256) void int8_scan(
    Int8Planes pl, const float* __restrict__ rows, const float* __restrict__ norms, int64_t n,
    int dim, const float* __restrict__ queries, const uint32_t* __restrict__ qidx,
    const int8_t* __restrict__ qcodes, const Int8QueryCoef* __restrict__ coefs, int metric, int kc,
    int cap, int64_t rows_per_block, int proof, FlatArgs fa, I8ScanBounds sb) {
    constexpr int NC8 = (NCH + 1) / 2;
    extern __shared__ uint64_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t q = qidx ? qidx[blockIdx.y] : blockIdx.y;
    Int8QueryCoef coef;
    i4v qc[NC8];
    if (sb.prep_codes_out) {
        // Sampled launch that also quantises the query (in every block;
        // block 0 stores the codes and coefficients for later launches).
        __shared__ __align__(16) float prep_q[kI8MaxDim];
        __shared__ __align__(16) int8_t prep_codes[kI8MaxDim];
        __shared__ Int8QueryCoef prep_coef;
        int8_prep_block(queries + (int64_t)q * dim, dim, pl.stride, prep_q, prep_codes, &prep_coef);
        __syncthreads();
        coef = prep_coef;
        int8_query_chunks<NC8>(prep_codes, 0, pl.stride, qc);
        if (blockIdx.x == 0) {
            for (int i = tid; i < pl.stride; i += blockDim.x)
                sb.prep_codes_out[(int64_t)q * pl.stride + i] = prep_codes[i];
            if (tid == 0) sb.prep_coefs_out[q] = prep_coef;
        }
    } else {
        coef = coefs[q];
        int8_query_chunks<NC8>(qcodes, q, pl.stride, qc);
    }

    WaveTopK sel;
    sel.init(lds + wave * cap, cap, kc);
    // A query's bound: no row with a larger slot is among its kc smallest,
    // so keys above its key are never admitted (ties at it are, which only
    // adds rows the selection then orders by slot).
    if (sb.qbound && sb.qbound[q] != kEmptySlot) sel.thresh = slot_key(sb.qbound[q]);
    const int64_t start = (int64_t)blockIdx.x * rows_per_block;
    const int64_t span = sb.scan_rows < rows_per_block ? sb.scan_rows : rows_per_block;
    const int64_t end = start + span < n ? start + span : n;
    int8_stream<NC8>(pl, qc, metric, coef, start, end,
                     [&](bool v, float key, uint32_t r) { sel.offer(v, key, r); });
    sel.finish();
    if (sb.block_min_out) {
        // Sampled launch: the block's smallest slot (each wave's list is
        // sorted, so its first slot is the wave's smallest).
        __shared__ uint64_t wmin[4];
        if (lane == 0) wmin[wave] = sel.buf[0];
        __syncthreads();
        uint64_t* mins = sb.block_min_out + (int64_t)blockIdx.y * gridDim.x;
        if (tid == 0) {
            uint64_t m = wmin[0];
            for (int w = 1; w < (int)(blockDim.x >> 6); ++w) m = wmin[w] < m ? wmin[w] : m;
            store_shared_slot(&mins[blockIdx.x], m);
        }
        if (!sb.qbound_out) return;
        // The last block of the query: the bound_kc-th smallest block minimum
        // (minima of distinct rows, so at least bound_kc rows have slots at
        // or below it).
        uint32_t* arrive = fa.counters + (int64_t)blockIdx.y * (fa.ngroups + 1);
        if (!block_arrive_last(arrive, gridDim.x)) return;
        if (tid == 0) __hip_atomic_store(arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int i = tid; i < (int)gridDim.x; i += blockDim.x) lds[i] = load_shared_slot(&mins[i]);
        __syncthreads();
        __shared__ uint32_t hist[256];
        uint64_t kth;
        block_radix_cut([&](int64_t i) { return lds[i]; }, gridDim.x, sb.bound_kc, hist, &kth);
        if (tid == 0) sb.qbound_out[blockIdx.y] = kth;
        return;
    }
    if (!flat_block_epilogue(sel, lds, cap, kc, fa)) return;

    const int lr = lane & 15, dim4 = dim >> 2;
    const float* qp = queries + (int64_t)q * dim;
    f4v qv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = lr + 16 * c;
        qv[c] = idx < dim4 ? *reinterpret_cast<const f4v*>(qp + 4 * idx) : f4v{0.f, 0.f, 0.f, 0.f};
    }
    final_rescore_f4<NCH>(qv, rows, norms, n, dim, metric, q, lds, kc, fa, kFltMax, proof);
}

template <int NCH>
static void launch_int8_scan(const FlatPlan& p, const Int8Planes& pl, const float* rows,
                             const float* norms, int64_t n, int dim, const float* queries,
                             const uint32_t* qidx, int64_t nq, const int8_t* qcodes,
                             const Int8QueryCoef* coefs, int metric, int proof, const FlatArgs& fa,
                             const I8ScanBounds& sb, hipStream_t s) {
    size_t shmem = sizeof(uint64_t) * 4 * (size_t)p.cap;
    if (sb.block_min_out) shmem = std::max(shmem, sizeof(uint64_t) * (size_t)p.nblk);
    hipLaunchKernelGGL(int8_scan<NCH>, dim3(p.nblk, (unsigned)nq), dim3(256), shmem, s, pl, rows,
                       norms, n, dim, queries, qidx, qcodes, coefs, metric, p.kc, p.cap,
                       p.rows_per_block, proof, fa, sb);
}

// Threshold-collect scan (one query per grid row; qidx, nullable, maps grid
// rows to queries).  Every row whose slot is at or below the row's bound
// (from a sample of rows: at least bound_kc rows lie at or below it) is
// gathered by its block, which rescores it exactly (the dots.c order) and
// appends its slot and its exact (distance, id) slot to the row's buffers.
// The last block of the grid row then runs the budget rounds of
// BoundedExactScan.search (BoundedExactScan.swift:96-121) on what was
// gathered: with `total` rows gathered at or below the bound, the budget
// smallest slots of the whole corpus are among them whenever budget <=
// total, so each round selects them (radix select), takes the k smallest
// exact slots of the selection and checks the proof; a failed proof grows
// the budget 4x and selects again.  Status: bits 0-1 the outcome (0 done, 1
// the proof still fails and the next budget exceeds `total`: the host scans
// again at budget kc 4^rounds; kStatusReselect: no round could run), bits
// 2-7 the rounds run.  A block with more than kCollectLdsSlots such rows, or
// more than I8Collect::ccap of them in all, gives kStatusReselect and
// nothing else is written (the caller selects again with the lists).
// The budget rounds of BoundedExactScan.search (BoundedExactScan.swift:96-121)
// over `total` gathered rows, run by one block: get(i) is the i-th gathered
// key slot, gete(i, cut) its exact (distance, id) slot when its key slot is
// at or below cut (else kEmptySlot).  With total rows gathered at or below
// a bound, the budget smallest key slots of the corpus are among them
// whenever budget <= total, so each round selects them (radix select),
// takes the k smallest exact slots of the selection, sorts them and checks
// the proof; a failed proof grows the budget 4x.  Writes the outputs of
// query q and fa.status[y]: bits 0-1 the outcome (0 done, 1 the proof still
// fails and the next budget exceeds total, kStatusReselect: no round could
// run), bits 2-7 the rounds run.  top: 256 slots of LDS.
template <class Get, class GetE>
__device__ void i8_budget_rounds(Get&& get, GetE&& gete, int64_t total, int kc, int64_t n,
                                 int proof, uint32_t q, uint32_t y, uint64_t* top, uint32_t* hist,
                                 int* ntop, const FlatArgs& fa) {
    const int tid = threadIdx.x;
    int64_t budget = kc;
    for (int round = 1;; ++round) {
        if (budget > total && total < n) {
            // The gathered rows no longer hold the budget smallest slots.
            if (tid == 0) fa.status[y] = round == 1 ? kStatusReselect : (uint8_t)(1 | ((round - 1) << 2));
            return;
        }
        // The selection: the budget smallest slots (every gathered row when
        // they are all there is), and the largest of them.
        const int64_t nsel = budget < total ? budget : total;
        uint64_t kth;
        const uint64_t cut = block_radix_cut(get, total, (int)nsel, hist, &kth);
        if (cut == kEmptySlot) {
            uint64_t mx = 0;
            for (int64_t i = tid; i < total; i += blockDim.x) {
                const uint64_t s = get(i);
                mx = s > mx ? s : mx;
            }
            kth = block_reduce_u64<true>(mx);
        }
        // The k smallest exact slots of the selection, sorted.
        const int kout = (int64_t)fa.k < nsel ? fa.k : (int)nsel;
        uint64_t ekth;
        const uint64_t ecut =
            block_radix_cut([&](int64_t i) { return gete(i, cut); }, total, kout, hist, &ekth);
        if (tid == 0) *ntop = 0;
        __syncthreads();
        for (int64_t i = tid; i < total; i += blockDim.x) {
            const uint64_t e = gete(i, cut);
            if (e != kEmptySlot && e <= ecut) {
                const int p = atomicAdd(ntop, 1);
                if (p < 256) top[p] = e;  // kout <= k <= 256 distinct slots
            }
        }
        __syncthreads();
        const int nout = *ntop < kout ? *ntop : kout;
        int sort_n = 64;
        while (sort_n < nout) sort_n <<= 1;
        for (int i = nout + tid; i < sort_n; i += blockDim.x) top[i] = kEmptySlot;
        __syncthreads();
        if (tid < 64) wave_bitonic_sort(top, sort_n);
        __syncthreads();
        const float cutoff = slot_key(kth);
        const float tau = nout > 0 ? slot_key(top[nout - 1]) : 0.0f;
        const bool all_rows = nsel >= n;
        bool ok;
        if (proof == kProofNone) {
            ok = true;
        } else if (proof == kProofMargin) {
            // BoundedExactScan.swift:101-113
            double margin = fabs((double)tau) * 1e-6;
            margin = margin < 1e-7 ? 1e-7 : margin;
            ok = all_rows || nsel < fa.k || (double)cutoff >= (double)tau + margin;
        } else {
            ok = all_rows || (nout > 0 && cutoff >= tau);
        }
        if (ok) {
            for (int i = tid; i < fa.k_stride; i += blockDim.x) {
                float dv = kFltMax;
                uint32_t id = kEmptyId;
                if (i < nout) {
                    id = slot_id(top[i]);
                    dv = slot_key(top[i]);
                }
                fa.out_dist[(int64_t)q * fa.k_stride + i] = dv;
                fa.out_ids[(int64_t)q * fa.k_stride + i] = id;
            }
            if (tid == 0) fa.status[y] = (uint8_t)(round << 2);
            return;
        }
        budget = budget * 4 < n ? budget * 4 : n;
        __syncthreads();  // top[] and *ntop are rewritten by the next round
    }
}

struct I8Collect {
    const uint64_t* qbound;  // [nq]
    uint64_t* cbuf;          // [nq][ccap] slots (int8 keys)
    uint64_t* ebuf;          // [nq][ccap] exact (distance, id) slots
    int64_t ccap;
    // Non-null: the last block only records the gathered count here and
    // int8_collect_rounds runs the budget rounds.
    int32_t* totals = nullptr;  // [nq]
};
constexpr int kCollectLdsSlots = 4096;  // rows gathered per block; candidates selected in LDS
constexpr size_t kCollectShmem = sizeof(uint64_t) * (256 + kCollectLdsSlots);
constexpr int64_t kCollectMaxCap = 65536;  // gathered rows per query
constexpr int64_t kCollectMaxQueries = 64;  // queries per collect launch

// grid (nblk, nq_launch); block 256; dynamic LDS kCollectShmem.
template <int NCH>
__global__ __launch_bounds__(256) void int8_collect(
    Int8Planes pl, const float* __restrict__ rows, const float* __restrict__ norms, int64_t n,
    int dim, const float* __restrict__ queries, const uint32_t* __restrict__ qidx,
    const int8_t* __restrict__ qcodes, const Int8QueryCoef* __restrict__ coefs, int metric,
    int kc, int64_t rows_per_block, int proof, FlatArgs fa, I8Collect cl) {
    constexpr int NC8 = (NCH + 1) / 2;
    extern __shared__ uint64_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t y = blockIdx.y;
    const uint32_t q = qidx ? qidx[y] : y;
    const Int8QueryCoef coef = coefs[q];
    i4v qc[NC8];
    int8_query_chunks<NC8>(qcodes, q, pl.stride, qc);
    const uint64_t bound = cl.qbound[y];
    uint32_t* arrive = fa.counters + (int64_t)y * (fa.ngroups + 1);
    uint32_t* appended = arrive + 1;
    uint64_t* cbuf = cl.cbuf + (int64_t)y * cl.ccap;
    uint64_t* ebuf = cl.ebuf + (int64_t)y * cl.ccap;
    const int64_t start = (int64_t)blockIdx.x * rows_per_block;
    const int64_t end = start + rows_per_block < n ? start + rows_per_block : n;
    uint64_t* top = lds;         // 256 slots (the last block's selection)
    uint64_t* cand = lds + 256;  // kCollectLdsSlots slots
    __shared__ uint32_t blk_count, blk_base;
    if (tid == 0) blk_count = 0;
    __syncthreads();
    int8_stream<NC8>(pl, qc, metric, coef, start, end, [&](bool v, float key, uint32_t r) {
        const uint64_t s = pack_slot(key, r);
        const bool pass = v && s <= bound;
        const uint64_t m = __ballot(pass);
        if (m == 0) return;
        const int leader = __ffsll((unsigned long long)m) - 1;
        uint32_t base = 0;
        if (lane == leader) base = atomicAdd(&blk_count, (uint32_t)__popcll(m));
        base = (uint32_t)__shfl((int)base, leader);
        const uint32_t pos = base + (uint32_t)__popcll(m & lanemask_lt());
        if (pass && pos < (uint32_t)kCollectLdsSlots) cand[pos] = s;
    });
    __syncthreads();
    const uint32_t nb = blk_count;
    if (nb > (uint32_t)kCollectLdsSlots) {
        // Too many rows for the block buffer: push the query's count past
        // the capacity so that its last block reports kStatusReselect.
        if (tid == 0)
            __hip_atomic_fetch_add(appended, (uint32_t)cl.ccap + 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    } else if (nb > 0) {
        if (tid == 0)
            blk_base = __hip_atomic_fetch_add(appended, nb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // Exact rescore of the gathered rows: one row per 16-lane group
        // (lane lr holds float4 chunks lr + 16 c of the row and the query).
        const int lr = lane & 15, grp = wave * 4 + (lane >> 4), dim4 = dim >> 2;
        const float* qp = queries + (int64_t)q * dim;
        f4v qv[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int idx = lr + 16 * c;
            qv[c] = idx < dim4 ? *reinterpret_cast<const f4v*>(qp + 4 * idx) : f4v{0.f, 0.f, 0.f, 0.f};
        }
        __syncthreads();
        const int64_t gb = blk_base;
        for (uint32_t i0 = 0; i0 < nb; i0 += 16) {
            const uint32_t i = i0 + grp;
            const bool valid = i < nb;
            const uint64_t s = valid ? cand[i] : 0ull;
            const uint32_t id = valid ? slot_id(s) : 0u;
            f4v a[NCH];
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int idx = lr + 16 * c;
                a[c] = (valid && idx < dim4) ? *reinterpret_cast<const f4v*>(rows + (int64_t)id * dim + 4 * idx)
                                             : f4v{0.f, 0.f, 0.f, 0.f};
            }
            const float dot = chain_dot<NCH>(a, qv, dim4);
            if (valid && lr == 0 && gb + i < cl.ccap) {
                const float dist = host_distance(dot, coef.qn, metric == kMetricIP ? 0.0f : norms[id], metric);
                store_shared_slot(cbuf + gb + i, s);
                store_shared_slot(ebuf + gb + i, pack_slot(dist, id));
            }
        }
    }
    if (!block_arrive_last(arrive, gridDim.x)) return;
    __shared__ uint32_t s_total;
    if (tid == 0) {
        s_total = __hip_atomic_load(appended, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(appended, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    const int64_t total = s_total;
    if (total > cl.ccap) {
        if (tid == 0) {
            fa.status[y] = kStatusReselect;
            if (cl.totals) cl.totals[y] = -1;
        }
        return;
    }
    if (cl.totals) {  // a one-block launch runs the rounds from LDS
        if (tid == 0) cl.totals[y] = (int32_t)total;
        return;
    }
    __shared__ uint32_t hist[256];
    __shared__ int ntop;
    const bool in_lds = total <= kCollectLdsSlots;
    if (in_lds)
        for (int64_t i = tid; i < total; i += blockDim.x) cand[i] = load_shared_slot(cbuf + i);
    __syncthreads();
    auto get = [&](int64_t i) { return in_lds ? cand[i] : load_shared_slot(cbuf + i); };
    auto gete = [&](int64_t i, uint64_t cut) {
        return get(i) <= cut ? load_shared_slot(ebuf + i) : kEmptySlot;
    };
    i8_budget_rounds(get, gete, total, kc, n, proof, q, y, top, hist, &ntop, fa);
}

// The budget rounds of the collect scan (grid (1, nq_launch), block
// kI8RoundsThreads; dynamic LDS kI8RoundsLds): the row's gathered key
// slots and exact slots are staged in LDS, then i8_budget_rounds; rows that
// gathered more than kI8RoundsSlots run the rounds from global memory.
constexpr int kI8RoundsSlots = 8192;
constexpr int kI8RoundsThreads = 512;
constexpr size_t kI8RoundsLds = sizeof(uint64_t) * (256 + 2 * (size_t)kI8RoundsSlots);

__global__ __launch_bounds__(kI8RoundsThreads) void int8_collect_rounds(
    int64_t n, const uint32_t* __restrict__ qidx, int kc, int proof, FlatArgs fa, I8Collect cl) {
    extern __shared__ uint64_t lds[];
    uint64_t* top = lds;
    uint64_t* cand = lds + 256;
    uint64_t* ex = cand + kI8RoundsSlots;
    __shared__ uint32_t hist[256];
    __shared__ int ntop;
    const int tid = threadIdx.x;
    const uint32_t y = blockIdx.y;
    const uint32_t q = qidx ? qidx[y] : y;
    const int32_t t = cl.totals[y];
    if (t < 0) return;  // the collect launch already set the status
    const int64_t total = t;
    const uint64_t* cbuf = cl.cbuf + (int64_t)y * cl.ccap;
    const uint64_t* ebuf = cl.ebuf + (int64_t)y * cl.ccap;
    if (total > kI8RoundsSlots) {
        auto getg = [&](int64_t i) { return cbuf[i]; };
        auto geteg = [&](int64_t i, uint64_t cut) { return cbuf[i] <= cut ? ebuf[i] : kEmptySlot; };
        i8_budget_rounds(getg, geteg, total, kc, n, proof, q, y, top, hist, &ntop, fa);
        return;
    }
    for (int64_t i = tid; i < total; i += blockDim.x) {
        cand[i] = cbuf[i];
        ex[i] = ebuf[i];
    }
    __syncthreads();
    auto get = [&](int64_t i) { return cand[i]; };
    auto gete = [&](int64_t i, uint64_t cut) { return cand[i] <= cut ? ex[i] : kEmptySlot; };
    i8_budget_rounds(get, gete, total, kc, n, proof, q, y, top, hist, &ntop, fa);
}

template <int NCH>
static hipError_t launch_int8_collect(const FlatPlan& p, const Int8Planes& pl, const float* rows,
                                      const float* norms, int64_t n, int dim, const float* queries,
                                      const uint32_t* qidx, int64_t nq, const int8_t* qcodes,
                                      const Int8QueryCoef* coefs, int metric, int kc, int proof,
                                      const FlatArgs& fa, const I8Collect& cl, hipStream_t s) {
    hipLaunchKernelGGL(int8_collect<NCH>, dim3(p.nblk, (unsigned)nq), dim3(256), kCollectShmem, s,
                       pl, rows, norms, n, dim, queries, qidx, qcodes, coefs, metric, kc,
                       p.rows_per_block, proof, fa, cl);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Batched queries: the code x code contraction on i8 MFMA
// (v_mfma_i32_32x32x32_i8), with the reference keys and the selection fused
// into the epilogue, so the nq x n key matrix is never written.
//
// Block: 4 waves and 128 queries (32 per wave) over one segment of rows.
// Rows are the MFMA A operand, 64 per stage (two 32-row tiles) staged
// through LDS (double-buffered, rows padded to an odd number of 16-byte
// units so the 32 lanes of a half-wave hit distinct banks); queries are the
// B operand and stay in registers (16 code bytes per lane per 32-byte
// k-step).  A and B use the same byte layout, so the hardware pairs code
// i of a row with code i of the query; the integer sums are exact in any
// order, so the dots equal the reference's i8 dot bit for bit.  In the
// 32 x 32 result a lane holds one query (lane % 32) against 16 rows of a
// tile (row 8 (v / 4) + 4 h + v % 4 for accumulator v, h = lane / 32).
// Each lane keeps the C smallest (key, row) slots it has seen in registers;
// a key enters only when it beats the lane's largest slot, which after the
// first rows is rare.  A stage's keys are offered while the next stage's
// MFMAs run.
//
// A first launch over the first sixteenth of every segment gives each
// query a bound: the kc-th smallest slot of its sampled lists, above which
// no slot can be among the query's kc smallest over all rows (kc sampled
// rows are at or below it).  The full launch then lets a key in only when
// it is at most the bound and beats the lane's largest slot, which keeps
// insertions into the lane lists rare.
//
// int8_lists_merge then selects each query's kc smallest slots over its
// 2 nseg lists.  A row a full list turned away has a slot above that list's
// largest, so the selection equals the streaming scan's (the kc smallest
// slots of all rows) whenever the kc-th selected slot is <= the smallest
// largest slot of the full lists; otherwise the query is selected again by
// the streaming scan at the same kc.
constexpr int kI8Queries = 128;  // queries per block
constexpr int kI8Rows = 64;      // rows per stage
constexpr int kI8List = 8;       // slots per lane list
constexpr int kI8GemmMaxKc = 256;

struct I8GemmArgs {
    int nseg;                 // row segments (multiple of 8)
    int nqb;                  // query blocks
    int64_t rows_per_seg;     // multiple of kI8Rows
    int64_t seg_rows;         // rows scanned from each segment's start (<= rows_per_seg)
    const uint64_t* qbound;   // nullable, per query: no slot above it is ever needed
    uint64_t* lists;          // [nq][nseg][2][kI8List]
    // Collect mode of the bounded launch (ccap > 0): every slot at or below
    // the query's bound is appended to its lane's region instead of the
    // lane list; a region that overflows sets cflag[query].
    uint64_t* cbuf = nullptr;     // [nq][nseg][2][ccap]
    int32_t* ccount = nullptr;    // [nq][nseg][2]
    uint32_t* cflag = nullptr;    // [nq]
    int ccap = 0;
};

// KS 32-byte k-steps per row: the code stride is 32 KS or 32 KS - 16 (the
// last 16 bytes of each LDS row and of the query are then zero).
template <int KS>
struct I8Shape {
    static constexpr int KB = 32 * KS;        // k bytes per row in LDS
    static constexpr int RS = KB + 16;        // LDS row pitch: an odd number of 16-byte units
    static constexpr int STAGE = kI8Rows * RS;
    static constexpr int CHUNKS = kI8Rows * KB / 16;
    static constexpr int LOADS = (CHUNKS + 255) / 256;  // 16-byte chunks per thread per stage
};

template <int KS>
size_t i8gemm_lds_bytes() {
    return 2 * (size_t)I8Shape<KS>::STAGE + sizeof(float) * 3 * 3 * kI8Rows;
}

template <int C>
__device__ __forceinline__ void lane_list_insert(uint64_t (&l)[C], uint64_t s) {
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
// blocks of one segment share b % 8, which places them on one XCD, so the
// segment's codes are read from HBM once into that XCD's L2.
// BOUNDED: the full launch (per-query bounds); otherwise the sampled one.
template <int KS, int METRIC, bool BOUNDED, bool COLLECT = false>
__global__ __launch_bounds__(256) void int8_gemm(Int8Planes pl, int64_t n,
                                                 const int8_t* __restrict__ qcodes,
                                                 const Int8QueryCoef* __restrict__ coefs, int64_t nq,
                                                 I8GemmArgs ga) {
    using G = I8Shape<KS>;
    constexpr int C = kI8List;
    extern __shared__ uint64_t lds[];
    int8_t* xs = reinterpret_cast<int8_t*>(lds);               // [2][64][RS]
    float* cf = reinterpret_cast<float*>(xs + 2 * G::STAGE);   // [3][3][64]: u, w, normSq|invSqrt
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, col = lane & 31;
    const int stride = pl.stride;
    const int row_chunks = stride >> 4;  // 16-byte code chunks per row in memory

    const int b = blockIdx.x, grp = 8 * ga.nqb;
    const int seg = 8 * (b / grp) + (b % 8);
    const int qb = (b % grp) / 8;

    // Lanes past the batch compute with query 0; their keys are never offered.
    const int64_t qid = (int64_t)qb * kI8Queries + wave * 32 + col;
    const bool qvalid = qid < nq;
    i4v qreg[KS];
    {
        const int8_t* qp = qcodes + (qvalid ? qid : 0) * stride;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const int ch = 2 * s + h;
            qreg[s] = ch < row_chunks ? *reinterpret_cast<const i4v*>(qp + 16 * ch) : i4v{0, 0, 0, 0};
        }
    }
    const Int8QueryCoef coef = coefs[qvalid ? qid : 0];
    uint64_t lst[C];
#pragma unroll
    for (int i = 0; i < C; ++i) lst[i] = kEmptySlot;
    // Slots above `bound` never enter; keys above thr (the key of the
    // smaller of bound and the lane's largest slot) cannot pass.
    const uint64_t bound = !qvalid ? 0ull : (BOUNDED ? ga.qbound[qid] : kEmptySlot);
    constexpr bool collect = BOUNDED && COLLECT;
    uint64_t* cregion = collect ? ga.cbuf + (((size_t)(qvalid ? qid : 0) * ga.nseg + seg) * 2 + h) * ga.ccap
                                : nullptr;
    int ccnt = 0;
    float thr = !qvalid ? -__int_as_float(0x7F800000)
                        : (bound == kEmptySlot ? __int_as_float(0x7F800000) : slot_key(bound));

    const int64_t seg0 = (int64_t)seg * ga.rows_per_seg;
    const int64_t seg1 = seg0 + ga.seg_rows < n ? seg0 + ga.seg_rows : n;
    const int64_t nst = seg1 > seg0 ? (seg1 - seg0 + kI8Rows - 1) / kI8Rows : 0;

    // The LDS pad chunk of each row (a stride of 32 KS - 16) stays zero.
    if (row_chunks < 2 * KS) {
        for (int r = tid; r < 2 * kI8Rows; r += 256)
            *reinterpret_cast<i4v*>(xs + (r / kI8Rows) * G::STAGE + (r % kI8Rows) * G::RS +
                                    16 * (2 * KS - 1)) = i4v{0, 0, 0, 0};
    }

    // Rows past the segment's end load the segment's last row (their keys
    // are never offered), so the loads need no branch.
    i4v pre[G::LOADS];
    auto load_stage = [&](int64_t st) {
#pragma unroll
        for (int u = 0; u < G::LOADS; ++u) {
            const int e = tid + 256 * u;
            const int r = e / (2 * KS), c = e % (2 * KS);
            int64_t row = seg0 + st * kI8Rows + r;
            row = row < seg1 ? row : seg1 - 1;
            const int cc = c < row_chunks ? c : row_chunks - 1;
            // Plain loads: the eight query blocks of a segment share it in L2.
            pre[u] = *reinterpret_cast<const i4v*>(pl.codes + row * stride + 16 * cc);
        }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int u = 0; u < G::LOADS; ++u) {
            const int e = tid + 256 * u;
            const int r = e / (2 * KS), c = e % (2 * KS);
            if ((G::CHUNKS % 256 == 0 || e < G::CHUNKS) && c < row_chunks)
                *reinterpret_cast<i4v*>(xs + buf * G::STAGE + r * G::RS + 16 * c) = pre[u];
        }
    };
    // Rows past the segment's end get NaN coefficients: their keys are NaN
    // and never pass the threshold test.  cb: the stage's coefficient buffer.
    auto store_coef = [&](int64_t st, int cb) {
        if (tid < kI8Rows) {
            const int64_t row = seg0 + st * kI8Rows + tid;
            const bool in = row < seg1;
            const int64_t r = in ? row : seg1 - 1;
            const float nan = __int_as_float(0x7FC00000);
            float* c = cf + cb * 3 * kI8Rows;
            c[tid] = in ? pl.u[r] : nan;
            c[kI8Rows + tid] = in ? pl.w[r] : nan;
            c[2 * kI8Rows + tid] = in ? (METRIC == kMetricL2 ? pl.normsq[r] : pl.invsqrt[r]) : nan;
        }
    };
    // Offers stage st's 32 keys per lane (st < 0: nothing).  All keys are
    // computed first, branch-free; only a lane whose smallest key is at or
    // below thr takes the insertion path, where each slot is checked
    // exactly.
    auto offer = [&](const i16v& a0, const i16v& a1, int64_t st, int cb) {
        if (st < 0) return;
        const float* c = cf + cb * 3 * kI8Rows;
        float key[32];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int m0 = 32 * t + 8 * g + 4 * h;  // four consecutive rows
                const f4v cu = *reinterpret_cast<const f4v*>(c + m0);
                const f4v cw = *reinterpret_cast<const f4v*>(c + kI8Rows + m0);
                const f4v cn = *reinterpret_cast<const f4v*>(c + 2 * kI8Rows + m0);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int v = 4 * g + j;
                    const float dot = (float)(t == 0 ? a0[v] : a1[v]);
                    key[16 * t + v] = int8_key(METRIC, coef, dot, cu[j], cw[j], cn[j], cn[j]);
                }
            }
        }
        float mn = key[0];
#pragma unroll
        for (int i = 1; i < 32; ++i) mn = fminf(mn, key[i]);  // NaN keys drop out
        if (mn <= thr) {
            const int64_t base = seg0 + st * kI8Rows;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                if (key[i] <= thr) {
                    const int m = 32 * (i >> 4) + 8 * ((i & 15) >> 2) + 4 * h + (i & 3);
                    const uint64_t slot = pack_slot(key[i], (uint32_t)(base + m));
                    if (slot <= bound) {
                        if constexpr (collect) {
                            if (ccnt < ga.ccap) cregion[ccnt] = slot;
                            ++ccnt;
                        } else {
                            lane_list_insert<C>(lst, slot);
                            const uint64_t top = lst[C - 1] < bound ? lst[C - 1] : bound;
                            thr = top == kEmptySlot ? thr : slot_key(top);
                        }
                    }
                }
            }
        }
    };

    if (nst > 0) {
        load_stage(0);
        store_stage(0);
        store_coef(0, 0);
    }
    __syncthreads();
    int buf = 0;
    int cb = 0;  // st % 3
    i16v prev0 = {}, prev1 = {};
    for (int64_t st = 0; st < nst; ++st) {
        // Prefetch the next stage (past the last one, reload the last).
        load_stage(st + 1 < nst ? st + 1 : st);
        const int8_t* xa = xs + buf * G::STAGE + col * G::RS + 16 * h;
        const int8_t* xb = xa + 32 * G::RS;
        i16v acc0 = {}, acc1 = {};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const i4v a0 = *reinterpret_cast<const i4v*>(xa + 32 * s);
            const i4v a1 = *reinterpret_cast<const i4v*>(xb + 32 * s);
            acc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, qreg[s], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, qreg[s], acc1, 0, 0, 0);
        }
        const int cb_prev = cb == 0 ? 2 : cb - 1, cb_next = cb == 2 ? 0 : cb + 1;
        // The previous stage's keys, while this stage's MFMAs run.
        offer(prev0, prev1, st - 1, cb_prev);
        if (st + 1 < nst) {
            store_stage(buf ^ 1);  // last read before the previous barrier
            store_coef(st + 1, cb_next);
        }
        __syncthreads();
        buf ^= 1;
        cb = cb_next;
        prev0 = acc0;
        prev1 = acc1;
    }
    offer(prev0, prev1, nst - 1, cb == 0 ? 2 : cb - 1);
    if (collect && qvalid) {
        ga.ccount[((size_t)qid * ga.nseg + seg) * 2 + h] = ccnt < ga.ccap ? ccnt : ga.ccap;
        if (ccnt > ga.ccap) atomicOr(&ga.cflag[qid], 1u);
    } else if (qvalid) {
        uint64_t* out = ga.lists + (((size_t)qid * ga.nseg + seg) * 2 + h) * C;
#pragma unroll
        for (int i = 0; i < C; ++i) out[i] = lst[i];
    }
}

// grid (1, nq): one block per query selects the kc smallest slots over its
// 2 nseg lists, then the exact rescore in the dots.c order and the proof
// (or none) of the streaming int8 scan; the status is kStatusReselect when
// the lists cannot show the selection is the kc smallest.
constexpr int kMergeLdsSlots = 4096;  // list slots selected in LDS (else read from memory)

template <int NCH>
__global__ __launch_bounds__(256) void int8_lists_merge(
    const float* __restrict__ rows, const float* __restrict__ norms, int64_t n, int dim,
    const float* __restrict__ queries, const Int8QueryCoef* __restrict__ coefs, int metric, int kc,
    int nlists, const uint64_t* __restrict__ lists, int proof, FlatArgs fa) {
    extern __shared__ uint64_t lds[];
    const int tid = threadIdx.x;
    const uint32_t q = blockIdx.y;
    const uint64_t* lq = lists + (size_t)q * nlists * kI8List;
    const int64_t total = (int64_t)nlists * kI8List;
    uint64_t* top = lds;         // 256 slots
    uint64_t* res = lds + 256;   // 256 slots
    uint64_t* cand = lds + 512;  // the lists' slots, then the rescore stage
    uint64_t mine = kEmptySlot;
    for (int i = tid; i < nlists; i += blockDim.x) {
        const uint64_t last = lq[(size_t)i * kI8List + kI8List - 1];
        mine = last < mine ? last : mine;  // a full list's largest slot
    }
    const uint64_t cut = block_reduce_u64<false>(mine);
    const bool in_lds = total <= kMergeLdsSlots;
    if (in_lds)
        for (int64_t i = tid; i < total; i += blockDim.x) cand[i] = lq[i];
    __shared__ uint32_t hist[256];
    __shared__ int ntop;
    if (tid == 0) ntop = 0;
    __syncthreads();
    // The kc smallest slots (the empty slots of lists that are not full
    // are the largest values and are never taken).
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
    final_rescore_wide(queries + (int64_t)q * dim, coefs[q].qn, rows, norms, n, dim, metric, q, top,
                       ncand, kc, res, reinterpret_cast<float*>(cand), fa, proof, cut);
}

// Budget rounds over the slots the collect-mode contraction gathered
// (grid (1, nq_launch), block kI8MergeThreads; dynamic LDS:
// kI8CollectMergeLds bytes).
// The query's regions are gathered into LDS; with `total` slots gathered at
// or below the query's bound, the budget smallest slots of the corpus are
// among them whenever budget <= total (BoundedExactScan.swift:96-121), so
// each round selects them (radix select), rescores the rows it adds in the
// dots.c order (16 lanes per row), takes the k smallest exact slots and
// checks the proof.  Status as int8_collect: bits 0-1 the outcome (0 done,
// 1 the next budget exceeds `total`, kStatusReselect: no round could run),
// bits 2-7 the rounds run.
constexpr int kI8GatherSlots = 8192;
constexpr int kI8MergeThreads = 512;  // one block per CU (the LDS): eight waves hide the row loads
constexpr size_t kI8CollectMergeLds =
    sizeof(uint64_t) * (256 + (size_t)kI8GatherSlots) + 2 * sizeof(uint32_t) * (size_t)kI8GatherSlots;

template <int NCH>
__global__ __launch_bounds__(kI8MergeThreads) void int8_collect_merge(
    const float* __restrict__ rows, const float* __restrict__ norms, int64_t n, int dim,
    const float* __restrict__ queries, const Int8QueryCoef* __restrict__ coefs, int metric, int kc,
    int nreg, const uint64_t* __restrict__ cbuf, const int32_t* __restrict__ ccount,
    const uint32_t* __restrict__ cflag, int ccap, int proof, FlatArgs fa) {
    extern __shared__ uint64_t lds[];
    uint64_t* top = lds;         // 256 slots: the k best exact slots
    uint64_t* cand = lds + 256;  // kI8GatherSlots gathered key slots
    float* exd = reinterpret_cast<float*>(cand + kI8GatherSlots);  // exact distances
    uint32_t* fresh_pos = reinterpret_cast<uint32_t*>(exd + kI8GatherSlots);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, grp = wave * 4 + (lane >> 4), dim4 = dim >> 2;
    constexpr int kGroups = kI8MergeThreads / 16;  // rows rescored per step
    const uint32_t q = blockIdx.y;
    __shared__ int s_total, ntop;
    __shared__ uint32_t hist[256];
    if (cflag[q] != 0) {  // a region overflowed: select again with the lists
        if (tid == 0) fa.status[q] = kStatusReselect;
        return;
    }
    if (tid == 0) s_total = 0;
    __syncthreads();
    for (int r = tid; r < nreg; r += blockDim.x) {
        const int c = ccount[(size_t)q * nreg + r];
        if (c == 0) continue;
        const int base = atomicAdd(&s_total, c);
        const uint64_t* src = cbuf + ((size_t)q * nreg + r) * ccap;
        for (int i = 0; i < c; ++i)
            if (base + i < kI8GatherSlots) cand[base + i] = src[i];
    }
    __syncthreads();
    const int64_t total = s_total;
    if (total > kI8GatherSlots) {
        if (tid == 0) fa.status[q] = kStatusReselect;
        return;
    }
    __shared__ int s_nfresh;
    const float* qp = queries + (int64_t)q * dim;
    f4v qv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = lr + 16 * c;
        qv[c] = idx < dim4 ? *reinterpret_cast<const f4v*>(qp + 4 * idx) : f4v{0.f, 0.f, 0.f, 0.f};
    }
    const float qn = coefs[q].qn;
    auto get = [&](int64_t i) { return cand[i]; };
    uint64_t done_cut = 0;  // rows with slots at or below it are rescored (round > 1)
    int64_t budget = kc;
    for (int round = 1;; ++round) {
        if (budget > total && total < n) {
            if (tid == 0) fa.status[q] = round == 1 ? kStatusReselect : (uint8_t)(1 | ((round - 1) << 2));
            return;
        }
        const int64_t nsel = budget < total ? budget : total;
        uint64_t kth;
        const uint64_t cut = block_radix_cut(get, total, (int)nsel, hist, &kth);
        if (cut == kEmptySlot) {
            uint64_t mx = 0;
            for (int64_t i = tid; i < total; i += blockDim.x) mx = cand[i] > mx ? cand[i] : mx;
            kth = block_reduce_u64<true>(mx);
        }
        // The positions this round adds, compacted; then their rows are
        // rescored two per 16-lane group at a time (interleaved chains), the
        // group's next two rows in flight.
        if (tid == 0) s_nfresh = 0;
        __syncthreads();
        for (int64_t i0 = 0; i0 < total; i0 += blockDim.x) {
            const int64_t i = i0 + tid;
            const uint64_t sl = i < total ? cand[i] : kEmptySlot;
            const bool fresh = i < total && sl <= cut && (round == 1 || sl > done_cut);
            const uint64_t m = __ballot(fresh);
            if (m == 0) continue;
            int base = 0;
            if (lane == 0) base = atomicAdd(&s_nfresh, __popcll(m));
            base = __shfl(base, 0);
            if (fresh) fresh_pos[base + __popcll(m & lanemask_lt())] = (uint32_t)i;
        }
        __syncthreads();
        const int nfresh = s_nfresh;
        auto load_row = [&](int j, f4v (&a)[NCH]) {
            const bool v = j < nfresh;
            const uint32_t pos = v ? fresh_pos[j] : 0u;
            const uint32_t id = v ? slot_id(cand[pos]) : 0u;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int idx = lr + 16 * c;
                a[c] = (v && idx < dim4) ? *reinterpret_cast<const f4v*>(rows + (int64_t)id * dim + 4 * idx)
                                         : f4v{0.f, 0.f, 0.f, 0.f};
            }
        };
        // Rows j and j2 > j of this group (j2 may be past the last: its
        // zero row is dotted and not written).
        auto rescore2 = [&](int j, const f4v (&a)[NCH], int j2, const f4v (&b)[NCH]) {
            if (j >= nfresh) return;  // the whole group agrees
            float d0, d1;
            chain_dot2<NCH>(a, b, qv, dim4, d0, d1);
            if (lr == 0) {
                const uint32_t pos = fresh_pos[j];
                const uint32_t id = slot_id(cand[pos]);
                exd[pos] = host_distance(d0, qn, metric == kMetricIP ? 0.0f : norms[id], metric);
                if (j2 < nfresh) {
                    const uint32_t pos2 = fresh_pos[j2];
                    const uint32_t id2 = slot_id(cand[pos2]);
                    exd[pos2] = host_distance(d1, qn, metric == kMetricIP ? 0.0f : norms[id2], metric);
                }
            }
        };
        f4v ra[NCH], rb[NCH], rc[NCH], rd[NCH];
        load_row(grp, ra);
        load_row(kGroups + grp, rb);
        for (int j0 = 0; j0 < nfresh; j0 += 4 * kGroups) {
            load_row(j0 + 2 * kGroups + grp, rc);
            load_row(j0 + 3 * kGroups + grp, rd);
            rescore2(j0 + grp, ra, j0 + kGroups + grp, rb);
            load_row(j0 + 4 * kGroups + grp, ra);
            load_row(j0 + 5 * kGroups + grp, rb);
            rescore2(j0 + 2 * kGroups + grp, rc, j0 + 3 * kGroups + grp, rd);
        }
        done_cut = cut;
        __syncthreads();  // exd[] is written
        // The k smallest exact slots of the selection, sorted.
        const int kout = (int64_t)fa.k < nsel ? fa.k : (int)nsel;
        auto gete = [&](int64_t i) {
            return cand[i] <= cut ? pack_slot(exd[i], slot_id(cand[i])) : kEmptySlot;
        };
        uint64_t ekth;
        const uint64_t ecut = block_radix_cut(gete, total, kout, hist, &ekth);
        if (tid == 0) ntop = 0;
        __syncthreads();
        for (int64_t i = tid; i < total; i += blockDim.x) {
            if (cand[i] > cut) continue;
            const uint64_t e = pack_slot(exd[i], slot_id(cand[i]));
            if (e <= ecut) {
                const int p = atomicAdd(&ntop, 1);
                if (p < 256) top[p] = e;
            }
        }
        __syncthreads();
        const int nout = ntop < kout ? ntop : kout;
        int sort_n = 64;
        while (sort_n < nout) sort_n <<= 1;
        for (int i = nout + tid; i < sort_n; i += blockDim.x) top[i] = kEmptySlot;
        __syncthreads();
        if (tid < 64) wave_bitonic_sort(top, sort_n);
        __syncthreads();
        const float cutoff = slot_key(kth);
        const float tau = nout > 0 ? slot_key(top[nout - 1]) : 0.0f;
        const bool all_rows = nsel >= n;
        bool ok;
        if (proof == kProofNone) {
            ok = true;
        } else if (proof == kProofMargin) {
            // BoundedExactScan.swift:101-113
            double margin = fabs((double)tau) * 1e-6;
            margin = margin < 1e-7 ? 1e-7 : margin;
            ok = all_rows || nsel < fa.k || (double)cutoff >= (double)tau + margin;
        } else {
            ok = all_rows || (nout > 0 && cutoff >= tau);
        }
        if (ok) {
            for (int i = tid; i < fa.k_stride; i += blockDim.x) {
                float dv = kFltMax;
                uint32_t id = kEmptyId;
                if (i < nout) {
                    id = slot_id(top[i]);
                    dv = slot_key(top[i]);
                }
                fa.out_dist[(int64_t)q * fa.k_stride + i] = dv;
                fa.out_ids[(int64_t)q * fa.k_stride + i] = id;
            }
            if (tid == 0) fa.status[q] = (uint8_t)(round << 2);
            return;
        }
        budget = budget * 4 < n ? budget * 4 : n;
        __syncthreads();  // top[] and ntop are rewritten by the next round
    }
}

// grid (1, nq): each query's bound, the kc-th smallest slot of its lists
// from the sampled launch (kEmptySlot when they hold fewer than kc).
__global__ __launch_bounds__(256) void int8_lists_bound(int kc, int nlists,
                                                        const uint64_t* __restrict__ lists,
                                                        uint64_t* __restrict__ qbound) {
    extern __shared__ uint64_t lds[];
    const uint32_t q = blockIdx.y;
    const uint64_t kth = block_kth_slot(lists + (size_t)q * nlists * kI8List,
                                        (int64_t)nlists * kI8List, kc, lds);
    if (threadIdx.x == 0) qbound[q] = kth;
}

static bool i8gemm_ks(int stride, int* ks) {
    const int k = (stride + 31) / 32;
    switch (k) {
    case 2: case 3: case 4: case 6: case 8: case 12: *ks = k; return true;
    default: return false;
    }
}

struct I8GemmPlan {
    int ks = 0;
    int nseg = 0;
    int nqb = 0;
    int64_t rows_per_seg = 0;
    // The bounding launch: s_nseg segments of s_rows_per_seg rows, the
    // first s_seg_rows of each scanned (about a sixteenth of the rows).
    int s_nseg = 0;
    int64_t s_rows_per_seg = 0;
    int64_t s_seg_rows = 0;
};

static bool plan_i8gemm(int64_t n, int stride, int64_t nq, int64_t kc, I8GemmPlan* out) {
    static const int64_t min_batch = [] {
        const char* e = std::getenv("MANS_I8GEMM_MIN_BATCH");
        return e ? std::max<int64_t>(1, std::atoll(e)) : (int64_t)16;
    }();
    static const int64_t target = [] {
        const char* e = std::getenv("MANS_I8GEMM_BLOCKS");
        return e ? std::max<int64_t>(8, std::atoll(e)) : (int64_t)1024;
    }();
    I8GemmPlan p;
    if (!i8gemm_ks(stride, &p.ks) || kc > kI8GemmMaxKc || nq < min_batch) return false;
    p.nqb = (int)((nq + kI8Queries - 1) / kI8Queries);
    // About `target` blocks, a multiple of 8 segments of >= 1024 rows each.
    int64_t nseg = (target + p.nqb - 1) / p.nqb;
    nseg = (nseg + 7) / 8 * 8;
    int64_t max_seg = n / 1024 / 8 * 8;
    if (nseg > max_seg) nseg = max_seg;
    if (nseg < 8) nseg = 8;
    const int64_t rps = (n + nseg - 1) / nseg;
    p.rows_per_seg = (rps + kI8Rows - 1) / kI8Rows * kI8Rows;
    p.nseg = (int)nseg;
    // Fewer, longer sampled segments than the full launch: each lane list
    // then sees enough rows to settle, and the bound selects over fewer lists.
    p.s_nseg = (int)std::min<int64_t>(nseg, 64);
    const int64_t srps = (n + p.s_nseg - 1) / p.s_nseg;
    p.s_rows_per_seg = (srps + kI8Rows - 1) / kI8Rows * kI8Rows;
    int64_t srows = (n / 16 / p.s_nseg + kI8Rows - 1) / kI8Rows * kI8Rows;
    srows = std::max<int64_t>(srows, kI8Rows);
    p.s_seg_rows = std::min(srows, p.s_rows_per_seg);
    *out = p;
    return true;
}

template <int KS>
static void launch_i8gemm_ks(const I8GemmPlan& p, const Int8Planes& pl, int64_t n,
                             const int8_t* qcodes, const Int8QueryCoef* coefs, int64_t nq,
                             int metric, const I8GemmArgs& ga, hipStream_t s) {
    const dim3 grid((unsigned)(ga.nseg * p.nqb));
    const size_t shmem = i8gemm_lds_bytes<KS>();
    const bool b = ga.qbound != nullptr;
    const bool c = b && ga.ccap > 0;
    switch (metric) {
    case kMetricCosine:
        if (c) hipLaunchKernelGGL((int8_gemm<KS, kMetricCosine, true, true>), grid, dim3(256), shmem, s, pl, n, qcodes, coefs, nq, ga);
        else if (b) hipLaunchKernelGGL((int8_gemm<KS, kMetricCosine, true>), grid, dim3(256), shmem, s, pl, n, qcodes, coefs, nq, ga);
        else hipLaunchKernelGGL((int8_gemm<KS, kMetricCosine, false>), grid, dim3(256), shmem, s, pl, n, qcodes, coefs, nq, ga);
        break;
    case kMetricL2:
        if (c) hipLaunchKernelGGL((int8_gemm<KS, kMetricL2, true, true>), grid, dim3(256), shmem, s, pl, n, qcodes, coefs, nq, ga);
        else if (b) hipLaunchKernelGGL((int8_gemm<KS, kMetricL2, true>), grid, dim3(256), shmem, s, pl, n, qcodes, coefs, nq, ga);
        else hipLaunchKernelGGL((int8_gemm<KS, kMetricL2, false>), grid, dim3(256), shmem, s, pl, n, qcodes, coefs, nq, ga);
        break;
    default:
        if (c) hipLaunchKernelGGL((int8_gemm<KS, kMetricIP, true, true>), grid, dim3(256), shmem, s, pl, n, qcodes, coefs, nq, ga);
        else if (b) hipLaunchKernelGGL((int8_gemm<KS, kMetricIP, true>), grid, dim3(256), shmem, s, pl, n, qcodes, coefs, nq, ga);
        else hipLaunchKernelGGL((int8_gemm<KS, kMetricIP, false>), grid, dim3(256), shmem, s, pl, n, qcodes, coefs, nq, ga);
        break;
    }
}

static hipError_t launch_i8gemm(const I8GemmPlan& p, const Int8Planes& pl, int64_t n,
                                const int8_t* qcodes, const Int8QueryCoef* coefs, int64_t nq,
                                int metric, bool sampled, const uint64_t* qbound,
                                uint64_t* lists, hipStream_t s, uint64_t* cbuf = nullptr,
                                int32_t* ccount = nullptr, uint32_t* cflag = nullptr,
                                int ccap = 0) {
    I8GemmArgs ga;
    ga.cbuf = cbuf;
    ga.ccount = ccount;
    ga.cflag = cflag;
    ga.ccap = ccap;
    ga.nseg = sampled ? p.s_nseg : p.nseg;
    ga.nqb = p.nqb;
    ga.rows_per_seg = sampled ? p.s_rows_per_seg : p.rows_per_seg;
    ga.seg_rows = sampled ? p.s_seg_rows : p.rows_per_seg;
    ga.qbound = qbound;
    ga.lists = lists;
    switch (p.ks) {
    case 2: launch_i8gemm_ks<2>(p, pl, n, qcodes, coefs, nq, metric, ga, s); break;
    case 3: launch_i8gemm_ks<3>(p, pl, n, qcodes, coefs, nq, metric, ga, s); break;
    case 4: launch_i8gemm_ks<4>(p, pl, n, qcodes, coefs, nq, metric, ga, s); break;
    case 6: launch_i8gemm_ks<6>(p, pl, n, qcodes, coefs, nq, metric, ga, s); break;
    case 8: launch_i8gemm_ks<8>(p, pl, n, qcodes, coefs, nq, metric, ga, s); break;
    case 12: launch_i8gemm_ks<12>(p, pl, n, qcodes, coefs, nq, metric, ga, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

constexpr int kI8CollectCap = 128;       // slots per lane region of the collect launch
constexpr int kI8CollectBoundKc = 256;   // the collect launch's bound: this many sampled slots

template <int NCH>
static hipError_t launch_i8_collect_merge(const float* rows, const float* norms, int64_t n,
                                          int dim, const float* queries,
                                          const Int8QueryCoef* coefs, int64_t nq, int metric,
                                          int kc, int nreg, const uint64_t* cbuf,
                                          const int32_t* ccount, const uint32_t* cflag, int proof,
                                          const FlatArgs& fa, hipStream_t s) {
    const size_t shmem = kI8CollectMergeLds;
    static const bool attr = [shmem] {
        (void)hipFuncSetAttribute((const void*)int8_collect_merge<NCH>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem);
        return true;
    }();
    (void)attr;
    hipLaunchKernelGGL(int8_collect_merge<NCH>, dim3(1, (unsigned)nq), dim3(kI8MergeThreads), shmem, s, rows,
                       norms, n, dim, queries, coefs, metric, kc, nreg, cbuf, ccount, cflag,
                       kI8CollectCap, proof, fa);
    return hipGetLastError();
}

template <int NCH>
static void launch_i8_merge(const I8GemmPlan& p, const float* rows, const float* norms, int64_t n,
                            int dim, const float* queries, const Int8QueryCoef* coefs, int64_t nq,
                            int metric, int kc, const uint64_t* lists, int proof, const FlatArgs& fa,
                            hipStream_t s) {
    const int64_t total = (int64_t)2 * p.nseg * kI8List;
    const size_t m = (size_t)(kc + 63) / 64;
    const size_t stage = sizeof(float) * 2 * 64 * m * kWideStride;
    const size_t slots = total <= kMergeLdsSlots ? sizeof(uint64_t) * (size_t)total : 0;
    const size_t shmem = sizeof(uint64_t) * 512 + std::max(stage, slots);
    hipLaunchKernelGGL(int8_lists_merge<NCH>, dim3(1, (unsigned)nq), dim3(256), shmem, s, rows,
                       norms, n, dim, queries, coefs, metric, kc, 2 * p.nseg, lists, proof, fa);
}

// Copies `count` rows of `width` floats: dst[i] = src[idx[i]].
__global__ void gather_rows_kernel(const float* __restrict__ src, const uint32_t* __restrict__ idx,
                                   int64_t count, int width, float* __restrict__ dst) {
    const int64_t i = blockIdx.x;
    if (i >= count) return;
    const float* s = src + (int64_t)idx[i] * width;
    for (int j = threadIdx.x; j < width; j += blockDim.x) dst[i * width + j] = s[j];
}

// dst[idx[i]] = src[i] for rows of `width` 32-bit words.
__global__ void scatter_rows_kernel(const uint32_t* __restrict__ src, const uint32_t* __restrict__ idx,
                                    int64_t count, int width, uint32_t* __restrict__ dst) {
    const int64_t i = blockIdx.x;
    if (i >= count) return;
    uint32_t* d = dst + (int64_t)idx[i] * width;
    for (int j = threadIdx.x; j < width; j += blockDim.x) d[j] = src[i * width + j];
}

hipError_t int8_refresh_rows(mans_corpus* c, int64_t first_row, int64_t count, hipStream_t s) {
    if (count <= 0) return hipSuccess;
    const int stride = int8_stride(c->dim);
    const int64_t blocks = (count + 3) / 4;
    hipLaunchKernelGGL(int8_build_codes, dim3((unsigned)blocks), dim3(256), 0, s,
                       (const float*)c->rows.p, (const float*)c->norms.p, first_row, count, (int)c->dim,
                       stride, (int8_t*)c->i8_codes.p, (float*)c->i8_u.p, (float*)c->i8_w.p,
                       (float*)c->i8_normsq.p, (float*)c->i8_invsqrt.p);
    return hipGetLastError();
}

// Builds the planes on first use (Int8CodeCache.buffer, Int8CodeCache.swift:140-187).
static int int8_ensure_codes(mans_ctx* ctx, mans_corpus* c) {
    std::lock_guard<std::mutex> g(c->mu);
    if (c->int8_valid) return MANS_OK;
    const size_t n = (size_t)c->n;
    hipError_t e = c->i8_codes.ensure(n * int8_stride(c->dim), ctx->fail_alloc);
    if (e == hipSuccess) e = c->i8_u.ensure(n * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = c->i8_w.ensure(n * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = c->i8_normsq.ensure(n * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = c->i8_invsqrt.ensure(n * sizeof(float), ctx->fail_alloc);
    if (e != hipSuccess) return hip_fail(e, "int8 planes");
    e = int8_refresh_rows(c, 0, c->n, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_fail(e, "int8 code build");
    c->int8_valid = true;
    return MANS_OK;
}

// Runs the pending queries' exact flat scan and scatters the results into
// the query-indexed outputs.
static int int8_exact_fallback(mans_ctx* ctx, const mans_corpus* c, const float* d_q,
                               const std::vector<uint32_t>& pending, int64_t k, uint32_t metric,
                               float* d_dist, uint32_t* d_ids, hipStream_t st, Slot* slot) {
    const int64_t np = (int64_t)pending.size();
    const int dim = (int)c->dim;
    hipError_t e = slot->qidx.ensure(np * sizeof(uint32_t), ctx->fail_alloc);
    if (e == hipSuccess) e = slot->aux2.ensure((size_t)np * dim * sizeof(float), ctx->fail_alloc);
    if (e == hipSuccess) e = slot->aux3.ensure((size_t)np * k * 2 * sizeof(uint32_t), ctx->fail_alloc);
    if (e == hipSuccess)
        e = hipMemcpyAsync(slot->qidx.p, pending.data(), np * sizeof(uint32_t), hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return hip_fail(e, "int8 fallback workspace");
    const uint32_t* d_idx = (const uint32_t*)slot->qidx.p;
    float* gq = (float*)slot->aux2.p;
    hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)np), dim3(256), 0, st, d_q, d_idx, np, dim, gq);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "int8 fallback gather");
    float* td = (float*)slot->aux3.p;
    uint32_t* ti = (uint32_t*)slot->aux3.p + np * k;
    int rc = flat_search_run(ctx, c, gq, np, k, metric, td, ti, st, slot, nullptr, nullptr);
    if (rc != MANS_OK) return rc;
    // flat_search_run reuses qidx for its own retries: upload the map again.
    e = hipMemcpyAsync(slot->qidx.p, pending.data(), np * sizeof(uint32_t), hipMemcpyHostToDevice, st);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(scatter_rows_kernel, dim3((unsigned)np), dim3(64), 0, st,
                           (const uint32_t*)td, d_idx, np, (int)k, (uint32_t*)d_dist);
        hipLaunchKernelGGL(scatter_rows_kernel, dim3((unsigned)np), dim3(64), 0, st, ti, d_idx, np,
                           (int)k, d_ids);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? MANS_OK : hip_fail(e, "int8 fallback scatter");
}

// MANS_INT8_BOUNDS=0 turns the streaming scan's sampled bounds off.
static bool int8_sampled_bounds() {
    static const bool on = [] {
        const char* e = std::getenv("MANS_INT8_BOUNDS");
        return !(e && e[0] == '0');
    }();
    return on;
}

// The threshold-collect scan for single queries and small batches
// (MANS_INT8_COLLECT=0 keeps the lists).
static bool int8_collect_enabled() {
    static const bool on = [] {
        const char* e = std::getenv("MANS_INT8_COLLECT");
        return !(e && e[0] == '0');
    }();
    return on;
}

// Mode-0 batches gather in the MFMA round and run the later budgets on what
// it gathered (MANS_INT8_BATCH_COLLECT=0 keeps the lists).
static bool int8_batch_collect_enabled() {
    static const bool on = [] {
        const char* e = std::getenv("MANS_INT8_BATCH_COLLECT");
        return !(e && e[0] == '0');
    }();
    return on;
}

// Device queries and outputs; h_rounds (nullable, host) receives the rounds.
static int int8_search_run(mans_ctx* ctx, mans_corpus* c, const float* d_q, int64_t nq, int64_t k,
                           uint32_t metric, int32_t mode, int64_t budget, float* d_dist,
                           uint32_t* d_ids, hipStream_t st, Slot* slot, int32_t* h_rounds) {
    if (metric > 2) return fail(MANS_SEARCH_FAILED, "int8 scan does not support this metric");
    if (mode != 0 && mode != 1) return fail(MANS_SEARCH_FAILED, "int8 scan: mode must be 0 or 1");
    if (mode == 1 && budget < 1) return fail(MANS_SEARCH_FAILED, "int8 scan: budget must be >= 1");
    if (c->n < kInt8MinRows)
        return fail(MANS_PIPELINE_UNAVAILABLE, "int8 scan needs at least 16384 rows");
    if (nq <= 0 || k <= 0) return MANS_OK;
    if (ctx->fail_launch) return fail(MANS_EXECUTION_FAILED, "injected launch failure");
    if (nq > 16384) return fail(MANS_SEARCH_FAILED, "int8 scan: at most 16384 queries per call");
    const int64_t n = c->n;
    const int dim = (int)c->dim;
    const int keff = (int)std::min<int64_t>(std::min<int64_t>(k, MANS_MAX_TOP_K), n);
    const bool aligned = (reinterpret_cast<uintptr_t>(d_q) & 15u) == 0;
    const int nch = dim <= kInt8MaxDim ? flat_nch_for_dim(dim) : 0;
    std::vector<int32_t> rounds((size_t)nq, 0);
    auto finish = [&](int rc) {
        if (rc == MANS_OK && h_rounds) std::memcpy(h_rounds, rounds.data(), nq * sizeof(int32_t));
        return rc;
    };
    if (nch == 0 || !aligned) {
        // The float4 rescore needs dim % 4 == 0 and aligned queries.  A
        // proof-checked search returns the exact result either way.
        if (mode == 1) return fail(MANS_PIPELINE_UNAVAILABLE, "int8 scan: unsupported dim or alignment");
        return finish(flat_search_run(ctx, c, d_q, nq, k, metric, d_dist, d_ids, st, slot, nullptr, nullptr));
    }
    int rc = int8_ensure_codes(ctx, c);
    if (rc != MANS_OK) return rc;
    const int stride = int8_stride(dim);
    hipError_t e = slot->aux0.ensure((size_t)nq * stride, ctx->fail_alloc);
    if (e == hipSuccess) e = slot->aux1.ensure((size_t)nq * sizeof(Int8QueryCoef), ctx->fail_alloc);
    if (e != hipSuccess) return hip_fail(e, "int8 query workspace");
    int8_t* qcodes = (int8_t*)slot->aux0.p;
    Int8QueryCoef* coefs = (Int8QueryCoef*)slot->aux1.p;
    // The query quantisation: its own launch, or (a first round on the
    // collect path) inside the sampled launch.
    bool prep_done = false;
    auto launch_prep = [&]() -> hipError_t {
        prep_done = true;
        hipLaunchKernelGGL(int8_query_prep, dim3((unsigned)nq), dim3(256), sizeof(float) * dim, st,
                           d_q, dim, stride, qcodes, coefs);
        return hipGetLastError();
    };

    Int8Planes pl;
    pl.codes = (const int8_t*)c->i8_codes.p;
    pl.u = (const float*)c->i8_u.p;
    pl.w = (const float*)c->i8_w.p;
    pl.normsq = (const float*)c->i8_normsq.p;
    pl.invsqrt = (const float*)c->i8_invsqrt.p;
    pl.stride = stride;

    int64_t kc = mode == 0 ? std::max<int64_t>(256, 16 * (int64_t)keff) : budget;
    kc = std::min<int64_t>(kc, n);
    const int proof = mode == 0 ? kProofMargin : kProofNone;
    const float* rows = (const float*)c->rows.p;
    const float* norms = (const float*)c->norms.p;

    // The sampled launch over every query: the first sixteenth of each
    // block's rows, one slot per wave; its last block per query writes the
    // kc-th smallest block minimum, the query's bound, after the minima in
    // slot->bounds.
    auto sampled_bounds = [&](const FlatPlan& p, int64_t kc, int64_t cnt, auto&& launch,
                              bool prep = false) {
        const size_t mins_bytes = (size_t)cnt * p.nblk * sizeof(uint64_t);
        hipError_t e = slot->bounds.ensure(mins_bytes + (size_t)cnt * sizeof(uint64_t), ctx->fail_alloc);
        if (e != hipSuccess) return e;
        uint64_t* mins = (uint64_t*)slot->bounds.p;
        FlatPlan p1 = p;
        p1.kc = 1;
        p1.cap = flat_cap_for(1);
        I8ScanBounds s0;
        s0.scan_rows = (p.rows_per_block / 16 + 15) / 16 * 16;
        s0.block_min_out = mins;
        s0.qbound_out = mins + (size_t)cnt * p.nblk;
        s0.bound_kc = (int)kc;
        if (prep) {
            s0.prep_codes_out = qcodes;
            s0.prep_coefs_out = coefs;
        }
        return launch(p1, s0);
    };

    // One streaming round over `idx` (empty: every query) at candidate count
    // kc; appends the queries whose proof failed to `grow`.
    auto stream_round = [&](const std::vector<uint32_t>& idx, int64_t kc, bool timed,
                            std::vector<uint32_t>& grow) -> int {
        const int64_t cnt = idx.empty() ? nq : (int64_t)idx.size();
        static const int64_t target = [] {
            const char* e = std::getenv("MANS_INT8_BLOCKS");
            return e ? std::max<int64_t>(1, std::atoll(e)) : (int64_t)512;
        }();
        FlatPlan p = plan_flat(n, cnt, (int)kc, target);
        const uint32_t* d_qidx = nullptr;
        hipError_t e = hipSuccess;
        if (!idx.empty()) {
            e = slot->qidx.ensure(idx.size() * sizeof(uint32_t), ctx->fail_alloc);
            if (e == hipSuccess)
                e = hipMemcpyAsync(slot->qidx.p, idx.data(), idx.size() * sizeof(uint32_t),
                                   hipMemcpyHostToDevice, st);
            d_qidx = (const uint32_t*)slot->qidx.p;
        }
        FlatBuffers fb;
        if (e == hipSuccess) e = prepare_flat_buffers(ctx, slot, p, cnt, st, &fb);
        if (e == hipSuccess) e = slot->status_h.ensure((size_t)cnt);
        if (e != hipSuccess) return hip_fail(e, "int8 scan workspace");
        FlatArgs fa = {};
        fa.cand = fb.cand;
        fa.gcand = fb.gcand;
        fa.counters = fb.counters;
        fa.out_dist = d_dist;
        fa.out_ids = d_ids;
        fa.status = fb.status;
        fa.k = keff;
        fa.k_stride = (int)k;
        fa.group_blocks = p.group_blocks;
        fa.ngroups = p.ngroups;
        if (timed) ctx->time_begin(slot, st);
        auto launch = [&](const FlatPlan& p, const I8ScanBounds& sb) {
            switch (nch) {
            case 1: launch_int8_scan<1>(p, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, proof, fa, sb, st); break;
            case 2: launch_int8_scan<2>(p, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, proof, fa, sb, st); break;
            case 3: launch_int8_scan<3>(p, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, proof, fa, sb, st); break;
            case 4: launch_int8_scan<4>(p, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, proof, fa, sb, st); break;
            case 6: launch_int8_scan<6>(p, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, proof, fa, sb, st); break;
            default: launch_int8_scan<8>(p, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, proof, fa, sb, st); break;
            }
            return hipGetLastError();
        };
        if (nch != 1 && nch != 2 && nch != 3 && nch != 4 && nch != 6 && nch != 8)
            return fail(MANS_PIPELINE_UNAVAILABLE, "int8 scan: unsupported dim");
        I8ScanBounds sb;
        // Blocks of at least 256 rows: a launch over the first sixteenth of
        // each block's rows gives every query its bound first.
        if (idx.empty() && p.rows_per_block >= 256 && p.nblk >= kc && int8_sampled_bounds()) {
            e = sampled_bounds(p, kc, cnt, launch);
            if (e != hipSuccess) return hip_fail(e, "int8 scan bounds");
            sb.qbound = (const uint64_t*)slot->bounds.p + (size_t)cnt * p.nblk;
        }
        if (e == hipSuccess) e = launch(p, sb);
        ctx->time_end(slot, st, "int8_scan");
        if (e == hipSuccess)
            e = hipMemcpyAsync(slot->status_h.p, fb.status, (size_t)cnt, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) {
            slot->counters_dirty = true;
            return hip_fail(e, "int8 scan");
        }
        const uint8_t* sh = (const uint8_t*)slot->status_h.p;
        for (int64_t i = 0; i < cnt; ++i) {
            const uint32_t qi = idx.empty() ? (uint32_t)i : idx[i];
            rounds[qi] += 1;
            if (sh[i]) grow.push_back(qi);
        }
        return MANS_OK;
    };

    // Rounds at budgets up to kInt8MaxBudget take the threshold-collect scan
    // when the sampled bound applies: blocks of at least 256 rows.  The
    // bound is the min(kc, nblk / 2)-th smallest block minimum of the
    // sample.
    static const int64_t collect_target = [] {
        const char* e = std::getenv("MANS_INT8_BLOCKS");
        return e ? std::max<int64_t>(1, std::atoll(e)) : (int64_t)512;
    }();
    auto collect_plan = [&](int64_t kc, FlatPlan* p) {
        if (kc > kInt8MaxBudget || !int8_collect_enabled() || !int8_sampled_bounds()) return false;
        *p = plan_flat(n, 1, (int)std::min<int64_t>(kc, 256), collect_target);
        return p->rows_per_block >= 256 && p->nblk >= 2;
    };
    // One threshold-collect launch over `idx` (empty: every query) starting
    // at budget kc; appends (query, next budget) for the queries whose proof
    // still fails.  Queries whose bound let more rows through than the
    // buffers hold repeat the round with the lists.
    auto collect_round = [&](const FlatPlan& p, const std::vector<uint32_t>& idx, int64_t kc,
                             std::vector<std::pair<uint32_t, int64_t>>& next) -> int {
        const int64_t cnt = idx.empty() ? nq : (int64_t)idx.size();
        FlatBuffers fb;
        hipError_t e = prepare_flat_buffers(ctx, slot, p, cnt, st, &fb);
        // Candidate buffers: slots, then exact slots, ccap each.
        const int64_t ccap = std::min<int64_t>((int64_t)p.nblk * std::max<int64_t>(kc, 256), kCollectMaxCap);
        if (e == hipSuccess)
            e = slot->cand.ensure((size_t)cnt * 2 * ccap * sizeof(uint64_t), ctx->fail_alloc);
        fb.cand = (uint64_t*)slot->cand.p;
        if (e == hipSuccess) e = slot->status_h.ensure((size_t)cnt);
        const uint32_t* d_qidx = nullptr;
        if (e == hipSuccess && !idx.empty()) {
            e = slot->qidx.ensure(idx.size() * sizeof(uint32_t), ctx->fail_alloc);
            if (e == hipSuccess)
                e = hipMemcpyAsync(slot->qidx.p, idx.data(), idx.size() * sizeof(uint32_t),
                                   hipMemcpyHostToDevice, st);
            d_qidx = (const uint32_t*)slot->qidx.p;
        }
        if (e != hipSuccess) return hip_fail(e, "int8 scan workspace");
        FlatArgs fa = {};
        fa.cand = fb.cand;
        fa.gcand = fb.gcand;
        fa.counters = fb.counters;
        fa.out_dist = d_dist;
        fa.out_ids = d_ids;
        fa.status = (uint8_t*)slot->status_h.p;  // pinned: read after the stream syncs
        fa.k = keff;
        fa.k_stride = (int)k;
        fa.group_blocks = p.group_blocks;
        fa.ngroups = p.ngroups;
        auto launch = [&](const FlatPlan& lp, const I8ScanBounds& sb) {
            switch (nch) {
            case 1: launch_int8_scan<1>(lp, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, proof, fa, sb, st); break;
            case 2: launch_int8_scan<2>(lp, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, proof, fa, sb, st); break;
            case 3: launch_int8_scan<3>(lp, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, proof, fa, sb, st); break;
            case 4: launch_int8_scan<4>(lp, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, proof, fa, sb, st); break;
            case 6: launch_int8_scan<6>(lp, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, proof, fa, sb, st); break;
            default: launch_int8_scan<8>(lp, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, proof, fa, sb, st); break;
            }
            return hipGetLastError();
        };
        ctx->time_begin(slot, st);
        const bool prep = !prep_done && dim <= kI8MaxDim;
        if (!prep_done && !prep) e = launch_prep();
        const int64_t bound_kc = std::min<int64_t>(kc, std::max<int64_t>(1, p.nblk / 2));
        if (e == hipSuccess) e = sampled_bounds(p, bound_kc, cnt, launch, prep);
        prep_done = true;
        ctx->time_end(slot, st, "int8_bound");
        I8Collect cl;
        cl.qbound = (const uint64_t*)slot->bounds.p + (size_t)cnt * p.nblk;
        cl.cbuf = fb.cand;
        cl.ebuf = fb.cand + (size_t)cnt * ccap;
        cl.ccap = ccap;
        // Mode 0: the budget rounds run from LDS in a one-block launch per
        // query after the collect launch (its last blocks only record their
        // gathered counts).
        const bool defer = proof == kProofMargin;
        if (defer) {
            if (e == hipSuccess) e = slot->aux2.ensure((size_t)cnt * sizeof(int32_t), ctx->fail_alloc);
            cl.totals = (int32_t*)slot->aux2.p;
        }
        ctx->time_begin(slot, st);
        if (e == hipSuccess) {
            switch (nch) {
            case 1: e = launch_int8_collect<1>(p, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, (int)kc, proof, fa, cl, st); break;
            case 2: e = launch_int8_collect<2>(p, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, (int)kc, proof, fa, cl, st); break;
            case 3: e = launch_int8_collect<3>(p, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, (int)kc, proof, fa, cl, st); break;
            case 4: e = launch_int8_collect<4>(p, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, (int)kc, proof, fa, cl, st); break;
            case 6: e = launch_int8_collect<6>(p, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, (int)kc, proof, fa, cl, st); break;
            default: e = launch_int8_collect<8>(p, pl, rows, norms, n, dim, d_q, d_qidx, cnt, qcodes, coefs, (int)metric, (int)kc, proof, fa, cl, st); break;
            }
        }
        if (e == hipSuccess && defer) {
            static const bool attr = [] {
                (void)hipFuncSetAttribute((const void*)int8_collect_rounds,
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)kI8RoundsLds);
                return true;
            }();
            (void)attr;
            hipLaunchKernelGGL(int8_collect_rounds, dim3(1, (unsigned)cnt), dim3(kI8RoundsThreads),
                               kI8RoundsLds, st, n, d_qidx, (int)kc, proof, fa, cl);
            e = hipGetLastError();
        }
        ctx->time_end(slot, st, "int8_scan");
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) {
            slot->counters_dirty = true;
            return hip_fail(e, "int8 scan");
        }
        std::vector<uint32_t> redo;
        const uint8_t* sh = (const uint8_t*)slot->status_h.p;
        for (int64_t i = 0; i < cnt; ++i) {
            const uint32_t qi = idx.empty() ? (uint32_t)i : idx[i];
            const int outcome = sh[i] & 3, ran = sh[i] >> 2;
            if (outcome == kStatusReselect) {
                redo.push_back(qi);
                continue;
            }
            rounds[qi] += ran;
            if (outcome == 1) {
                int64_t b = kc;
                for (int r = 0; r < ran; ++r) b = std::min<int64_t>(b * 4, n);
                next.emplace_back(qi, b);
            }
        }
        ctx->reselects += (int64_t)redo.size();
        if (!redo.empty()) {
            std::vector<uint32_t> grow;
            int rc = stream_round(redo, kc, true, grow);
            if (rc != MANS_OK) return rc;
            for (uint32_t qi : grow) next.emplace_back(qi, std::min<int64_t>(kc * 4, n));
        }
        return MANS_OK;
    };

    // Mode-0 batches: the first round's contraction gathers every slot at or
    // below a bound of max(kc, kI8CollectBoundKc) sampled slots, and one block
    // per query runs the budget rounds on what was gathered
    // (int8_collect_merge); queries it cannot serve repeat the round on the
    // streaming scan.
    auto gemm_collect_round = [&](const I8GemmPlan& gp, int64_t kc,
                                  std::vector<std::pair<uint32_t, int64_t>>& next) -> int {
        const int nreg = 2 * gp.nseg;
        const size_t lbytes = (size_t)nq * gp.nseg * 2 * kI8List * sizeof(uint64_t);
        const size_t cbytes = (size_t)nq * nreg * kI8CollectCap * sizeof(uint64_t);
        const size_t nbytes = ((size_t)nq * nreg * sizeof(int32_t) + 255) / 256 * 256;
        const size_t fbytes = ((size_t)nq * sizeof(uint32_t) + 255) / 256 * 256;
        hipError_t e = slot->cand.ensure(lbytes + (size_t)nq * sizeof(uint64_t), ctx->fail_alloc);
        if (e == hipSuccess) e = slot->aux2.ensure(cbytes + nbytes + fbytes, ctx->fail_alloc);
        if (e == hipSuccess) e = slot->status_h.ensure((size_t)nq);
        if (e != hipSuccess) return hip_fail(e, "int8 batch workspace");
        uint64_t* lists = (uint64_t*)slot->cand.p;
        uint64_t* qbound = lists + lbytes / sizeof(uint64_t);
        uint64_t* cbuf = (uint64_t*)slot->aux2.p;
        int32_t* ccount = (int32_t*)((char*)slot->aux2.p + cbytes);
        uint32_t* cflag = (uint32_t*)((char*)slot->aux2.p + cbytes + nbytes);
        const int64_t sampled_slots = (int64_t)2 * gp.s_nseg * kI8List;
        const int bound_kc = (int)std::min<int64_t>(std::max<int64_t>(kc, kI8CollectBoundKc),
                                                    sampled_slots / 2);
        ctx->time_begin(slot, st);
        e = hipMemsetAsync(cflag, 0, (size_t)nq * sizeof(uint32_t), st);
        if (e == hipSuccess)
            e = launch_i8gemm(gp, pl, n, qcodes, coefs, nq, (int)metric, true, nullptr, lists, st);
        if (e == hipSuccess) {
            hipLaunchKernelGGL(int8_lists_bound, dim3(1, (unsigned)nq), dim3(256),
                               sampled_slots <= kKthLdsSlots ? sizeof(uint64_t) * (size_t)sampled_slots : 0,
                               st, bound_kc, 2 * gp.s_nseg, (const uint64_t*)lists, qbound);
            e = hipGetLastError();
        }
        ctx->time_end(slot, st, "int8_bound");
        ctx->time_begin(slot, st);
        if (e == hipSuccess)
            e = launch_i8gemm(gp, pl, n, qcodes, coefs, nq, (int)metric, false, qbound, lists, st,
                              cbuf, ccount, cflag, kI8CollectCap);
        ctx->time_end(slot, st, "int8_gemm");
        FlatArgs fa = {};
        fa.out_dist = d_dist;
        fa.out_ids = d_ids;
        fa.status = (uint8_t*)slot->status_h.p;  // pinned: read after the stream syncs
        fa.k = keff;
        fa.k_stride = (int)k;
        ctx->time_begin(slot, st);
        if (e == hipSuccess) {
            switch (nch) {
            case 1: e = launch_i8_collect_merge<1>(rows, norms, n, dim, d_q, coefs, nq, (int)metric, (int)kc, nreg, cbuf, ccount, cflag, proof, fa, st); break;
            case 2: e = launch_i8_collect_merge<2>(rows, norms, n, dim, d_q, coefs, nq, (int)metric, (int)kc, nreg, cbuf, ccount, cflag, proof, fa, st); break;
            case 3: e = launch_i8_collect_merge<3>(rows, norms, n, dim, d_q, coefs, nq, (int)metric, (int)kc, nreg, cbuf, ccount, cflag, proof, fa, st); break;
            case 4: e = launch_i8_collect_merge<4>(rows, norms, n, dim, d_q, coefs, nq, (int)metric, (int)kc, nreg, cbuf, ccount, cflag, proof, fa, st); break;
            case 6: e = launch_i8_collect_merge<6>(rows, norms, n, dim, d_q, coefs, nq, (int)metric, (int)kc, nreg, cbuf, ccount, cflag, proof, fa, st); break;
            case 8: e = launch_i8_collect_merge<8>(rows, norms, n, dim, d_q, coefs, nq, (int)metric, (int)kc, nreg, cbuf, ccount, cflag, proof, fa, st); break;
            default: return fail(MANS_PIPELINE_UNAVAILABLE, "int8 scan: unsupported dim");
            }
        }
        ctx->time_end(slot, st, "int8_merge");
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "int8 batch scan");
        std::vector<uint32_t> redo;
        const uint8_t* sh = (const uint8_t*)slot->status_h.p;
        for (int64_t i = 0; i < nq; ++i) {
            const int outcome = sh[i] & 3, ran = sh[i] >> 2;
            if (outcome == kStatusReselect) {
                redo.push_back((uint32_t)i);
                continue;
            }
            rounds[i] += ran;
            if (outcome == 1) {
                int64_t b = kc;
                for (int r = 0; r < ran; ++r) b = std::min<int64_t>(b * 4, n);
                next.emplace_back((uint32_t)i, b);
            }
        }
        ctx->reselects += (int64_t)redo.size();
        if (!redo.empty()) {
            std::vector<uint32_t> grow;
            int rc = stream_round(redo, kc, true, grow);
            if (rc != MANS_OK) return rc;
            for (uint32_t qi : grow) next.emplace_back(qi, std::min<int64_t>(kc * 4, n));
        }
        return MANS_OK;
    };

    // The first round of a batch on i8 MFMA; queries whose lists cannot
    // show an exact selection repeat the round on the streaming scan.
    auto gemm_round = [&](const I8GemmPlan& gp, int64_t kc, std::vector<uint32_t>& grow) -> int {
        const size_t lbytes = (size_t)nq * gp.nseg * 2 * kI8List * sizeof(uint64_t);
        hipError_t e = slot->cand.ensure(lbytes + (size_t)nq * sizeof(uint64_t), ctx->fail_alloc);
        if (e == hipSuccess) e = slot->status.ensure((size_t)nq, ctx->fail_alloc);
        if (e == hipSuccess) e = slot->status_h.ensure((size_t)nq);
        if (e != hipSuccess) return hip_fail(e, "int8 batch workspace");
        uint64_t* lists = (uint64_t*)slot->cand.p;
        uint64_t* qbound = lists + lbytes / sizeof(uint64_t);
        // Bounds from the sampled rows, then the full contraction.
        ctx->time_begin(slot, st);
        e = launch_i8gemm(gp, pl, n, qcodes, coefs, nq, (int)metric, true, nullptr, lists, st);
        if (e == hipSuccess) {
            const int64_t slots = (int64_t)2 * gp.s_nseg * kI8List;
            hipLaunchKernelGGL(int8_lists_bound, dim3(1, (unsigned)nq), dim3(256),
                               slots <= kKthLdsSlots ? sizeof(uint64_t) * (size_t)slots : 0, st,
                               (int)kc, 2 * gp.s_nseg, (const uint64_t*)lists, qbound);
            e = hipGetLastError();
        }
        ctx->time_end(slot, st, "int8_bound");
        ctx->time_begin(slot, st);
        if (e == hipSuccess)
            e = launch_i8gemm(gp, pl, n, qcodes, coefs, nq, (int)metric, false, qbound,
                              lists, st);
        ctx->time_end(slot, st, "int8_gemm");
        FlatArgs fa = {};
        fa.out_dist = d_dist;
        fa.out_ids = d_ids;
        fa.status = (uint8_t*)slot->status.p;
        fa.k = keff;
        fa.k_stride = (int)k;
        ctx->time_begin(slot, st);
        if (e == hipSuccess) {
            switch (nch) {
            case 1: launch_i8_merge<1>(gp, rows, norms, n, dim, d_q, coefs, nq, (int)metric, (int)kc, lists, proof, fa, st); break;
            case 2: launch_i8_merge<2>(gp, rows, norms, n, dim, d_q, coefs, nq, (int)metric, (int)kc, lists, proof, fa, st); break;
            case 3: launch_i8_merge<3>(gp, rows, norms, n, dim, d_q, coefs, nq, (int)metric, (int)kc, lists, proof, fa, st); break;
            case 4: launch_i8_merge<4>(gp, rows, norms, n, dim, d_q, coefs, nq, (int)metric, (int)kc, lists, proof, fa, st); break;
            case 6: launch_i8_merge<6>(gp, rows, norms, n, dim, d_q, coefs, nq, (int)metric, (int)kc, lists, proof, fa, st); break;
            case 8: launch_i8_merge<8>(gp, rows, norms, n, dim, d_q, coefs, nq, (int)metric, (int)kc, lists, proof, fa, st); break;
            default: return fail(MANS_PIPELINE_UNAVAILABLE, "int8 scan: unsupported dim");
            }
            e = hipGetLastError();
        }
        ctx->time_end(slot, st, "int8_merge");
        if (e == hipSuccess)
            e = hipMemcpyAsync(slot->status_h.p, slot->status.p, (size_t)nq, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "int8 batch scan");
        std::vector<uint32_t> redo;
        const uint8_t* sh = (const uint8_t*)slot->status_h.p;
        for (int64_t i = 0; i < nq; ++i) {
            if (sh[i] == kStatusReselect) {
                redo.push_back((uint32_t)i);
                continue;
            }
            rounds[i] += 1;
            if (sh[i]) grow.push_back((uint32_t)i);
        }
        ctx->reselects += (int64_t)redo.size();
        if (!redo.empty()) {
            int rc = stream_round(redo, kc, true, grow);
            if (rc != MANS_OK) return rc;
            std::sort(grow.begin(), grow.end());
        }
        return MANS_OK;
    };

    // Budgets still to run, each with its queries (an empty list at the
    // first budget: every query).  Budgets grow 4x per failed proof
    // (BoundedExactScan.swift:115-118); past kInt8MaxBudget the exact scan
    // finishes the remaining queries.
    std::map<int64_t, std::vector<uint32_t>> todo;
    todo[kc] = {};
    bool first = true;
    while (!todo.empty()) {
        const int64_t bkc = todo.begin()->first;
        std::vector<uint32_t> idx = std::move(todo.begin()->second);
        todo.erase(todo.begin());
        if (bkc > kInt8MaxBudget) {
            if (mode == 1)
                return fail(MANS_PIPELINE_UNAVAILABLE, "int8 scan: fixed budget above 1024");
            if (idx.empty()) {
                idx.resize((size_t)nq);
                for (int64_t i = 0; i < nq; ++i) idx[i] = (uint32_t)i;
            }
            for (auto& rest : todo) idx.insert(idx.end(), rest.second.begin(), rest.second.end());
            std::sort(idx.begin(), idx.end());
            for (uint32_t qi : idx) rounds[qi] += 1;
            return finish(int8_exact_fallback(ctx, c, d_q, idx, k, metric, d_dist, d_ids, st, slot));
        }
        std::vector<std::pair<uint32_t, int64_t>> next;
        I8GemmPlan gp;
        FlatPlan cp;
        int rc;
        const bool gemm = first && idx.empty() && plan_i8gemm(n, stride, nq, bkc, &gp);
        // Many queries at once keep HBM busy on the list scan; the collect
        // launch serves single queries and small groups.
        const bool collect =
            !gemm && (idx.empty() ? nq : (int64_t)idx.size()) <= kCollectMaxQueries &&
            collect_plan(bkc, &cp);
        if (!prep_done && !collect) {
            e = launch_prep();
            if (e != hipSuccess) return hip_fail(e, "int8 query prep");
        }
        if (collect) {
            rc = collect_round(cp, idx, bkc, next);
        } else if (gemm && mode == 0 && int8_batch_collect_enabled()) {
            rc = gemm_collect_round(gp, bkc, next);
        } else {
            std::vector<uint32_t> grow;
            rc = gemm ? gemm_round(gp, bkc, grow) : stream_round(idx, bkc, !first, grow);
            for (uint32_t qi : grow) next.emplace_back(qi, std::min<int64_t>(bkc * 4, n));
        }
        if (rc != MANS_OK) return rc;
        first = false;
        for (const auto& qn : next) {
            if (qn.second <= bkc)  // the budget cannot grow: every row was selected
                return fail(MANS_SEARCH_FAILED, "int8 scan: proof failed with every row selected");
            todo[qn.second].push_back(qn.first);
            ctx->proof_retries += 1;
        }
        for (auto& t : todo) std::sort(t.second.begin(), t.second.end());
    }
    return finish(MANS_OK);
}

}  // namespace mans

using namespace mans;

extern "C" {

int mans_int8_search_device(mans_ctx* ctx, mans_corpus* c, const float* d_queries, int64_t nq,
                            int64_t k, uint32_t metric, int32_t mode, int64_t budget,
                            float* d_out_dist, uint32_t* d_out_ids, void* stream) {
    if (!ctx || !c) return fail(MANS_SEARCH_FAILED, "NULL context or corpus");
    if (check_k(k) != MANS_OK) return MANS_SEARCH_FAILED;
    if (nq > 0 && k > 0 && (!d_queries || !d_out_dist || !d_out_ids))
        return fail(MANS_SEARCH_FAILED, "NULL buffer");
    DeviceGuard dg(ctx->device);
    SlotLease lease(ctx);
    if (!lease.slot) return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    hipStream_t st = stream ? (hipStream_t)stream : lease.slot->stream;
    return int8_search_run(ctx, c, d_queries, nq, k, metric, mode, budget, d_out_dist, d_out_ids,
                           st, lease.slot, nullptr);
}

int mans_int8_search(mans_ctx* ctx, mans_corpus* c, const float* queries, int64_t nq, int64_t k,
                     uint32_t metric, int32_t mode, int64_t budget, float* out_dist,
                     uint32_t* out_ids, int32_t* out_rounds) {
    if (!ctx || !c) return fail(MANS_SEARCH_FAILED, "NULL context or corpus");
    if (check_k(k) != MANS_OK) return MANS_SEARCH_FAILED;
    if (nq <= 0 || k <= 0) return MANS_OK;
    if (!queries || !out_dist || !out_ids) return fail(MANS_SEARCH_FAILED, "NULL buffer");
    DeviceGuard dg(ctx->device);
    SlotLease lease(ctx);
    Slot* s = lease.slot;
    if (!s) return fail(MANS_RESOURCE_EXHAUSTED, "could not create a HIP stream");
    const size_t qbytes = (size_t)nq * c->dim * sizeof(float);
    const size_t obytes = (size_t)nq * k * sizeof(float);
    hipError_t e = s->queries.ensure(qbytes, ctx->fail_alloc);
    if (e == hipSuccess) e = s->dist.ensure(obytes, ctx->fail_alloc);
    if (e == hipSuccess) e = s->ids.ensure(obytes, ctx->fail_alloc);
    if (e == hipSuccess) e = stage_to_device(s, s->queries.p, queries, qbytes);
    if (e != hipSuccess) return hip_fail(e, "int8 scan staging");
    int rc = int8_search_run(ctx, c, (const float*)s->queries.p, nq, k, metric, mode, budget,
                             (float*)s->dist.p, (uint32_t*)s->ids.p, s->stream, s, out_rounds);
    if (rc != MANS_OK) return rc;
    e = stage_from_device(s, out_dist, s->dist.p, obytes, out_ids, s->ids.p, obytes);
    return e == hipSuccess ? MANS_OK : hip_fail(e, "int8 scan results");
}

int mans_int8_codes_download(mans_ctx* ctx, mans_corpus* c, int8_t* codes, float* u, float* w,
                             float* normsq, float* invsqrt) {
    if (!ctx || !c) return fail(MANS_SEARCH_FAILED, "NULL context or corpus");
    DeviceGuard dg(ctx->device);
    int rc = int8_ensure_codes(ctx, c);
    if (rc != MANS_OK) return rc;
    const int64_t n = c->n, dim = c->dim;
    const int stride = int8_stride(dim);
    hipError_t e = hipSuccess;
    if (codes && n > 0)
        e = hipMemcpy2D(codes, (size_t)dim, c->i8_codes.p, (size_t)stride, (size_t)dim, (size_t)n,
                        hipMemcpyDeviceToHost);
    const size_t pb = (size_t)n * sizeof(float);
    if (e == hipSuccess && u) e = hipMemcpy(u, c->i8_u.p, pb, hipMemcpyDeviceToHost);
    if (e == hipSuccess && w) e = hipMemcpy(w, c->i8_w.p, pb, hipMemcpyDeviceToHost);
    if (e == hipSuccess && normsq) e = hipMemcpy(normsq, c->i8_normsq.p, pb, hipMemcpyDeviceToHost);
    if (e == hipSuccess && invsqrt) e = hipMemcpy(invsqrt, c->i8_invsqrt.p, pb, hipMemcpyDeviceToHost);
    return e == hipSuccess ? MANS_OK : hip_fail(e, "int8 planes download");
}

}  // extern "C"
