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

// One block per query (BoundedExactScan.swift:52-94).  dynamic LDS: dim floats.
__global__ __launch_bounds__(256) void int8_query_prep(const float* __restrict__ queries, int dim,
                                                       int stride, int8_t* __restrict__ qcodes,
                                                       Int8QueryCoef* __restrict__ coefs) {
    extern __shared__ float qsh[];
    __shared__ uint32_t max_bits;
    __shared__ int abs_sum;
    const int tid = threadIdx.x;
    const int64_t q = blockIdx.x;
    const float* qp = queries + q * dim;
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
        qcodes[q * stride + d] = (int8_t)c;
        a += c < 0 ? -c : c;
    }
    atomicAdd(&abs_sum, a);
    __syncthreads();
    if (tid == 0) {
        float qn = 0.0f;  // the sequential norm of FlatGPUSearch.swift:532-535
#pragma unroll 16
        for (int d = 0; d < dim; ++d) qn += qsh[d] * qsh[d];
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
        coefs[q] = c;
    }
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

struct Int8Planes {
    const int8_t* codes;
    const float* u;
    const float* w;
    const float* normsq;
    const float* invsqrt;
    int stride;
};

// grid (nblk, nq_launch); block 256; dynamic LDS: 4 * cap slots.
// NCH: float4 chunks per lane for the rescore (16 lanes per row); the int8
// rows use (NCH + 1) / 2 16-byte chunks per lane with 8 lanes per row.
template <int NCH>
__global__ __launch_bounds__(256) void int8_scan(
    Int8Planes pl, const float* __restrict__ rows, const float* __restrict__ norms, int64_t n,
    int dim, const float* __restrict__ queries, const uint32_t* __restrict__ qidx,
    const int8_t* __restrict__ qcodes, const Int8QueryCoef* __restrict__ coefs, int metric, int kc,
    int cap, int64_t rows_per_block, int proof, FlatArgs fa) {
    constexpr int NC8 = (NCH + 1) / 2;
    extern __shared__ uint64_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g8 = lane >> 3, l8 = lane & 7;
    const uint32_t q = qidx ? qidx[blockIdx.y] : blockIdx.y;
    const int nchunk = pl.stride >> 4;
    const Int8QueryCoef coef = coefs[q];

    i4v qc[NC8];
#pragma unroll
    for (int c = 0; c < NC8; ++c) {
        const int idx = l8 + 8 * c;
        qc[c] = idx < nchunk ? *reinterpret_cast<const i4v*>(qcodes + (int64_t)q * pl.stride + 16 * idx)
                             : i4v{0, 0, 0, 0};
    }

    WaveTopK sel;
    sel.init(lds + wave * cap, cap, kc);
    const int64_t start = (int64_t)blockIdx.x * rows_per_block;
    const int64_t end = start + rows_per_block < n ? start + rows_per_block : n;
    // Each 8-lane group takes kRows rows per step (rows g8 + 8 j of the
    // wave's 8 kRows), so a wave has 8 kRows rows of codes in flight.
    constexpr int kRows = 4;
    for (int64_t base = start; base < end; base += 4 * 8 * kRows) {
        int64_t r[kRows];
        bool v[kRows];
        float pu[kRows], pw[kRows], pn[kRows];
        i4v a[kRows][NC8];
#pragma unroll
        for (int j = 0; j < kRows; ++j) {
            r[j] = base + wave * 8 * kRows + g8 + 8 * j;
            v[j] = r[j] < end;
            // Plane values of clamped rows, so every load is unconditional.
            const int64_t cr = v[j] ? r[j] : start;
            pu[j] = pl.u[cr];
            pw[j] = pl.w[cr];
            pn[j] = metric == kMetricL2 ? pl.normsq[cr] : pl.invsqrt[cr];
            // Chunks past the row's end re-read its last chunk; the query's
            // codes there are zero, so they add nothing (and the load needs
            // no branch).
            const i4v* src = reinterpret_cast<const i4v*>(pl.codes + cr * pl.stride);
#pragma unroll
            for (int c = 0; c < NC8; ++c) {
                const int idx = l8 + 8 * c;
                a[j][c] = __builtin_nontemporal_load(src + (idx < nchunk ? idx : nchunk - 1));
            }
        }
        // Every lane of a group ends with the group's dot of each row; lane
        // l8 = j < kRows then keys row j, so one offer covers the step.
        int sj = 0;
        float uj = 0.0f, wj = 0.0f, nj = 0.0f;
        int64_t rj = 0;
        bool vj = false;
#pragma unroll
        for (int j = 0; j < kRows; ++j) {
            int s = 0;
#pragma unroll
            for (int c = 0; c < NC8; ++c) s = dot16_i8(a[j][c], qc[c], s);
            s = sum8(s);
            const bool mine = l8 == j;
            sj = mine ? s : sj;
            uj = mine ? pu[j] : uj;
            wj = mine ? pw[j] : wj;
            nj = mine ? pn[j] : nj;
            rj = mine ? r[j] : rj;
            vj = mine ? v[j] : vj;
        }
        const float key = int8_key(metric, coef, (float)sj, uj, wj, nj, nj);
        sel.offer(vj, key, (uint32_t)rj);
    }
    sel.finish();
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
                             hipStream_t s) {
    size_t shmem = sizeof(uint64_t) * 4 * (size_t)p.cap;
    hipLaunchKernelGGL(int8_scan<NCH>, dim3(p.nblk, (unsigned)nq), dim3(256), shmem, s, pl, rows,
                       norms, n, dim, queries, qidx, qcodes, coefs, metric, p.kc, p.cap,
                       p.rows_per_block, proof, fa);
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
    ctx->time_begin(slot, st);
    hipLaunchKernelGGL(int8_query_prep, dim3((unsigned)nq), dim3(256), sizeof(float) * dim, st, d_q,
                       dim, stride, qcodes, coefs);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "int8 query prep");

    Int8Planes pl;
    pl.codes = (const int8_t*)c->i8_codes.p;
    pl.u = (const float*)c->i8_u.p;
    pl.w = (const float*)c->i8_w.p;
    pl.normsq = (const float*)c->i8_normsq.p;
    pl.invsqrt = (const float*)c->i8_invsqrt.p;
    pl.stride = stride;

    int64_t kc = mode == 0 ? std::max<int64_t>(256, 16 * (int64_t)keff) : budget;
    kc = std::min<int64_t>(kc, n);
    std::vector<uint32_t> pending;  // empty = all queries
    int64_t npend = nq;
    bool first = true;
    for (;;) {
        if (kc > kInt8MaxBudget) {
            if (mode == 1)
                return fail(MANS_PIPELINE_UNAVAILABLE, "int8 scan: fixed budget above 1024");
            std::vector<uint32_t> all;
            const std::vector<uint32_t>* idx = &pending;
            if (pending.empty()) {
                all.resize((size_t)nq);
                for (int64_t i = 0; i < nq; ++i) all[i] = (uint32_t)i;
                idx = &all;
            }
            for (uint32_t qi : *idx) rounds[qi] += 1;
            return finish(int8_exact_fallback(ctx, c, d_q, *idx, k, metric, d_dist, d_ids, st, slot));
        }
        static const int64_t target = [] {
            const char* e = std::getenv("MANS_INT8_BLOCKS");
            return e ? std::max<int64_t>(1, std::atoll(e)) : (int64_t)512;
        }();
        FlatPlan p = plan_flat(n, npend, (int)kc, target);
        const uint32_t* d_qidx = nullptr;
        if (!pending.empty()) {
            e = slot->qidx.ensure(pending.size() * sizeof(uint32_t), ctx->fail_alloc);
            if (e == hipSuccess)
                e = hipMemcpyAsync(slot->qidx.p, pending.data(), pending.size() * sizeof(uint32_t),
                                   hipMemcpyHostToDevice, st);
            d_qidx = (const uint32_t*)slot->qidx.p;
        }
        FlatBuffers fb;
        if (e == hipSuccess) e = prepare_flat_buffers(ctx, slot, p, npend, st, &fb);
        if (e == hipSuccess) e = slot->status_h.ensure((size_t)npend);
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
        const int proof = mode == 0 ? kProofMargin : kProofNone;
        if (!first) ctx->time_begin(slot, st);
        switch (nch) {
        case 1: launch_int8_scan<1>(p, pl, (const float*)c->rows.p, (const float*)c->norms.p, n, dim, d_q, d_qidx, npend, qcodes, coefs, (int)metric, proof, fa, st); break;
        case 2: launch_int8_scan<2>(p, pl, (const float*)c->rows.p, (const float*)c->norms.p, n, dim, d_q, d_qidx, npend, qcodes, coefs, (int)metric, proof, fa, st); break;
        case 3: launch_int8_scan<3>(p, pl, (const float*)c->rows.p, (const float*)c->norms.p, n, dim, d_q, d_qidx, npend, qcodes, coefs, (int)metric, proof, fa, st); break;
        case 4: launch_int8_scan<4>(p, pl, (const float*)c->rows.p, (const float*)c->norms.p, n, dim, d_q, d_qidx, npend, qcodes, coefs, (int)metric, proof, fa, st); break;
        case 6: launch_int8_scan<6>(p, pl, (const float*)c->rows.p, (const float*)c->norms.p, n, dim, d_q, d_qidx, npend, qcodes, coefs, (int)metric, proof, fa, st); break;
        case 8: launch_int8_scan<8>(p, pl, (const float*)c->rows.p, (const float*)c->norms.p, n, dim, d_q, d_qidx, npend, qcodes, coefs, (int)metric, proof, fa, st); break;
        default: return fail(MANS_PIPELINE_UNAVAILABLE, "int8 scan: unsupported dim");
        }
        e = hipGetLastError();
        ctx->time_end(slot, st, "int8_scan");
        first = false;
        if (e == hipSuccess)
            e = hipMemcpyAsync(slot->status_h.p, fb.status, (size_t)npend, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) {
            slot->counters_dirty = true;
            return hip_fail(e, "int8 scan");
        }
        const uint8_t* sh = (const uint8_t*)slot->status_h.p;
        std::vector<uint32_t> next;
        for (int64_t i = 0; i < npend; ++i) {
            const uint32_t qi = pending.empty() ? (uint32_t)i : pending[i];
            rounds[qi] += 1;
            if (sh[i]) next.push_back(qi);
        }
        if (next.empty()) return finish(MANS_OK);
        if (kc >= n) return fail(MANS_SEARCH_FAILED, "int8 scan: proof failed with every row selected");
        pending.swap(next);
        npend = (int64_t)pending.size();
        kc = std::min<int64_t>(kc * 4, n);
        ctx->proof_retries += npend;
    }
}

}  // namespace mans

using namespace mans;

extern "C" {

int mans_int8_search_device(mans_ctx* ctx, mans_corpus* c, const float* d_queries, int64_t nq,
                            int64_t k, uint32_t metric, int32_t mode, int64_t budget,
                            float* d_out_dist, uint32_t* d_out_ids, void* stream) {
    if (!ctx || !c) return fail(MANS_SEARCH_FAILED, "NULL context or corpus");
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
