// Exact flat scan on gfx950: FlatGPUSearch.batchSearch / ParallelFlatScan.search
// (FlatGPUSearch.swift:103-181, ParallelFlatScan.swift:96-155) as three steps.
//
//  1. flat_scan_f4: HBM-bound streaming pass.  16 lanes per row, 128-bit loads,
//     fused multiply-adds in any order, a 16-lane DPP reduction, then a
//     provable lower bound on the exact distance (the "key").  Each wave keeps
//     its best kc keys in LDS (WaveTopK); the block merges its 4 waves and
//     writes kc slots.
//  2. flat_merge_rescore: one block per query picks the kc smallest keys over
//     all blocks, recomputes those rows' distances in the scalar order of
//     dots.c:40-47 with the host formulas (bit-identical to the CPU path),
//     sorts by (distance, id) and writes k.  The query passes the proof when
//     the kc-th key is >= the k-th exact distance: every row left out then
//     has an exact distance >= that of every row returned.
//  3. The host re-runs queries that fail the proof with a larger kc, and
//     past the largest kc with flat_scan_rows (exact distances as keys).
//
// The lower bound: any summation order of d products has error at most
// gamma_d * sum|q_i v_i| <= gamma_d * |q| |v|, gamma_d = d u / (1 - d u),
// u = 2^-24 (Higham, Accuracy and Stability of Numerical Algorithms, 3.1).
// Both the fast dot and the sequential dot obey it, so their difference is
// at most twice that; the per-metric constants also absorb the rounding of
// the finalising operations and of the fast query norm.
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

// grid: (nblk, nq_launch); block 256 = 4 waves; dynamic LDS: 4 * cap slots.
template <int NCH>
__global__ __launch_bounds__(256) void flat_scan_f4(
    const float* __restrict__ rows, const float* __restrict__ norms, int64_t n, int dim,
    const float* __restrict__ queries, const uint32_t* __restrict__ qidx, int metric,
    BoundCoef bc, int kc, int cap, int64_t rows_per_block, uint64_t* __restrict__ cand) {
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
    __syncthreads();
    block_bitonic_sort(lds, 4 * cap);
    uint64_t* out = cand + ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * kc;
    for (int i = tid; i < kc; i += 256) out[i] = lds[i];
}

// Exact-key variant: one thread per row, distances in the scalar dots.c
// order with the host formulas.  Used for dims the float4 path does not
// cover and as the terminal round of the proof loop.
// dynamic LDS: 4 * cap slots + dim floats.
__global__ __launch_bounds__(256) void flat_scan_rows(
    const float* __restrict__ rows, const float* __restrict__ norms, int64_t n, int dim,
    const float* __restrict__ queries, const uint32_t* __restrict__ qidx, int metric, int kc,
    int cap, int64_t rows_per_block, uint64_t* __restrict__ cand) {
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
    __syncthreads();
    block_bitonic_sort(lds, 4 * cap);
    uint64_t* out = cand + ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * kc;
    for (int i = tid; i < kc; i += 256) out[i] = lds[i];
}

// One block per query.  dynamic LDS: 4 * cap slots (cap >= 2 kc).
__global__ __launch_bounds__(256) void flat_merge_rescore(
    const uint64_t* __restrict__ cand, int nblk, int kc, int cap,
    const float* __restrict__ rows, const float* __restrict__ norms, int64_t n, int dim,
    const float* __restrict__ queries, const uint32_t* __restrict__ qidx, int metric, int k,
    int k_stride, float* __restrict__ out_dist, uint32_t* __restrict__ out_ids,
    uint8_t* __restrict__ status) {
    extern __shared__ uint64_t lds[];
    __shared__ float qn_sh;
    __shared__ int ncand_sh;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t q = qidx ? qidx[blockIdx.x] : blockIdx.x;
    const uint64_t* src = cand + (int64_t)blockIdx.x * nblk * kc;
    const int64_t total = (int64_t)nblk * kc;

    WaveTopK sel;
    sel.init(lds + wave * cap, cap, kc);
    for (int64_t base = (int64_t)wave * 64; base < total; base += 256) {
        int64_t i = base + lane;
        uint64_t s = i < total ? src[i] : kEmptySlot;
        bool v = s != kEmptySlot;
        sel.offer(v, v ? slot_key(s) : 0.0f, slot_id(s));
    }
    sel.finish();
    __syncthreads();
    block_bitonic_sort(lds, 4 * cap);  // lds[0, kc) = kc smallest keys

    const float* qp = queries + (int64_t)q * dim;
    if (tid == 0) {
        qn_sh = (metric == kMetricIP) ? 0.0f : exact_dot(qp, qp, dim);
        int c = 0;
        while (c < kc && lds[c] != kEmptySlot) ++c;
        ncand_sh = c;
    }
    __syncthreads();
    const float qn = qn_sh;
    const int ncand = ncand_sh;
    const float cutoff = ncand > 0 ? slot_key(lds[ncand - 1]) : 0.0f;

    // Rescore into lds[kc, 2 kc).
    uint64_t* res = lds + kc;
    for (int i = tid; i < kc; i += 256) {
        uint64_t s = lds[i];
        if (i < ncand) {
            uint32_t id = slot_id(s);
            float dot = exact_dot(rows + (int64_t)id * dim, qp, dim);
            float dist = host_distance(dot, qn, metric == kMetricIP ? 0.0f : norms[id], metric);
            res[i] = pack_slot(dist, id);
        } else {
            res[i] = kEmptySlot;
        }
    }
    __syncthreads();
    block_bitonic_sort(res, kc);

    const int kout = k < ncand ? k : ncand;
    for (int i = tid; i < k_stride; i += 256) {
        float dv = kFltMax;
        uint32_t id = kEmptyId;
        if (i < kout) {
            id = slot_id(res[i]);
            dv = slot_key(res[i]);
        }
        out_dist[(int64_t)q * k_stride + i] = dv;
        out_ids[(int64_t)q * k_stride + i] = id;
    }
    if (tid == 0) {
        bool all_rows = (int64_t)ncand >= n;
        bool ok = all_rows || (kout > 0 && cutoff >= slot_key(res[kout - 1]));
        status[blockIdx.x] = ok ? 0 : 1;
    }
}

// Squared norms in the scalar order of dots.c:40-47 (one thread per row).
__global__ void row_norms_kernel(const float* __restrict__ rows, int64_t n, int dim,
                                 float* __restrict__ out) {
    int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n) return;
    const float* p = rows + r * dim;
    float acc = 0.0f;
    for (int d = 0; d < dim; ++d) acc = acc + p[d] * p[d];
    out[r] = acc;
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
    int64_t want_blocks = (4096 + nq - 1) / nq;
    int64_t max_blocks = (n + 127) / 128;
    if (want_blocks > max_blocks) want_blocks = max_blocks;
    if (want_blocks < 1) want_blocks = 1;
    int64_t rpb = (n + want_blocks - 1) / want_blocks;
    rpb = (rpb + 255) / 256 * 256;
    p.rows_per_block = rpb;
    p.nblk = (int)((n + rpb - 1) / rpb);
    return p;
}

template <int NCH>
static void launch_f4(const FlatPlan& p, const float* rows, const float* norms, int64_t n, int dim,
                      const float* queries, const uint32_t* qidx, int64_t nq, int metric,
                      const BoundCoef& bc, uint64_t* cand, hipStream_t s) {
    size_t shmem = sizeof(uint64_t) * 4 * (size_t)p.cap;
    hipLaunchKernelGGL(flat_scan_f4<NCH>, dim3(p.nblk, (unsigned)nq), dim3(256), shmem, s, rows,
                       norms, n, dim, queries, qidx, metric, bc, p.kc, p.cap, p.rows_per_block,
                       cand);
}

hipError_t launch_flat_scan(const FlatPlan& p, bool exact, const float* rows, const float* norms,
                            int64_t n, int dim, const float* queries, const uint32_t* qidx,
                            int64_t nq, int metric, uint64_t* cand, hipStream_t s) {
    int nch = exact ? 0 : flat_nch_for_dim(dim);
    BoundCoef bc = make_bounds(dim);
    switch (nch) {
    case 1: launch_f4<1>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, cand, s); break;
    case 2: launch_f4<2>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, cand, s); break;
    case 3: launch_f4<3>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, cand, s); break;
    case 4: launch_f4<4>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, cand, s); break;
    case 6: launch_f4<6>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, cand, s); break;
    case 8: launch_f4<8>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, cand, s); break;
    case 12: launch_f4<12>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, cand, s); break;
    case 16: launch_f4<16>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, cand, s); break;
    case 24: launch_f4<24>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, cand, s); break;
    case 32: launch_f4<32>(p, rows, norms, n, dim, queries, qidx, nq, metric, bc, cand, s); break;
    default: {
        size_t shmem = sizeof(uint64_t) * 4 * (size_t)p.cap + sizeof(float) * (size_t)dim;
        hipLaunchKernelGGL(flat_scan_rows, dim3(p.nblk, (unsigned)nq), dim3(256), shmem, s, rows,
                           norms, n, dim, queries, qidx, metric, p.kc, p.cap, p.rows_per_block,
                           cand);
    }
    }
    return hipGetLastError();
}

hipError_t launch_flat_merge(const FlatPlan& p, const float* rows, const float* norms, int64_t n,
                             int dim, const float* queries, const uint32_t* qidx, int64_t nq,
                             int metric, int k, int k_stride, const uint64_t* cand,
                             float* out_dist, uint32_t* out_ids, uint8_t* status, hipStream_t s) {
    size_t shmem = sizeof(uint64_t) * 4 * (size_t)p.cap;
    hipLaunchKernelGGL(flat_merge_rescore, dim3((unsigned)nq), dim3(256), shmem, s, cand, p.nblk,
                       p.kc, p.cap, rows, norms, n, dim, queries, qidx, metric, k, k_stride,
                       out_dist, out_ids, status);
    return hipGetLastError();
}

}  // namespace mans
