// The exact flat scan for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc): mans_flat_search_device_noalloc.  It has no counterpart in the
// reference.  Results are those of mans_flat_search_device's streaming scan
// (the same kernels, the same proof loop), with every workspace taken from
// `scratch`, a fixed array in device memory that each GPU holds until the
// process ends.
//
// `scratch` is a device symbol: in host code its name is only a stand-in, so
// the library takes its device address once per device, with that device
// current, when a context is created (noalloc_init), and passes that address
// to the kernels.  The entry point calls no hipMalloc, hipFree or allocating
// library routine, uses the caller's stream (NULL: the null stream), and
// clears what must start at zero with a fill kernel, not a memset.  Calls on
// one device share the array (it keeps the last call's contents); a
// per-device lock serialises them within the process.
#include <algorithm>
#include <mutex>
#include <string>

#include "mans_hip.h"
#include "mans_internal.hpp"
#include "mans_runtime.hpp"

namespace {

constexpr size_t kScratchBytes = (size_t)MANS_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
constexpr int64_t kQueryChunk = 1024;  // queries per round of the proof loop

__device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_init_mu;
void* g_scratch[kMaxDevices] = {};       // scratch's device address per device
std::mutex g_call_mu[kMaxDevices];       // one call at a time per device

__global__ void fill_u32_kernel(uint32_t* __restrict__ p, int64_t count, uint32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = v;
}

hipError_t fill_u32(void* p, int64_t count, uint32_t v, hipStream_t s) {
    if (count <= 0) return hipSuccess;
    hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s,
                       (uint32_t*)p, count, v);
    return hipGetLastError();
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// The scratch layout of one launch of m queries under plan p.
struct Layout {
    size_t qidx = 0, status = 0, counters = 0, heads = 0, cand = 0, gcand = 0, end = 0;
    int64_t counter_words = 0;
};

Layout layout_for(const mans::FlatPlan& p, int64_t m) {
    Layout l;
    size_t off = 0;
    l.qidx = off;
    off = align256(off + (size_t)m * sizeof(uint32_t));
    l.status = off;
    off = align256(off + (size_t)m);
    l.counter_words = m * (p.ngroups + 1);
    l.counters = off;
    off = align256(off + (size_t)l.counter_words * sizeof(uint32_t));
    l.heads = off;
    if (p.fast) off = align256(off + (size_t)m * p.nblk * sizeof(uint64_t));
    l.cand = off;
    off = align256(off + (size_t)m * p.nblk * p.kc * sizeof(uint64_t));
    l.gcand = off;
    off = align256(off + (size_t)m * p.ngroups * p.kc * sizeof(uint64_t));
    l.end = off;
    return l;
}

int pow2_ceil(int64_t x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

}  // namespace

namespace mans {

int noalloc_init(int device) {
    if (device < 0 || device >= kMaxDevices)
        return fail(MANS_DEVICE_NOT_SUPPORTED, "device index above the no-allocation table");
    std::lock_guard<std::mutex> g(g_init_mu);
    if (g_scratch[device]) return MANS_OK;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return hip_fail(e, "no-allocation scratch address");
    g_scratch[device] = ptr;
    return MANS_OK;
}

}  // namespace mans

using namespace mans;

extern "C" {

int mans_flat_search_device_noalloc(mans_ctx* ctx, const mans_corpus* c, const float* d_queries,
                                    int64_t nq, int64_t k, uint32_t metric, float* d_out_dist,
                                    uint32_t* d_out_ids, void* stream) {
    if (!ctx || !c) return fail(MANS_SEARCH_FAILED, "NULL context or corpus");
    if (check_k(k) != MANS_OK) return MANS_SEARCH_FAILED;
    if (metric > 2) return fail(MANS_SEARCH_FAILED, "flat scan does not support this metric");
    if (nq <= 0 || k <= 0) return MANS_OK;
    if (!d_queries || !d_out_dist || !d_out_ids) return fail(MANS_SEARCH_FAILED, "NULL buffer");
    if (nq > (int64_t)0xFFFFFFFFll)
        return fail(MANS_SEARCH_FAILED, "no-allocation flat scan: more than 2^32 - 1 queries");
    if (ctx->device < 0 || ctx->device >= kMaxDevices || !g_scratch[ctx->device])
        return fail(MANS_PIPELINE_UNAVAILABLE, "no-allocation scratch is not set up on this device");
    if (ctx->fail_launch) return fail(MANS_EXECUTION_FAILED, "injected launch failure");
    DeviceGuard dg(ctx->device);
    std::lock_guard<std::mutex> lock(g_call_mu[ctx->device]);
    uint8_t* base = (uint8_t*)g_scratch[ctx->device];
    hipStream_t st = (hipStream_t)stream;
    const int64_t n = c->n;
    const int dim = (int)c->dim;
    const int kstride = (int)k;
    hipError_t e = hipSuccess;
    if (n == 0) {
        e = fill_u32(d_out_dist, nq * k, 0x7F7FFFFFu, st);
        if (e == hipSuccess) e = fill_u32(d_out_ids, nq * k, MANS_EMPTY_ID, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        return e == hipSuccess ? MANS_OK : hip_fail(e, "no-allocation fill");
    }
    const int keff = (int)std::min<int64_t>(std::min<int64_t>(k, MANS_MAX_TOP_K), n);
    const bool unaligned = (reinterpret_cast<uintptr_t>(d_queries) & 15u) != 0;
    // Host bookkeeping lives on the stack: query indices of the current and
    // the next round, and the statuses read back.
    uint32_t cur[kQueryChunk], next[kQueryChunk];
    uint8_t status_h[kQueryChunk];
    for (int64_t q0 = 0; q0 < nq; q0 += kQueryChunk) {
        int64_t npend = std::min<int64_t>(kQueryChunk, nq - q0);
        for (int64_t i = 0; i < npend; ++i) cur[i] = (uint32_t)(q0 + i);
        bool exact = flat_nch_for_dim(dim) == 0 || unaligned;
        int kc = pow2_ceil(std::max(32, 2 * keff));
        for (;;) {
            if (exact) kc = pow2_ceil(std::max(32, keff));
            int64_t nnext = 0;
            for (int64_t s0 = 0; s0 < npend;) {
                // The largest run of pending queries whose workspace fits.
                int64_t m = npend - s0;
                FlatPlan p = plan_flat(n, m, kc);
                Layout l = layout_for(p, m);
                while (l.end > kScratchBytes && m > 1) {
                    m = (m + 1) / 2;
                    p = plan_flat(n, m, kc);
                    l = layout_for(p, m);
                }
                if (l.end > kScratchBytes)
                    return fail(MANS_RESOURCE_EXHAUSTED,
                                "no-allocation flat scan: one query needs " + std::to_string(l.end) +
                                    " bytes of workspace, above the " +
                                    std::to_string(kScratchBytes) + "-byte scratch");
                e = hipMemcpyAsync(base + l.qidx, cur + s0, (size_t)m * sizeof(uint32_t),
                                   hipMemcpyHostToDevice, st);
                if (e == hipSuccess) e = fill_u32(base + l.counters, l.counter_words, 0u, st);
                FlatBuffers fb;
                fb.cand = (uint64_t*)(base + l.cand);
                fb.gcand = (uint64_t*)(base + l.gcand);
                fb.counters = (uint32_t*)(base + l.counters);
                fb.heads = p.fast ? (uint64_t*)(base + l.heads) : nullptr;
                fb.out_dist = d_out_dist;
                fb.out_ids = d_out_ids;
                fb.status = base + l.status;
                if (e == hipSuccess)
                    e = launch_flat_search(p, exact, (const float*)c->rows.p, (const float*)c->norms.p,
                                           n, dim, d_queries, (const uint32_t*)(base + l.qidx), m,
                                           (int)metric, fb, keff, kstride, st);
                if (e == hipSuccess)
                    e = hipMemcpyAsync(status_h, base + l.status, (size_t)m, hipMemcpyDeviceToHost, st);
                if (e == hipSuccess) e = hipStreamSynchronize(st);
                if (e != hipSuccess) return hip_fail(e, "no-allocation flat scan");
                for (int64_t i = 0; i < m; ++i)
                    if (status_h[i]) next[nnext++] = cur[s0 + i];
                s0 += m;
            }
            if (nnext == 0) break;
            if (exact) return fail(MANS_SEARCH_FAILED, "exact round failed its own proof");
            for (int64_t i = 0; i < nnext; ++i) cur[i] = next[i];
            npend = nnext;
            kc *= 4;
            if (kc > 1024) exact = true;
        }
    }
    return MANS_OK;
}

}  // extern "C"
