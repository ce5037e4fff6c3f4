// Host-side runtime objects behind the C ABI handles.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "mans_hip.h"
#include "mans_internal.hpp"

namespace mans {

int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

// Output rows are k slots apart and the kernels index them with a 32-bit
// stride, so every search entry point rejects a larger k.
constexpr int64_t kMaxOutputK = 0x7FFFFFFF;
inline int check_k(int64_t k) {
    return k > kMaxOutputK ? fail(MANS_SEARCH_FAILED, "k above 2^31 - 1 is not supported") : 0;
}

struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    hipError_t ensure(size_t need, bool inject_fail);
    void release();
    ~DevBuf() { release(); }
};

struct PinnedBuf {
    void* p = nullptr;
    size_t bytes = 0;
    hipError_t ensure(size_t need);
    void release();
    ~PinnedBuf() { release(); }
};

// One pooled stream with its workspace.
struct Slot {
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    DevBuf queries, qidx, cand, gcand, counters, dist, ids, status;
    DevBuf heads;                 // block heads of the flat scan's threshold merge
    bool counters_dirty = false;  // a launch failed: re-zero the merge counters
    DevBuf aux0, aux1, aux2, aux3;
    DevBuf qsplit, qbad;          // split-bf16 queries and their range flags
    DevBuf bounds;                // per-query bounds of the int8 streaming scan
    PinnedBuf status_h, stage_h, result_h;  // pinned status, query staging, results
    ~Slot();
};

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int d) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        (void)hipSetDevice(d);
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

}  // namespace mans

struct mans_ctx {
    int device = 0;
    int num_cus = 256;
    bool fail_alloc = false;   // MANS_HIP_FAIL=alloc: every workspace allocation fails
    bool fail_launch = false;  // MANS_HIP_FAIL=launch: every search reports a failed launch
    std::mutex mu;
    std::vector<mans::Slot*> free_slots;
    std::vector<mans::Slot*> all_slots;
    std::atomic<bool> timing{false};
    std::atomic<int64_t> proof_retries{0};
    std::atomic<int64_t> reselects{0};  // batched int8 queries selected again by the streaming scan
    std::mutex tmu;
    std::map<std::string, std::pair<double, int64_t>> times;

    mans::Slot* acquire();
    void release(mans::Slot* s);
    void time_begin(mans::Slot* s, hipStream_t st);
    void time_end(mans::Slot* s, hipStream_t st, const char* name);
};

struct mans_corpus {
    mans_ctx* ctx = nullptr;
    int64_t n = 0;
    int64_t dim = 0;
    mans::DevBuf rows;   // n x dim f32, row-major
    mans::DevBuf norms;  // n f32, squared norms in the dots.c order
    std::mutex mu;
    // int8 planes (Int8CodeCache.swift:22-108), built on first use.
    bool int8_valid = false;
    mans::DevBuf i8_codes, i8_u, i8_w, i8_normsq, i8_invsqrt;
    // The rows' bf16 high parts ([n][dim]) and key records ([2][n] float4s)
    // for the batched split-bf16 contraction, built on first use; bf_ok:
    // every value is in the split range.
    bool bf_valid = false;
    bool bf_ok = false;
    mans::DevBuf bf_hi, bf_rec, bf_flag;
};

namespace mans {

struct SlotLease {
    mans_ctx* ctx;
    Slot* slot;
    explicit SlotLease(mans_ctx* c) : ctx(c), slot(c->acquire()) {}
    ~SlotLease() {
        if (slot) ctx->release(slot);
    }
};

hipError_t fill_empty(float* dist, uint32_t* ids, int64_t count, hipStream_t s);
hipError_t prepare_flat_buffers(mans_ctx* ctx, Slot* slot, const FlatPlan& p, int64_t nq,
                                hipStream_t st, FlatBuffers* out);
hipError_t stage_to_device(Slot* s, void* dst, const void* src, size_t bytes);
hipError_t stage_from_device(Slot* s, void* dst0, const void* src0, size_t b0, void* dst1,
                             const void* src1, size_t b1);
// h_dist/h_ids (nullable, pinned) receive the results with the same
// synchronisation that reads the proof status.
int flat_search_run(mans_ctx* ctx, const mans_corpus* c, const float* d_q, int64_t nq, int64_t k,
                    uint32_t metric, float* d_dist, uint32_t* d_ids, hipStream_t st, Slot* slot,
                    float* h_dist, uint32_t* h_ids);
hipError_t int8_refresh_rows(mans_corpus* c, int64_t first_row, int64_t count, hipStream_t s);
// Takes the no-allocation scratch array's device address on `device`
// (current); called once per device when a context is created.
int noalloc_init(int device);

}  // namespace mans
