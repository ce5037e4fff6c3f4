// Internal interfaces between the C ABI (mans_api.hip) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mans {

struct FlatPlan {
    int kc = 0;              // candidates kept per block and per query
    int cap = 0;             // LDS slots per wave (power of two, >= kc + 64, >= 2 kc)
    int64_t rows_per_block = 0;
    int nblk = 0;
};

FlatPlan plan_flat(int64_t n, int64_t nq, int kc);
int flat_nch_for_dim(int dim);
int flat_cap_for(int kc);

hipError_t launch_row_norms(const float* rows, int64_t n, int dim, float* out, hipStream_t s);

// exact == true forces the row-wise kernel whose keys are exact distances.
hipError_t launch_flat_scan(const FlatPlan& p, bool exact, const float* rows, const float* norms,
                            int64_t n, int dim, const float* queries, const uint32_t* qidx,
                            int64_t nq, int metric, uint64_t* cand, hipStream_t s);

hipError_t launch_flat_merge(const FlatPlan& p, const float* rows, const float* norms, int64_t n,
                             int dim, const float* queries, const uint32_t* qidx, int64_t nq,
                             int metric, int k, int k_stride, const uint64_t* cand,
                             float* out_dist, uint32_t* out_ids, uint8_t* status, hipStream_t s);

}  // namespace mans
