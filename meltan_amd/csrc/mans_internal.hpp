// Internal interfaces between the C ABI (mans_api.hip) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mans {

constexpr int kGroupBlocks = 32;  // blocks whose lists one group merge combines
// Threshold merge of the flat scan: used when kc <= kFastMaxKc and a query
// has at most kFastMaxBlocks block lists.
constexpr int kFastMaxKc = 64;
constexpr int kFastMaxBlocks = 8192;
constexpr int kFastListCap = 1024;  // lists whose head is <= the threshold, held in LDS
constexpr int kFastCandCap = 512;   // candidate slots the merge block sorts in LDS

struct FlatPlan {
    int kc = 0;              // candidates kept per wave, block, group and query
    int cap = 0;             // LDS slots per wave (power of two, >= kc + 64, >= 2 kc)
    int64_t rows_per_block = 0;
    int nblk = 0;            // blocks per query
    int group_blocks = kGroupBlocks;
    int ngroups = 0;         // groups per query
    bool fast = false;       // threshold merge (kc <= kFastMaxKc, nblk <= kFastMaxBlocks)
};

// Device buffers of one flat-scan launch.
struct FlatBuffers {
    uint64_t* cand = nullptr;      // nq * nblk * kc slots
    uint64_t* gcand = nullptr;     // nq * ngroups * kc slots
    uint32_t* counters = nullptr;  // nq * (ngroups + 1), zero before and after a launch
    uint64_t* heads = nullptr;     // nq * nblk (threshold merge)
    float* out_dist = nullptr;     // indexed by query id, k_stride per query
    uint32_t* out_ids = nullptr;
    uint8_t* status = nullptr;     // nq
};

// Batched path: fp32 MFMA contraction with fused selection, then one merge
// and rescore block per query.
constexpr int kGemmMaxKc = 64;        // k <= 32: the lane lists keep 4 or 8 slots each
constexpr int64_t kGemmMinRows = 4096;  // smaller corpora stay on the streaming scan
struct GemmPlan {
    int kc = 0;
    int cap = 0;   // LDS slots per wave in the merge
    int nseg = 0;  // row segments, a multiple of 8
    int nqb = 0;   // blocks of 128 queries
    int64_t rows_per_seg = 0;
    int lps = 2;   // lane lists per query and segment (4 on the split-bf16 path)
    // The split-bf16 path's bounding launch over sampled rows.
    int s_nseg = 0;
    int64_t s_rows_per_seg = 0;
    int64_t s_seg_rows = 0;
};
// False when the batch, dimension or kc does not suit the batched path.
bool plan_gemm(int64_t n, int dim, int64_t nq, int kc, GemmPlan* out);
size_t gemm_lists_bytes(const GemmPlan& p, int64_t nq);
// The contraction with the fused selection: writes the lane lists
// (gemm_lists_bytes of workspace).
hipError_t launch_flat_gemm(const GemmPlan& p, const float* rows, const float* norms, int64_t n,
                            int dim, const float* queries, int64_t nq, int metric,
                            uint64_t* lists, hipStream_t s);
// The per-query merge, exact rescore and proof: writes the k results and the
// proof status of every query (as launch_flat_search).  qbound (nullable):
// per-query bounds of the split-bf16 path; qbad (nullable): queries whose
// keys are not valid (status 1).
hipError_t launch_flat_gemm_merge(const GemmPlan& p, const float* rows, const float* norms,
                                  int64_t n, int dim, const float* queries, int64_t nq, int metric,
                                  const uint64_t* lists, const uint64_t* qbound,
                                  const uint32_t* qbad, const FlatBuffers& b, int k, int k_stride,
                                  hipStream_t s);

// Split-bf16 contraction (fp32-level accuracy on bf16 MFMA).
// Splits `count` queries of dim floats into [8 hi | 8 lo] bf16 parts per 8
// elements; bad[query] is or-ed with 1 for a value outside [2^-50, 2^50]
// (other than 0).
hipError_t launch_split_queries(const float* src, int64_t count, int dim, uint32_t* dst,
                                uint32_t* bad, hipStream_t s);
// Rows: hi gets the bf16 high parts ([count][dim]), recs the per-row key
// records ([2][count] float4s: cosine, then L2 and inner product) from the
// rows and their squared norms; bad[0] is or-ed with 1 for a value outside
// the range.
hipError_t launch_split_rows(const float* src, const float* norms, int64_t count, int dim,
                             uint16_t* hi, float* recs, uint32_t* bad, hipStream_t s);
// sampled: the bounding launch (no bounds, sorted lane lists); otherwise the
// full launch with the per-query bounds qbound (candidate buffers; a query
// whose buffer fills up gets bit 2 in qflag).
hipError_t launch_flat_bf2(const GemmPlan& p, bool sampled, const uint16_t* hi_rows,
                           const float* recs, int64_t n, int dim, const uint32_t* split_q,
                           const float* queries, int64_t nq, int metric, const uint64_t* qbound,
                           uint64_t* lists, uint32_t* qflag, hipStream_t s);
// bound[q]: from the sampled lists of query q, a slot whose key is the
// largest exact distance among the k rows with the smallest keys.
hipError_t launch_bf2_bounds(const GemmPlan& p, int64_t nq, int k, const uint64_t* lists,
                             const float* rows, const float* norms, int dim, const float* queries,
                             int metric, uint64_t* bound, hipStream_t s);

// target_blocks: blocks over all queries of a launch (0: the flat scan's default).
FlatPlan plan_flat(int64_t n, int64_t nq, int kc, int64_t target_blocks = 0);
int flat_nch_for_dim(int dim);
int flat_cap_for(int kc);

hipError_t launch_row_norms(const float* rows, int64_t n, int dim, float* out, hipStream_t s);

// One launch: scan, merges, exact rescore, results and proof status.
// exact == true forces the row-wise kernel whose keys are exact distances.
hipError_t launch_flat_search(const FlatPlan& p, bool exact, const float* rows, const float* norms,
                              int64_t n, int dim, const float* queries, const uint32_t* qidx,
                              int64_t nq, int metric, const FlatBuffers& b, int k, int k_stride,
                              hipStream_t s);

}  // namespace mans
