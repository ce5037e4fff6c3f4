/*
 * mans_hip.h -- C ABI of the MI355X (gfx950) search hot path for MetalANNS.
 *
 * This header extends the reference's C target MetalANNSC
 * (Sources/MetalANNSC/include/MetalANNSC.h:13-38).  The three CPU functions
 * declared there (mans_f32_dot_rows, mans_i8_dot_rows_f32,
 * mans_f32_dot_rows_gather) stay in the reference's dots.c, unchanged: the
 * CPU tiers keep calling them.  Everything below replaces the Metal backend
 * of MetalANNSCore for the four scans of the exact-search path:
 *
 *   - fused exact flat scan (distance + top-k)
 *       replaces FlatGPUSearch.runChunk + flat_scan_distances + host top-k
 *       (FlatGPUSearch.swift:652-707, 786-977; Shaders/FlatSearch.metal:33-77)
 *   - int8 prefilter -> fp32 rerank, proof-checked
 *       replaces BoundedExactScan.search + Int8CodeBuffer
 *       (BoundedExactScan.swift:30-369; Int8CodeCache.swift:22-108)
 *   - IVF-flat probe scan
 *       replaces IVFFlatSearch.scanProbedLists + assignRows
 *       (IVFFlatSearch.swift:214-291, 633-703)
 *   - IVF-PQ ADC probe scan
 *       replaces _IVFPQIndex.search/add + GPUADCSearch.computeDistances
 *       (IVFPQIndex.swift:106-226; GPUADCSearch.swift:35-173;
 *        Shaders/PQDistance.metal:4-66)
 *
 * Conventions
 *   - Metric codes follow FlatGPUSearch.swift:134-140: cosine 0, l2 1,
 *     innerProduct 2, hamming 3 (hamming is rejected with MANS_SEARCH_FAILED,
 *     as FlatGPUSearch.swift:118-120 does).
 *   - Scores are distances, ascending (FlatSearch.metal:17-31 semantics with
 *     the host cosine denominator sqrt(qn*vn), ParallelFlatScan.swift:254).
 *   - Per query, k slots are written, sorted by (distance, id); slots past
 *     min(k, n) hold FLT_MAX / 0xFFFFFFFF (the reference's emptyID,
 *     FlatGPUSearch.swift:19).  k is capped at 256 (FlatGPUSearch.swift:13)
 *     for the flat and int8 scans.
 *   - Return codes map one to one onto ANNSError (Errors.swift:6-31).  The
 *     last four are tier-degradeable: a caller falls back to the next tier.
 *   - Host pointers are caller-owned and only read/written during the call.
 *     Calls block until results are on the host (or, for the _device
 *     variants, complete in device memory).
 *   - A mans_ctx may be used from many threads at once: each call takes a
 *     HIP stream and workspace from a pool (the analogue of
 *     CommandQueuePool.swift:27-31 and FlatWorkspacePool,
 *     FlatGPUSearch.swift:1070-1139).
 */
#ifndef MANS_HIP_H
#define MANS_HIP_H

#include <stdint.h>

#if defined(__cplusplus)
extern "C" {
#endif

#define MANS_OK 0
#define MANS_DEVICE_NOT_SUPPORTED (-1)  /* ANNSError.deviceNotSupported */
#define MANS_DIMENSION_MISMATCH (-2)    /* ANNSError.dimensionMismatch */
#define MANS_PIPELINE_UNAVAILABLE (-3)  /* ANNSError.gpuPipelineUnavailable (degradeable) */
#define MANS_RESOURCE_EXHAUSTED (-4)    /* ANNSError.gpuResourceExhausted (degradeable) */
#define MANS_EXECUTION_FAILED (-5)      /* ANNSError.gpuExecutionFailed (degradeable) */
#define MANS_SEARCH_FAILED (-6)         /* ANNSError.searchFailed (degradeable) */
#define MANS_CORRUPT_FILE (-7)          /* ANNSError.corruptFile */

#define MANS_METRIC_COSINE 0u
#define MANS_METRIC_L2 1u
#define MANS_METRIC_INNER_PRODUCT 2u
#define MANS_METRIC_HAMMING 3u

#define MANS_MAX_TOP_K 256
#define MANS_EMPTY_ID 0xFFFFFFFFu

typedef struct mans_ctx mans_ctx;       /* device, stream/workspace pool, timing */
typedef struct mans_corpus mans_corpus; /* device-resident f32 rows, norms, int8 planes */
typedef struct mans_ivf mans_ivf;       /* IVF-flat: centroids, CSR lists, packed rows */
typedef struct mans_ivfpq mans_ivfpq;   /* IVF-PQ: coarse centroids, codebooks, list codes */

/* Thread-local message for the last non-zero return on this thread. */
const char *mans_last_error(void);

/* Device context.  Replaces MetalContext (MetalDevice.swift:9-111).
 * Returns MANS_DEVICE_NOT_SUPPORTED when no gfx950 device is present. */
int mans_ctx_create(int device, mans_ctx **out);
void mans_ctx_destroy(mans_ctx *ctx);

/* Corpus upload.  The rows are the row-major f32 matrix that VectorBuffer
 * and the MANN v3 vector section hold (VectorBuffer.swift:12-111,
 * IndexSerializer.swift:74-140), copied once into HBM; squared row norms are
 * computed on the device in the scalar order of dots.c:40-47. */
int mans_corpus_upload_f32(mans_ctx *ctx, const float *rows, int64_t n, int64_t dim,
                           mans_corpus **out);
/* MANN v3 (mmap-compatible) index files, IndexSerializer.saveMmapCompatible
 * (IndexSerializer.swift:74-140) and MmapIndexLoader.load
 * (MmapIndexLoader.swift:38-196): a 28-byte little-endian header ("MANN",
 * version 3, node count, degree, dim, metric code, storage type), then the
 * vector, adjacency and distance sections each starting on a page boundary,
 * then the trailer (IDMap byte count, IDMap JSON, entry point).  The page
 * size is the writer's (getpagesize(); 16384 on Apple silicon): page_size 0
 * means this host's.
 *
 * mans_mann_inspect validates a file as MmapIndexLoader.load does (magic,
 * version, metric and storage codes, non-zero counts, section and trailer
 * bounds, an IDMap JSON payload that decodes with exactly node-count entries
 * (MmapIndexLoader.swift:174-182), entry point below the node count) and
 * fills `info`; MANS_CORRUPT_FILE with the reference's reason otherwise.
 * Needs no device. */
typedef struct mans_mann_info {
    uint32_t version, node_count, degree, dim, metric, storage_type, entry_point;
    int64_t page_size;
    int64_t vector_offset, vector_bytes, adjacency_offset, distance_offset, trailer_offset;
    int64_t idmap_bytes;
} mans_mann_info;
int mans_mann_inspect(const char *path, int64_t page_size, mans_mann_info *info);
/* The loadReadOnly(.mmap) path: maps the file read-only and uploads its
 * vector section straight from the mapping into a new corpus (through
 * pinned staging buffers, two copies in flight), then computes the norms.
 * fp32 storage only (FlatGPUSearch.isEligible, FlatGPUSearch.swift:193-209):
 * f16 and binary files give MANS_PIPELINE_UNAVAILABLE.  out_metric
 * (nullable) receives the file's metric code. */
int mans_corpus_upload_mann(mans_ctx *ctx, const char *path, int64_t page_size, mans_corpus **out,
                            uint32_t *out_metric);
/* In-place row writes: copies `count` rows starting at `first_row` and
 * refreshes every derived plane of those rows (norms, int8 codes), the
 * analogue of the VectorBuffer write hooks that invalidate the norm and code
 * caches (VectorBuffer.swift:44-51, 71-73, 87-89). */
int mans_corpus_write_rows(mans_corpus *corpus, int64_t first_row, const float *rows,
                           int64_t count);
/* Drops derived planes (int8 codes) so they are rebuilt on next use
 * (Int8CodeCache.invalidate, Int8CodeCache.swift:189-193). */
int mans_corpus_invalidate(mans_corpus *corpus);
void mans_corpus_release(mans_corpus *corpus);
int64_t mans_corpus_count(const mans_corpus *corpus);
int64_t mans_corpus_dim(const mans_corpus *corpus);

/* Exact flat scan: FlatGPUSearch.batchSearch (FlatGPUSearch.swift:103-181)
 * on the device.  queries: nq x dim host f32.  out_dist/out_ids: nq x k. */
int mans_flat_search(mans_ctx *ctx, const mans_corpus *corpus, const float *queries, int64_t nq,
                     int64_t k, uint32_t metric, float *out_dist, uint32_t *out_ids);

/* Same, with queries and outputs in device memory and work on `stream`
 * (a hipStream_t, or NULL for the pooled stream).  Blocks until done. */
int mans_flat_search_device(mans_ctx *ctx, const mans_corpus *corpus, const float *d_queries,
                            int64_t nq, int64_t k, uint32_t metric, float *d_out_dist,
                            uint32_t *d_out_ids, void *stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): mans_flat_search_device's results (its streaming scan
 * and proof loop) with every workspace taken from a fixed device array of
 * MANS_NOALLOC_SCRATCH_BYTES that each GPU holds until the process ends.
 * Calls no hipMalloc/hipFree or allocating library routine; work runs on
 * `stream` (NULL: the null stream) and the call blocks until done.  Queries
 * go through in rounds sized to the array; a corpus for which one query's
 * workspace does not fit gives MANS_RESOURCE_EXHAUSTED.  Calls on one GPU
 * share the array (it keeps the last call's contents) and are serialised by
 * a per-device lock. */
#define MANS_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
int mans_flat_search_device_noalloc(mans_ctx *ctx, const mans_corpus *corpus,
                                    const float *d_queries, int64_t nq, int64_t k, uint32_t metric,
                                    float *d_out_dist, uint32_t *d_out_ids, void *stream);

/* int8 prefilter + fp32 rerank: BoundedExactScan.search
 * (BoundedExactScan.swift:30-122).  mode 0: adaptive budget with the
 * reference's lower-bound proof (results are exact); mode 1: one round at
 * `budget` candidates, no proof (the fixed "prefilter top-B, rerank" form).
 * The int8 codes are built on the device on first use, bit-exact with
 * Int8CodeCache.swift:64-99.  out_rounds (nullable): per query, the number
 * of selection rounds used. */
int mans_int8_search(mans_ctx *ctx, mans_corpus *corpus, const float *queries, int64_t nq,
                     int64_t k, uint32_t metric, int32_t mode, int64_t budget, float *out_dist,
                     uint32_t *out_ids, int32_t *out_rounds);
int mans_int8_search_device(mans_ctx *ctx, mans_corpus *corpus, const float *d_queries,
                            int64_t nq, int64_t k, uint32_t metric, int32_t mode, int64_t budget,
                            float *d_out_dist, uint32_t *d_out_ids, void *stream);
/* Copies the int8 planes back (codes n*dim, then u, w, normSq, invSqrt, n
 * each) for bit-exact checks against Int8CodeCache.swift:64-99. */
int mans_int8_codes_download(mans_ctx *ctx, mans_corpus *corpus, int8_t *codes, float *u,
                             float *w, float *normsq, float *invsqrt);

/* IVF-flat build from given centroids: assignment on the device (argmin,
 * ties to the lower list, IVFFlatSearch.swift:633-703), CSR lists in row
 * order and rows packed list by list (IVFFlatSearch.swift:589-615). */
int mans_ivf_flat_build(mans_ctx *ctx, const mans_corpus *corpus, const float *centroids,
                        int64_t nlist, uint32_t metric, mans_ivf **out);
/* Lloyd k-means on the device, KMeans.cluster (KMeans.swift:53-257):
 * assignment by SIMDDistance.distance (SIMDDistance.swift:17-80) with strict
 * < (the first centroid wins ties); the loop stops when no assignment
 * changes; each centroid is its rows' float sum in row order times
 * 1/count (the single-worker order, KMeans.swift:208-250); empty clusters
 * keep their centroid.  The reference seeds k-means++ from Swift's stdlib
 * RNG, which is not reproduced: the initial centroids are rows 0, s, 2s, ...
 * with s = max(1, n / k). */
int mans_kmeans(mans_ctx *ctx, const mans_corpus *corpus, int64_t k, int64_t iters,
                uint32_t metric, float *out_centroids);
/* The centroids IVFFlatSearch.buildPartition trains
 * (IVFFlatSearch.swift:517-551): L = min(max(1, nlist), n) lists, a strided
 * sample of min(n, max(L, min(4096, 16 L))) rows, mans_kmeans on the sample
 * with 8 iterations and the index's metric.  Writes L x dim centroids
 * (out_centroids holds nlist x dim floats) and L to out_nlist. */
int mans_ivf_flat_train(mans_ctx *ctx, const mans_corpus *corpus, int64_t nlist, uint32_t metric,
                        float *out_centroids, int64_t *out_nlist);
/* IVFFlatSearch.search over a built partition (IVFFlatSearch.swift:115-137,
 * 214-291).  out_probes (nullable): nq x nprobe list ids, ascending. */
int mans_ivf_flat_search(mans_ctx *ctx, const mans_ivf *ivf, const float *queries, int64_t nq,
                         int64_t k, int64_t nprobe, float *out_dist, uint32_t *out_ids,
                         int32_t *out_probes);
int mans_ivf_flat_search_device(mans_ctx *ctx, const mans_ivf *ivf, const float *d_queries,
                                int64_t nq, int64_t k, int64_t nprobe, float *d_out_dist,
                                uint32_t *d_out_ids, void *stream);
/* Copies the CSR layout back: offsets (nlist+1, int64) and list ids (n). */
int mans_ivf_download_lists(const mans_ivf *ivf, int64_t *offsets, uint32_t *list_ids);
void mans_ivf_release(mans_ivf *ivf);

/* _IVFPQIndex.train (IVFPQIndex.swift:54-104) on the rows of `train`:
 * coarse k-means (nlist, iters, metric; mans_kmeans), each row's residual
 * against its centroid from the last assignment, then
 * ProductQuantizer.train (ProductQuantizer.swift:10-85): per subspace
 * k-means of the residual subvectors with 256 centroids, L2 and iters
 * iterations, same rules.  Needs n >= 256, n >= nlist and dim % m == 0.
 * out_coarse: nlist x dim; out_codebooks: m x 256 x dim/m. */
int mans_ivfpq_train(mans_ctx *ctx, const mans_corpus *train, int64_t nlist, int64_t m,
                     int64_t iters, uint32_t metric, float *out_coarse, float *out_codebooks);
/* IVF-PQ: coarse centroids (nlist x dim) and codebooks (M x 256 x dim/M)
 * are given (trained by the caller, IVFPQIndex.swift:54-104).  Adds every
 * corpus row: coarse assignment (IVFPQIndex.swift:514-550) and
 * encode(vector:subtracting:) (ProductQuantizer.swift:120-169) on the
 * device, bit-exact; lists hold ids in row order. */
int mans_ivfpq_build(mans_ctx *ctx, const mans_corpus *corpus, const float *coarse,
                     int64_t nlist, const float *codebooks, int64_t m, uint32_t metric,
                     mans_ivfpq **out);
/* _IVFPQIndex.search (IVFPQIndex.swift:177-226): probes by
 * selectClosestCentroids, per-probe residual LUT held in LDS, ADC, merge
 * with BoundedSortedList semantics (BoundedSelection.swift:158-214) into the
 * best `k_adc`.  If rerank_k > 0 the k_adc ADC results are re-ranked by the
 * exact fp32 distance on the corpus rows and rerank_k are returned (a step
 * with no counterpart in the reference); otherwise k_adc ADC scores. */
int mans_ivfpq_search(mans_ctx *ctx, const mans_ivfpq *pq, const float *queries, int64_t nq,
                      int64_t k_adc, int64_t nprobe, int64_t rerank_k, float *out_score,
                      uint32_t *out_ids);
int mans_ivfpq_search_device(mans_ctx *ctx, const mans_ivfpq *pq, const float *d_queries,
                             int64_t nq, int64_t k_adc, int64_t nprobe, int64_t rerank_k,
                             float *d_out_score, uint32_t *d_out_ids, void *stream);
/* Copies codes back in row order (n x M) plus coarse assignments (n). */
int mans_ivfpq_download_codes(const mans_ivfpq *pq, uint8_t *codes, int32_t *assign);
/* Binary persistence of a built index, in place of the JSON "IVFP" state of
 * _IVFPQIndex.save/load (IVFPQIndex.swift:252-324), which does not scale to
 * 10M codes: a 48-byte header ("IVPB", version 1, dim, metric, n, nlist, m,
 * dim/m), then the coarse centroids, codebooks, list offsets, list ids,
 * codes (list by list) and coarse assignments, little-endian.  Load
 * validates the file
 * (MANS_CORRUPT_FILE with a reason) and uploads it; `corpus` (nullable)
 * serves the exact rerank and must hold the same n x dim rows. */
int mans_ivfpq_save(const mans_ivfpq *pq, const char *path);
int mans_ivfpq_load(mans_ctx *ctx, const mans_corpus *corpus, const char *path, mans_ivfpq **out);
void mans_ivfpq_release(mans_ivfpq *pq);

/* Kernel timing with HIP events on the stream each kernel runs on.
 * enable != 0 starts accumulating; read returns the summed milliseconds and
 * launch count of the named kernel class ("flat_scan", "flat_gemm",
 * "flat_merge", "int8_scan", "ivf_scan", "ivfpq_scan") since the last
 * reset.  While enabled, each timed launch is waited for. */
int mans_timing_enable(mans_ctx *ctx, int enable);
int mans_timing_read(mans_ctx *ctx, const char *kernel, double *total_ms, int64_t *launches);
int mans_timing_reset(mans_ctx *ctx);

#if defined(__cplusplus)
}
#endif

#endif /* MANS_HIP_H */
