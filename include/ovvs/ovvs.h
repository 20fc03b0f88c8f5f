/* libovvs — MI355X (gfx950) implementation of the ovVS IVF-PQ search path.
 *
 * This header declares the subset of the reference C ABI that reaches IVF-PQ
 * (reference include/ovvs/ovvs.h:11-121,165-214,276-286,406) with identical enum
 * values, struct layouts, symbol names and signatures, so the reference's C,
 * C++ (ovvs.hpp) and Python ctypes callers bind to libovvs.so unchanged.
 * Every computation behind these entry points runs on the GPU; there is no CPU
 * route. Entry points marked ADDITIVE have no reference counterpart.
 *
 * Pointers are host memory unless the entry point says "device". */
#pragma once

#include "export.h"
#include "status.h"
#include "version.h"

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference include/ovvs/ovvs.h:13-19 */
typedef enum ovvsDevice {
  OVVS_DEVICE_AUTO = 0,
  OVVS_DEVICE_CPU = 1,
  OVVS_DEVICE_NPU = 2,
  OVVS_DEVICE_GPU = 3,
  OVVS_DEVICE_HETERO = 4
} ovvsDevice;

/* reference include/ovvs/ovvs.h:21-29. Every non-forced policy and FORCE_GPU run
 * on the GPU. FORCE_CPU and FORCE_NPU name devices this library does not drive
 * and make compute entry points return OVVS_STATUS_DEVICE_UNAVAILABLE. */
typedef enum ovvsPolicy {
  OVVS_POLICY_AUTO = 0,
  OVVS_POLICY_NPU_IF_FASTER = 1,
  OVVS_POLICY_GPU_IF_FASTER = 2,
  OVVS_POLICY_HETERO = 3,
  OVVS_POLICY_FORCE_NPU = 4,
  OVVS_POLICY_FORCE_GPU = 5,
  OVVS_POLICY_FORCE_CPU = 6
} ovvsPolicy;

/* reference include/ovvs/ovvs.h:31-38. The metric only changes the exact
 * re-rank; the coarse probe and the lookup tables are always L2. */
typedef enum ovvsMetric {
  OVVS_METRIC_L2_EXPANDED = 0,
  OVVS_METRIC_L2_SQRT_EXPANDED = 1,
  OVVS_METRIC_INNER_PRODUCT = 2,
  OVVS_METRIC_COSINE_EXPANDED = 3,
  OVVS_METRIC_BITWISE_HAMMING = 4,
  OVVS_METRIC_LP_UNEXPANDED = 5
} ovvsMetric;

/* reference include/ovvs/ovvs.h:40-48 */
typedef enum ovvsDType {
  OVVS_DTYPE_F32 = 0,
  OVVS_DTYPE_F16 = 1,
  OVVS_DTYPE_I8 = 2,
  OVVS_DTYPE_U8 = 3,
  OVVS_DTYPE_F8E4M3 = 4,
  OVVS_DTYPE_F8E5M2 = 5,
  OVVS_DTYPE_F4E2M1 = 6
} ovvsDType;

/* Opaque handles (reference include/ovvs/ovvs.h:77,80). */
typedef struct ovvsResourcesImpl* ovvsResources_t;
typedef struct ovvsIvfPqIndexImpl* ovvsIvfPqIndex_t;
/* reference include/ovvs/ovvs.h:77 */
typedef struct ovvsScannIndexImpl* ovvsScannIndex_t;

#define OVVS_IVF_PQ_SEARCH_STATS_ABI_V1 1u

/* Cumulative telemetry of successful IVF-PQ searches on one Resources object.
 * Frozen 200-byte layout (reference include/ovvs/ovvs.h:89-121); counters
 * saturate at INT64_MAX. Stage times come from HIP events on the Resources
 * stream: coarse_pairwise_ns is the coarse distance kernel, coarse_topk_ns the
 * probe selection (with the ordering of the queries for the scan),
 * adc_scan_select_ns the fused LUT-build + code-scan +
 * shortlist kernel (lut_build_ns stays 0 because the LUT is built inside that
 * kernel), refine_distance_ns the fused gather + exact distance + final select
 * kernel. candidate_rows counts every (query, probed list) row scanned, so
 * candidate_rows * pq_m is the algorithmic code-byte volume. */
typedef struct ovvsIvfPqSearchStatsV1 {
  uint32_t abi_version;
  uint32_t struct_size;
  int64_t successful_calls;
  int64_t blocks;
  int64_t queries;
  int64_t tasks;
  int64_t candidate_rows;
  int64_t selected_rows;
  int64_t total_wall_ns;
  int64_t coarse_pairwise_ns;
  int64_t coarse_topk_ns;
  int64_t planning_ns;
  int64_t lut_build_ns;
  int64_t adc_scan_select_ns;
  int64_t shortlist_select_validate_ns;
  int64_t refine_gather_ns;
  int64_t refine_distance_ns;
  int64_t refine_topk_ns;
  int64_t gpu_allocation_calls;
  int64_t gpu_allocation_bytes;
  int64_t gpu_h2d_calls;
  int64_t gpu_h2d_bytes;
  int64_t gpu_d2h_calls;
  int64_t gpu_d2h_bytes;
  int64_t gpu_kernel_launches;
  int64_t gpu_wait_calls;
} ovvsIvfPqSearchStatsV1;

/* Concurrency (reference include/ovvs/ovvs.h:165-166): concurrent searches may
 * share one immutable index when each thread uses its own Resources. Each
 * Resources owns one HIP stream and one device workspace. Do not mutate,
 * serialize or destroy an index while it is being searched. */

/* reference include/ovvs/ovvs.h:171-172 */
OVVS_API const char* ovvsGetVersion(void);
OVVS_API const char* ovvsStatusString(ovvsStatus status);

/* reference include/ovvs/ovvs.h:174-184,210-211. Creating Resources does not
 * touch the GPU; the device is opened on first use. */
OVVS_API ovvsStatus ovvsResourcesCreate(ovvsResources_t* res);
OVVS_API ovvsStatus ovvsResourcesDestroy(ovvsResources_t res);
OVVS_API ovvsStatus ovvsResourcesSetPolicy(ovvsResources_t res, ovvsPolicy policy);
OVVS_API ovvsStatus ovvsResourcesGetPolicy(ovvsResources_t res, ovvsPolicy* policy);
OVVS_API ovvsStatus ovvsResourcesNpuAvailable(ovvsResources_t res, int32_t* available);
OVVS_API ovvsStatus ovvsResourcesGpuAvailable(ovvsResources_t res, int32_t* available);
OVVS_API ovvsStatus ovvsResourcesSku(ovvsResources_t res, char* buf, int32_t len);
OVVS_API ovvsStatus ovvsResourcesLastDevice(ovvsResources_t res, ovvsDevice* device);
OVVS_API ovvsStatus ovvsResourcesLastComputeDtype(ovvsResources_t res, ovvsDType* dtype);
OVVS_API ovvsStatus ovvsResourcesIvfPqSearchStatsV1(ovvsResources_t res,
                                                    ovvsIvfPqSearchStatsV1* stats);

/* ADDITIVE (no reference counterpart: the reference has one scan). The number of
 * queries, over all IVF-PQ searches on res, whose lower bounds pruned too little
 * and that the bounded scan therefore handed off to the full-table scan (data
 * without cluster structure). Telemetry only: results do not depend on it. */
OVVS_API ovvsStatus ovvsResourcesIvfPqTableQueries(ovvsResources_t res, int64_t* count);

/* IVF-PQ (reference include/ovvs/ovvs.h:276-286). */
OVVS_API ovvsStatus ovvsIvfPqBuild(ovvsResources_t res, const float* dataset, int64_t n,
                                   int64_t dim, ovvsMetric metric, int32_t nlist, int32_t pq_m,
                                   int32_t pq_nbits, ovvsIvfPqIndex_t* index);
OVVS_API ovvsStatus ovvsIvfPqSearch(ovvsResources_t res, ovvsIvfPqIndex_t index,
                                    const float* queries, int64_t nq, int64_t k, int32_t nprobe,
                                    int32_t krefine, const uint8_t* bitset, int64_t* neighbors,
                                    float* distances);
OVVS_API ovvsStatus ovvsIvfPqSerialize(ovvsIvfPqIndex_t index, const char* path);
OVVS_API ovvsStatus ovvsIvfPqDeserialize(ovvsResources_t res, const char* path,
                                         ovvsIvfPqIndex_t* index);
OVVS_API ovvsStatus ovvsIvfPqExtend(ovvsResources_t res, ovvsIvfPqIndex_t index,
                                    const float* extra, int64_t nextra);
OVVS_API ovvsStatus ovvsIvfPqDestroy(ovvsIvfPqIndex_t index);

/* ADDITIVE (no reference counterpart; the reference builds fp32 tables only).
 * ovvsIvfPqSearch with a requested lookup-table precision: lut_dtype is
 * OVVS_DTYPE_F32 or OVVS_DTYPE_F16; any other dtype returns
 * OVVS_STATUS_UNSUPPORTED. The scan computes each table entry in registers where
 * a row uses it and stores no table, so binary16 entries would save neither
 * memory traffic nor storage; both precisions are served with fp32 entries and
 * return exactly the results of ovvsIvfPqSearch (no entry can overflow a
 * binary16 range, and ovvsResourcesLastComputeDtype reports OVVS_DTYPE_F32). */
OVVS_API ovvsStatus ovvsIvfPqSearchEx(ovvsResources_t res, ovvsIvfPqIndex_t index,
                                      const float* queries, int64_t nq, int64_t k,
                                      int32_t nprobe, int32_t krefine, const uint8_t* bitset,
                                      ovvsDType lut_dtype, int64_t* neighbors,
                                      float* distances);

/* ADDITIVE (no reference counterpart). Same search with every buffer already
 * in device memory of the current HIP device: queries [nq*dim] f32, bitset
 * ((n+7)/8 bytes, may be NULL), neighbors [nq*k] i64, distances [nq*k] f32.
 * Returns after the results are complete. For callers that keep queries and
 * results resident in HBM (no PCIe copies on the search path). The results are
 * written in place by the search's last kernel: argument, limit and device
 * errors leave neighbors and distances untouched, but OVVS_STATUS_ERROR from the
 * search's own consistency checks (read after that kernel) may leave them
 * written. */
OVVS_API ovvsStatus ovvsIvfPqSearchDevice(ovvsResources_t res, ovvsIvfPqIndex_t index,
                                          const float* queries, int64_t nq, int64_t k,
                                          int32_t nprobe, int32_t krefine,
                                          const uint8_t* bitset, ovvsDType lut_dtype,
                                          int64_t* neighbors, float* distances);

/* ADDITIVE — no counterpart in the reference. For callers that cannot allocate
 * memory on the search path (code that must not call hipMalloc/hipFree or
 * allocate pinned host memory: tight serving loops, harnesses that forbid
 * allocation). Same arguments, semantics and results as ovvsIvfPqSearchDevice,
 * but no device or host memory is allocated: the search's workspace is carved
 * from a fixed device array of OVVS_NOALLOC_SCRATCH_BYTES that every GPU the
 * library runs on holds until the process ends.
 *   - The index must already have its device copy on this GPU: the first search
 *     of an index through ovvsIvfPqSearch, ovvsIvfPqSearchEx or
 *     ovvsIvfPqSearchDevice makes it (ovvsIvfPqExtend drops it again). Without it
 *     the call returns OVVS_STATUS_INVALID_ARGUMENT.
 *   - A batch whose workspace exceeds the array returns OVVS_STATUS_SHAPE_MISMATCH
 *     with the outputs untouched. The workspace is about
 *     nq * (40 + 4 * nprobe + 12 * max(k, krefine)) bytes plus one row of
 *     4 * nlist bytes of coarse scores (C2's 10,000-query batch: 4.2 MB).
 *   - Calls on one GPU share its array and run one at a time (the library
 *     serializes them); the array keeps the last call's contents and the search
 *     clears what it needs itself.
 *   - The first call on a Resources opens its HIP stream, as any entry point
 *     does. */
#define OVVS_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
OVVS_API ovvsStatus ovvsIvfPqSearchDeviceNoAlloc(ovvsResources_t res, ovvsIvfPqIndex_t index,
                                                 const float* queries, int64_t nq, int64_t k,
                                                 int32_t nprobe, int32_t krefine,
                                                 const uint8_t* bitset, ovvsDType lut_dtype,
                                                 int64_t* neighbors, float* distances);

/* ADDITIVE (the reference computes this inside its CAGRA build: the IVF-PQ
 * initializer, reference src/neighbors/graphs.cpp:767-797, with no entry point of its
 * own). The k-nearest-neighbour graph of the rows by IVF-PQ: an index is built with
 * ovvsIvfPqBuild(nlist = max(2, min(8, n/4)), pq_m = the largest divisor of dim not
 * above 4, 8-bit codes), every row is searched with k = krefine = degree + 1 and every
 * list probed, and graph[i * degree ...] (int32, caller-allocated, n * degree) holds
 * row i's results other than i itself and -1, in rank order, padded with -1. The rows'
 * searches run as batches (each batch is one IVF-PQ search in the telemetry); the
 * index is destroyed before returning. degree < 0 is INVALID_ARGUMENT, degree >= 1024
 * DEVICE_UNAVAILABLE (the search's shortlist limit); the build's statuses pass through.
 * graph is untouched on failure. */
OVVS_API ovvsStatus ovvsIvfPqKnnGraph(ovvsResources_t res, const float* dataset, int64_t n,
                                      int64_t dim, ovvsMetric metric, int32_t degree,
                                      int32_t* graph);

/* ScaNN-style index: IVF-PQ trained on column-scaled rows, re-ranked in the
 * original space (reference include/ovvs/ovvs.h:393-399,
 * src/neighbors/graphs.cpp:3286-3385).
 *
 * Build: aniso[d] = sqrt(var_d + 1e-6) per column (population variance from
 * left-to-right fp32 sums), computed on the GPU; the index keeps the rows and an
 * IVF-PQ index built by ovvsIvfPqBuild (8-bit codes) on the rows scaled by
 * aniso. On failure the build returns the inner build's status and leaves
 * *index unchanged, as the reference does.
 *
 * Search: krefine := max(krefine, (int32)k); the queries scaled by aniso are
 * searched with ovvsIvfPqSearch semantics for krefine results (k = krefine),
 * which counts in the IVF-PQ telemetry as one search; the returned ids are
 * re-ranked by the index metric on the original rows and queries, the first
 * min(k, candidates) by (distance, result rank) are written, inner-product
 * distances as +ip, the rest padded with (-1, +inf). k <= 0 writes nothing and
 * succeeds when the inner search does. Every step runs on the GPU. */
OVVS_API ovvsStatus ovvsScannBuild(ovvsResources_t res, const float* dataset, int64_t n,
                                   int64_t dim, ovvsMetric metric, int32_t nlist, int32_t pq_m,
                                   ovvsScannIndex_t* index);
OVVS_API ovvsStatus ovvsScannSearch(ovvsResources_t res, ovvsScannIndex_t index,
                                    const float* queries, int64_t nq, int64_t k, int32_t nprobe,
                                    int32_t krefine, int64_t* neighbors, float* distances);
OVVS_API ovvsStatus ovvsScannDestroy(ovvsScannIndex_t index);

/* Entry points of algorithms outside the IVF-PQ path (reference
 * include/ovvs/ovvs.h:218-242,252-300,311-391,409-415,460-465). They are exported
 * with the reference's names and signatures so that the reference's own callers
 * (its Python package binds all of these when it loads the library) can load
 * libovvs.so and use its IVF-PQ and ScaNN entry points. Each returns
 * OVVS_STATUS_UNSUPPORTED and writes nothing (a Destroy given NULL returns
 * OVVS_STATUS_SUCCESS; ovvsSyclEnabled returns 0). */
typedef struct ovvsBruteForceIndexImpl* ovvsBruteForceIndex_t;
typedef struct ovvsIvfFlatIndexImpl* ovvsIvfFlatIndex_t;
typedef struct ovvsIvfRabitqIndexImpl* ovvsIvfRabitqIndex_t;
typedef struct ovvsCagraIndexImpl* ovvsCagraIndex_t;
typedef struct ovvsVamanaIndexImpl* ovvsVamanaIndex_t;
typedef struct ovvsHnswIndexImpl* ovvsHnswIndex_t;
typedef struct ovvsKMeansModelImpl* ovvsKMeansModel_t;
typedef struct ovvsBatcherImpl* ovvsBatcher_t;
OVVS_API int32_t ovvsSyclEnabled(void);
OVVS_API ovvsStatus ovvsResourcesEnergyUj(ovvsResources_t res, int64_t* uj);
OVVS_API ovvsStatus ovvsGemm(ovvsResources_t res, const float* a, const float* b, float* c,
                             int64_t m, int64_t n, int64_t k, int32_t trans_b);
OVVS_API ovvsStatus ovvsGemmEx(ovvsResources_t res, const float* a, const float* b, float* c,
                               int64_t m, int64_t n, int64_t k, int32_t trans_b,
                               ovvsDType compute);
OVVS_API ovvsStatus ovvsTopk(ovvsResources_t res, const float* scores, int64_t rows,
                             int64_t cols, int64_t k, int64_t* indices, float* values,
                             int32_t largest);
OVVS_API ovvsStatus ovvsGatherRows(ovvsResources_t res, const float* src, int64_t src_rows,
                                   int64_t dim, const int64_t* idx, int64_t nidx, float* out);
OVVS_API ovvsStatus ovvsBruteForceBuild(ovvsResources_t res, const float* dataset, int64_t n,
                                        int64_t dim, ovvsMetric metric,
                                        ovvsBruteForceIndex_t* index);
OVVS_API ovvsStatus ovvsBruteForceSearch(ovvsResources_t res, ovvsBruteForceIndex_t index,
                                         const float* queries, int64_t nq, int64_t k,
                                         const uint8_t* bitset, int64_t* neighbors,
                                         float* distances);
OVVS_API ovvsStatus ovvsBruteForceDestroy(ovvsBruteForceIndex_t index);
OVVS_API ovvsStatus ovvsIvfFlatBuild(ovvsResources_t res, const float* dataset, int64_t n,
                                     int64_t dim, ovvsMetric metric, int32_t nlist,
                                     ovvsIvfFlatIndex_t* index);
OVVS_API ovvsStatus ovvsIvfFlatSearch(ovvsResources_t res, ovvsIvfFlatIndex_t index,
                                      const float* queries, int64_t nq, int64_t k,
                                      int32_t nprobe, const uint8_t* bitset,
                                      int64_t* neighbors, float* distances);
OVVS_API ovvsStatus ovvsIvfFlatDestroy(ovvsIvfFlatIndex_t index);
OVVS_API ovvsStatus ovvsIvfRabitqBuild(ovvsResources_t res, const float* dataset, int64_t n,
                                       int64_t dim, ovvsMetric metric, int32_t nlist,
                                       ovvsIvfRabitqIndex_t* index);
OVVS_API ovvsStatus ovvsIvfRabitqSearch(ovvsResources_t res, ovvsIvfRabitqIndex_t index,
                                        const float* queries, int64_t nq, int64_t k,
                                        int32_t nprobe, int32_t krefine, const uint8_t* bitset,
                                        int64_t* neighbors, float* distances);
OVVS_API ovvsStatus ovvsIvfRabitqSerialize(ovvsIvfRabitqIndex_t index, const char* path);
OVVS_API ovvsStatus ovvsIvfRabitqDeserialize(ovvsResources_t res, const char* path,
                                             ovvsIvfRabitqIndex_t* index);
OVVS_API ovvsStatus ovvsIvfRabitqExtend(ovvsResources_t res, ovvsIvfRabitqIndex_t index,
                                        const float* extra, int64_t nextra);
OVVS_API ovvsStatus ovvsIvfRabitqDestroy(ovvsIvfRabitqIndex_t index);
OVVS_API ovvsStatus ovvsCagraBuild(ovvsResources_t res, const float* dataset, int64_t n,
                                   int64_t dim, ovvsMetric metric, int32_t graph_degree,
                                   int32_t intermediate_degree, ovvsCagraIndex_t* index);
OVVS_API ovvsStatus ovvsCagraSearch(ovvsResources_t res, ovvsCagraIndex_t index,
                                    const float* queries, int64_t nq, int64_t k,
                                    int32_t itopk_size, int32_t search_width,
                                    const uint8_t* bitset, int64_t* neighbors, float* distances);
OVVS_API ovvsStatus ovvsCagraExtend(ovvsResources_t res, ovvsCagraIndex_t index,
                                    const float* extra, int64_t nextra);
OVVS_API ovvsStatus ovvsCagraDestroy(ovvsCagraIndex_t index);
OVVS_API ovvsStatus ovvsHnswFromCagra(ovvsResources_t res, ovvsCagraIndex_t cagra,
                                      ovvsHnswIndex_t* index);
OVVS_API ovvsStatus ovvsHnswSearch(ovvsResources_t res, ovvsHnswIndex_t index,
                                   const float* queries, int64_t nq, int64_t k, int32_t ef,
                                   int64_t* neighbors, float* distances);
OVVS_API ovvsStatus ovvsHnswSerialize(ovvsHnswIndex_t index, const char* path);
OVVS_API ovvsStatus ovvsHnswDeserialize(ovvsResources_t res, const char* path,
                                        ovvsHnswIndex_t* index);
OVVS_API ovvsStatus ovvsHnswDestroy(ovvsHnswIndex_t index);
OVVS_API ovvsStatus ovvsVamanaBuild(ovvsResources_t res, const float* dataset, int64_t n,
                                    int64_t dim, ovvsMetric metric, int32_t graph_degree,
                                    float alpha, ovvsVamanaIndex_t* index);
OVVS_API ovvsStatus ovvsVamanaSearch(ovvsResources_t res, ovvsVamanaIndex_t index,
                                     const float* queries, int64_t nq, int64_t k, int32_t beam,
                                     const uint8_t* bitset, int64_t* neighbors,
                                     float* distances);
OVVS_API ovvsStatus ovvsVamanaDestroy(ovvsVamanaIndex_t index);
OVVS_API ovvsStatus ovvsKMeansFit(ovvsResources_t res, const float* dataset, int64_t n,
                                  int64_t dim, int32_t nclusters, int32_t iters,
                                  ovvsKMeansModel_t* model);
OVVS_API ovvsStatus ovvsKMeansPredict(ovvsResources_t res, ovvsKMeansModel_t model,
                                      const float* x, int64_t n, int64_t* labels,
                                      float* distances);
OVVS_API ovvsStatus ovvsKMeansDestroy(ovvsKMeansModel_t model);
OVVS_API ovvsStatus ovvsBatcherCreate(ovvsResources_t res, ovvsBruteForceIndex_t index,
                                      int32_t max_batch, int32_t max_wait_ms,
                                      ovvsBatcher_t* out);
OVVS_API ovvsStatus ovvsBatcherSearch(ovvsBatcher_t batcher, const float* queries, int64_t nq,
                                      int64_t k, int64_t* neighbors, float* distances);
OVVS_API ovvsStatus ovvsBatcherDestroy(ovvsBatcher_t batcher);

/* Allow-list to an LSB-first bitset of (n+7)/8 bytes; ids outside [0,n) are
 * ignored (reference include/ovvs/ovvs.h:406, src/rt/resources.cpp:218-229). */
OVVS_API ovvsStatus ovvsBitsetFromAllowList(int64_t n, const int64_t* ids, int64_t nids,
                                            uint8_t* bitset);

#ifdef __cplusplus
}
#endif
