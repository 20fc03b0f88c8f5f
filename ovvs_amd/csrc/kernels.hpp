// kernels.hpp — the thin C ABI between libovvs's C++ host code and its gfx950
// HIP kernels. Every function enqueues work on `stream` and returns the launch
// status (hipSuccess == 0); none of them synchronizes or allocates. Shapes are
// validated by the host caller before launch; each launcher re-checks the
// limits its kernel relies on and returns hipErrorInvalidValue instead of
// launching when they do not hold.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// Largest shortlist (krefine) and final k the scan/refine kernels hold in
// registers: 64 keys per register row, up to 16 rows per wave.
#define OVVS_HIP_MAX_REFINE 1024
// Largest probe count the in-LDS probe selection sorts (32 KiB of 64-bit keys).
#define OVVS_HIP_MAX_PROBES 4096

// Device layout of the packed PQ codes. Rows keep the list-major order of the
// reference's packed CSR (packed position p); they are grouped in tiles of
// OVVS_CODE_TILE_ROWS rows, and inside a tile the codes of subspace block b
// (OVVS_CODE_BLOCK subspaces, one byte each, zero-padded past pq_m) of the
// tile's rows are contiguous:
//   offset(p, b) = (p / 64) * (nblocks * 64 * 8) + b * (64 * 8) + (p % 64) * 8.
#define OVVS_CODE_BLOCK 8
#define OVVS_CODE_TILE_ROWS 64

// Scan order of the device mirror: each list's rows are split into segments of
// at most OVVS_SEGMENT_ROWS rows with nearby PQ reconstructions; a segment
// starts at a code tile and carries the (lo, hi) range of its rows'
// reconstructions in every subspace dimension (its box). Rows keep their
// index within the list, which is what orders candidates.
#define OVVS_SEGMENT_ROWS 128
// Segments are grouped (maximal subtrees of the segmentation with at most this many
// segments), each group with the union of its segments' boxes.
#define OVVS_GROUP_SEGMENTS 4
// Boxes are used when pq_m * dsub is at most this (the scan's rounding-error
// allowance for its lower bounds holds up to there).
#define OVVS_MAX_BOX_DIMS 2048

// out[i] = sum_t x[i*dim+t]^2, left to right from +0 (reference internal.hpp:221-225).
hipError_t ovvs_hip_row_norms(const float* x, int64_t n, int32_t dim, float* out,
                              hipStream_t stream);

// Exact expanded-L2 coarse scores: S[q*ldS + c] = (qn[q] + cn[c]) - 2*dot(q, c),
// dot a left-to-right fp32 sum (reference mixer.cpp:177-198, cpu_prims.cpp:48-58).
hipError_t ovvs_hip_coarse_scores(const float* Q, const float* qn, int64_t nq, const float* C,
                                  const float* cn, int32_t nlist, int32_t dim, float* S,
                                  int64_t ldS, hipStream_t stream);

// Per row, the first P columns of S under the total order (score ascending,
// +-0 equal, NaN last, column ascending), written in rank order to
// out[row*P + r] (reference cpu_prims.cpp:24-106). P <= OVVS_HIP_MAX_PROBES, P <= N.
hipError_t ovvs_hip_select_topk(const float* S, int64_t ldS, int64_t nrows, int32_t N, int32_t P,
                                int32_t* out, hipStream_t stream);

// ---- coarse probe on the matrix cores (probe.hip) ----

// Limits of the fused probe: dim <= 32 * OVVS_PROBE_MAX_KSTEPS, P <= OVVS_PROBE_MAX_P, at
// least 2P of its (at most OVVS_PROBE_MAX_GROUPS) centroid groups, its LDS within 160 KiB,
// at most 256 (P <= 64), 512 (P <= 128) or OVVS_PROBE_CAP (512 where that does not fit
// the LDS; 2P + 32, at least 256, where that lets three workgroups share a CU) exact
// re-scores per query (a query with more takes the exact route).
#define OVVS_PROBE_MAX_KSTEPS 32
#define OVVS_PROBE_MAX_P 256
#define OVVS_PROBE_MAX_GROUPS 512
#define OVVS_PROBE_CAP 1024

struct OvvsProbeArgs {
  const float* queries;    // [nq * dim]
  const float* qnorm;      // [nq], exact row norms; or nullptr: the probe computes them
                           // (sequential sums, as ovvs_hip_row_norms) into qnorm_out
  float* qnorm_out;        // [nq] out when qnorm is nullptr
  unsigned long long* zero; // [8] set to 0 by the launch (the search's counters), or nullptr
  const int32_t* list_rank;  // with order_keys: [nlist] spatial rank of every list
  int32_t key_shift;         // order_keys[q] = list_rank[nearest probe] >> key_shift
  int32_t* order_keys;       // [nq] out (0 for flagged queries), or nullptr
  int64_t nq;
  int32_t dim;
  int32_t nlist;
  int32_t P;               // probes per query
  const float* centroids;  // [nlist * dim] row-major (exact re-score)
  const float* cnorm;      // [nlist], exact row norms
  float cnorm_max;         // max of cnorm (+inf if any is NaN or inf)
  const uint32_t* cmfma;   // centred centroids as bf16 matrix-core operands, see
                           // ovvs_probe_prepare
  const float* cmu;        // [dim] the centring vector mu
  const float* cnc;        // [nlist] centred squared norms
  float cnc_max;           // max of cnc (+inf if any is NaN or inf)
  int32_t* probes;         // [nq * P] out, rank order (rows with fallback[q] = 0)
  int32_t* fallback;       // [nq] out: 1 where the query needs the exact route
  unsigned long long* stamp; // or nullptr: the launch's first workgroup writes the
                             // device wall clock (wall_clock64) at its start here
};

// 1 when the fused probe handles these shapes.
int ovvs_hip_probe_mfma_supported(int32_t dim, int32_t nlist, int32_t P);
// 32-bit words in the bf16 centroid operand copy (0 if dim is unsupported).
size_t ovvs_hip_probe_cmfma_words(int32_t dim, int32_t nlist);
// Host-side preparation of the probe's centroid operands: mu[t] = the mean of column t
// (double sum, rounded to float); cnc[c] = left-to-right fp32 sum of fl(C[c][t] -
// mu[t])^2 and *cnc_max their maximum (+inf if any is not finite); ops: for tile t (16
// centroids), k-step s (32 dims) and lane l, the 16 bytes at word ((t * ceil(dim/32) + s)
// * 64 + l) * 4 hold the 8 bf16 values (round to nearest even) of fl(C[16t + l%16][k] -
// mu[k]), k = 32s + 8(l/16) + j, j = 0..7 (zero past nlist or dim).
void ovvs_probe_prepare(const float* C, int32_t nlist, int32_t dim, uint32_t* ops, float* mu,
                        float* cnc, float* cnc_max);
// Probe selection for every query; flags the queries the exact route must finish.
hipError_t ovvs_hip_probe_mfma(const OvvsProbeArgs* args, hipStream_t stream);
// The exact route for the queries with flags[q] != 0 (the ones the fused probe could
// not certify): exact scores of every centroid into S[q*nlist + c] (a scratch of
// nq * nlist floats), then their first P centroids in rank order into out[q*P ...].
// Unflagged queries are left untouched.
// stamp: as OvvsProbeArgs::stamp, or nullptr.
hipError_t ovvs_hip_probe_fallback(const float* Q, const float* qn, int64_t nq, const float* C,
                                   const float* cn, int32_t nlist, int32_t dim,
                                   const int32_t* flags, float* S, int32_t P, int32_t* out,
                                   unsigned long long* stamp, hipStream_t stream);

// Exact argmin over all centroids for each row of Q (top-1 of the coarse score
// under the same total order), fused with the score computation: labels[i].
hipError_t ovvs_hip_coarse_argmin(const float* Q, const float* qn, int64_t nq, const float* C,
                                  const float* cn, int32_t nlist, int32_t dim, int32_t* labels,
                                  hipStream_t stream);

struct OvvsScanArgs {
  const float* queries;        // [nq * dim]
  int64_t nq;
  int32_t dim;
  int32_t P;                   // probes per query
  const int32_t* probes;       // [nq * P] list ids in rank order
  const float* centroids;      // [nlist * dim]
  const float* codebooks;      // [pq_m * ks * dsub]
  int32_t pq_m;
  int32_t ks;                  // power of two, 16..256
  int32_t dsub;
  int32_t code_blocks;         // ceil(pq_m / OVVS_CODE_BLOCK)
  int32_t nlist;
  const int64_t* list_offsets; // [nlist + 1] the reference's list CSR (rows per list)
  const int32_t* list_seg;     // [nlist + 1] segment CSR
  const int32_t* seg_start;    // [nseg] first scan position of each segment (tile aligned)
  const int32_t* seg_len;      // [nseg] rows of each segment
  const uint32_t* seg_box;     // [nseg * pq_m * dsub] per dimension, the range of the rows'
                               // reconstructions plus the list centroid (absolute
                               // coordinates), binary16 rounded outward, packed
                               // lo | hi << 16; or nullptr
  const uint32_t* list_box;    // [nlist * pq_m * dsub] the same over each list; or nullptr
  const int32_t* list_grp;     // [nlist + 1] group CSR
  const int32_t* grp_seg;      // [ngrp + 1] first segment of each group
  const uint32_t* grp_box;     // [ngrp * pq_m * dsub] the same over each group; or nullptr
  const int32_t* order;        // [nq] queries in processing order (ovvs_hip_query_order), or
                               // nullptr for query b in workgroup b
  float box_cmax;              // max |centroid coordinate| (+inf if any is not finite)
  int64_t positions;           // scan positions
  const uint8_t* codes;        // tiled codes by scan position, see OVVS_CODE_TILE_ROWS
  const int64_t* ids;          // [positions] row ids by scan position
  const int32_t* rord;         // [positions] index of each row within its list
  const uint8_t* bitset;       // (n+7)/8 bytes or nullptr
  unsigned long long* stamp;   // as OvvsProbeArgs::stamp (k_scan's first workgroup), or nullptr
  int32_t K;                   // shortlist length (krefine), 1..OVVS_HIP_MAX_REFINE
  uint64_t* out_keys;          // [nq * K] (score key << 32 | dense ordinal), ascending
  int32_t* out_pos;            // [nq * K] scan positions
  int32_t* out_count;          // [nq]
  int32_t* out_stats;          // [nq * 4] per query: rows of the probed lists, non-empty
                               // probed lists, shortlist entries, 1 if a probe id is out
                               // of range
  // Handoff to the full-table scan (ovvs_hip_scan_table): a query whose rows past
  // the scan's first phase exceed a work budget (its lower bounds prune too little)
  // stops scoring and is appended to punt[] (*punt_count, cleared before the search);
  // that kernel then rewrites all its outputs. nullptr: no handoff.
  int32_t* punt;               // [nq]
  unsigned int* punt_count;
};

// Code scan + per-query shortlist of the K best (ADC score, dense ordinal) rows
// over all probed lists.
hipError_t ovvs_hip_scan(const OvvsScanArgs* args, hipStream_t stream);
// Full scan of the queries ovvs_hip_scan handed off (punt[0 .. *punt_count)): every
// row of every probed list scored, with the same outputs (out_keys, out_pos,
// out_count, out_stats) as ovvs_hip_scan, bit for bit. When the codebook fits in LDS
// beside sixteen waves (dsub 1, 2, 4 or 8, K <= 128), one query per wave computes the
// entries each row uses from it; otherwise each list's whole table is built in LDS.
// A fixed number of workgroups take the handed-off queries in turn (a search without
// any returns at once).
hipError_t ovvs_hip_scan_table(const OvvsScanArgs* args, hipStream_t stream);
// Dynamic LDS bytes of the full-table scan (0 if it does not fit the 160 KiB of a
// gfx950 workgroup, the table holding pq_m * ks fp32 entries, or if dim > 1024 or
// P > 1024).
size_t ovvs_hip_scan_table_lds_bytes(int32_t pq_m, int32_t ks, int32_t dim, int32_t K, int32_t P);
// order = the queries 0 .. nq-1 sorted by the spatial rank (list_rank, a permutation
// of the lists) of their nearest probed list (probes[q * P]); the scan's workgroups
// take it in turn, so that the queries resident on an XCD probe lists near each other.
// keys: [nq] workspace; with keys_ready it already holds every query's bucket
// (list_rank[probes[q * P]] >> ovvs_hip_query_key_shift(nlist)).
hipError_t ovvs_hip_query_order(const int32_t* probes, int64_t nq, int32_t P, const int32_t* list_rank,
                                int32_t nlist, int32_t* keys, int32_t keys_ready, int32_t* order,
                                hipStream_t stream);
int32_t ovvs_hip_query_key_shift(int32_t nlist);
// Dynamic LDS bytes the scan kernel needs for these shapes, shortlist length and
// probe count (0 if they exceed the 160 KiB a gfx950 workgroup can hold).
size_t ovvs_hip_scan_lds_bytes(int32_t pq_m, int32_t ks, int32_t dim, int32_t K,
                               int32_t P);

struct OvvsRefineArgs {
  const float* queries;   // [nq * dim]
  const float* qnorm;     // [nq]
  int64_t nq;
  int32_t dim;
  int32_t metric;         // ovvsMetric
  const float* dataset;   // [n * dim], row = id
  const float* xnorm;     // [n]
  int64_t n;
  int64_t positions;      // entries of ids
  const int64_t* ids;     // [positions] scan position -> id
  int32_t K;              // shortlist stride
  const int32_t* short_pos;    // [nq * K]
  const int32_t* short_count;  // [nq]
  int64_t k;              // outputs per query
  int64_t* out_ids;       // [nq * k]
  float* out_dist;        // [nq * k]
  unsigned long long* invalid;  // += shortlist entries whose position or id is out of range
  // Optional (both or neither): counters[i] += sum over the queries of
  // stats[q * 4 + i], i < 4 (the scan's per-query statistics), by extra
  // workgroups of the same launch.
  const int32_t* stats;
  unsigned long long* counters;
  // Optional: the launch's last workgroup copies counters[0, 5) here (host memory
  // mapped into the device's address space) after every other workgroup's atomics;
  // done is its ticket counter, zero before the launch.
  unsigned long long* counters_out;
  unsigned int* done;
  // Optional: the search's stage stamps [5] (device wall clock; [0, 3) written by the
  // probe, fallback and scan launches): the launch's first workgroup writes stamps[3]
  // when it starts; with counters_out, the last workgroup copies stamps[0, 4) and the
  // clock at its end to counters_out[8, 13).
  unsigned long long* stamps;
};

// Exact re-rank of each query's shortlist by the index metric and final select
// of the first min(k, count) by (distance, shortlist rank); (-1, +inf) padding;
// inner-product distances are returned as +ip (reference indexes.cpp:1067-1096).
hipError_t ovvs_hip_refine(const OvvsRefineArgs* args, hipStream_t stream);

// IVF-PQ k-nearest-neighbour graph (reference src/neighbors/graphs.cpp:767-797): for
// rows row0 + r, r < n, with search results nb[r * (degree + 1) ...] (rank order),
// graph[(row0 + r) * degree ...] = the results other than the row itself and -1, at
// most degree of them, then -1.
hipError_t ovvs_hip_knn_graph_rows(const int64_t* nb, int64_t n, int64_t row0, int32_t degree,
                                   int32_t* graph, hipStream_t stream);

// ScaNN-style index (reference src/neighbors/graphs.cpp:3286-3374).
// aniso[d] = sqrt(var_d / max(n, 1) + 1e-6) from left-to-right fp32 column sums
// (mean = sum / n, then var_d = sum of (x - mean)^2); one thread per column.
hipError_t ovvs_hip_column_aniso(const float* x, int64_t n, int32_t dim, float* aniso,
                                 hipStream_t stream);
// out[i*dim+d] = x[i*dim+d] * s[d]
hipError_t ovvs_hip_scale_columns(const float* x, int64_t rows, int32_t dim, const float* s,
                                  float* out, hipStream_t stream);
// Re-rank candidates from IVF-PQ results ids [nq * R]: pos[q*R+j] = q*R + t for the
// j-th result t whose id lies in [0, n), count[q] = j. nq * R < 2^31.
hipError_t ovvs_hip_ids_shortlist(const int64_t* ids, int64_t nq, int32_t R, int64_t n,
                                  int32_t* pos, int32_t* count, hipStream_t stream);

// ---- index build helpers (reference indexes.cpp:459-536, mixer.cpp:866-921) ----

// out[i*dsub+u] = x[i*dim + m*dsub + u]
hipError_t ovvs_hip_gather_sub(const float* x, int64_t n, int32_t dim, int32_t m, int32_t dsub,
                               float* out, hipStream_t stream);
// out[i*dim+t] = x[i*dim+t] - C[labels[i]*dim+t]
hipError_t ovvs_hip_residuals(const float* x, int64_t n, int32_t dim, const int32_t* labels,
                              const float* C, float* out, hipStream_t stream);
// out[c*dim+t] = x[rows[c]*dim+t]
hipError_t ovvs_hip_gather_rows(const float* x, int32_t dim, const int64_t* rows, int32_t count,
                                float* out, hipStream_t stream);
// Stable grouping of rows by label: order[] lists row indices grouped by label,
// ascending within a label; offsets[c] = first slot of label c, offsets[k] = n.
// temp/temp_bytes: scratch from ovvs_hip_group_temp_bytes.
size_t ovvs_hip_group_temp_bytes(int64_t n);
hipError_t ovvs_hip_group_by_label(const int32_t* labels, int64_t n, int32_t k,
                                   int32_t* sorted_labels, int32_t* order, int64_t* offsets,
                                   void* temp, size_t temp_bytes, hipStream_t stream);
// Lloyd mean update: for each centroid with rows, C[c] = (sum of its rows,
// left to right in row order) * (1/count); empty centroids keep their value.
hipError_t ovvs_hip_kmeans_update(const float* x, int32_t dim, const int32_t* order,
                                  const int64_t* offsets, int32_t k, float* C,
                                  hipStream_t stream);
// codes[i*pq_m+m] = argmin_j l2(resid_i,m - B[m][j]), first minimum wins
// (reference indexes.cpp:211-229).
hipError_t ovvs_hip_pq_encode(const float* resid, int64_t n, int32_t dim, int32_t pq_m,
                              int32_t ks, int32_t dsub, const float* codebooks, uint8_t* codes,
                              hipStream_t stream);

#ifdef __cplusplus
}
#endif
