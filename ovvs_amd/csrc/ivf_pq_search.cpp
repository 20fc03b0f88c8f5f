// ivf_pq_search.cpp — ovvsIvfPqSearch and its additive variants on one MI355X.
//
// Reference: ovvsIvfPqSearch, src/neighbors/indexes.cpp:538-1134. The argument
// checks, their order and their status codes follow the reference (:541-575);
// the clamps are nprobe := clamp(nprobe, 1, nlist) and krefine := max(krefine,
// k); outputs are staged and published only on success (:1101-1102); telemetry
// is merged only on success (:1103-1125).
//
// Device pipeline per call, all on the Resources stream:
//   1. query norms and probe selection, either
//      a. matrix-core probe with exact       ovvs_hip_probe_mfma (it also computes the
//         re-score (dim <= 1024, enough       query norms and clears the counters), then
//         centroid groups)                    for the queries it flags
//                                             ovvs_hip_probe_fallback
//      b. query norms, exact coarse scores   ovvs_hip_row_norms, ovvs_hip_coarse_scores
//         chunked over queries, row select   + ovvs_hip_select_topk
//   2. the scan's query order                ovvs_hip_query_order
//   3. fused LUT + code scan + shortlist    ovvs_hip_scan, then ovvs_hip_scan_table for
//                                           the queries it hands off (bounds that do
//                                           not prune: a whole table per list)
//   4. exact re-rank + final select, and    ovvs_hip_refine
//      the sum of the scan's statistics
// There is no host compute path: without a usable GPU the call fails with
// OVVS_STATUS_DEVICE_UNAVAILABLE.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <limits>
#include <new>

#include "internal.hpp"

using ovvs::GpuWork;

namespace {

using Clock = std::chrono::steady_clock;

size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

// Budget for one chunk of the [queries x nlist] coarse score matrix.
constexpr size_t kScoreChunkBytes = size_t(512) << 20;
// Batches of fewer queries than this (the scan's workgroups then number fewer than the
// compute units) skip the query order, which only decides which queries share an
// XCD's L2, and take the search counters from the refine launch's last workgroup
// instead of a copy (every workgroup of that launch takes a ticket from one counter,
// which costs more than the copy once there are thousands of them).
constexpr int64_t kSmallBatch = 256;

int64_t elapsed_ns(Clock::time_point a, Clock::time_point b) {
  const auto d = std::chrono::duration_cast<std::chrono::nanoseconds>(b - a).count();
  return d > 0 ? d : 0;
}

int64_t event_ns(hipEvent_t a, hipEvent_t b) {
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, a, b) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return static_cast<int64_t>(static_cast<double>(ms) * 1e6);
}

struct Carver {
  unsigned char* base;
  size_t off = 0;
  template <class T>
  T* take(size_t count) {
    T* p = reinterpret_cast<T*>(base + off);
    off += align256(count * sizeof(T));
    return p;
  }
};

#define SEARCH_HIP(expr)                            \
  do {                                              \
    const hipError_t hip_e_ = (expr);               \
    if (hip_e_ != hipSuccess) {                     \
      (void)hipGetLastError();                      \
      return ovvs::status_from_hip(hip_e_);         \
    }                                               \
  } while (0)

#define SEARCH_TRY(expr)                      \
  do {                                        \
    const ovvsStatus st_ = (expr);            \
    if (st_ != OVVS_STATUS_SUCCESS) return st_; \
  } while (0)

// Where the caller's buffers live and where the workspace comes from.
enum class Io {
  kHost,     // host queries, bitset and outputs; the Resources' workspace
  kDevice,   // device buffers; the Resources' workspace
  kScratch,  // device buffers; the caller's scratch, nothing allocated
};

ovvsStatus search_impl(ovvsResources_t res, ovvsIvfPqIndex_t index, const float* queries,
                       int64_t nq, int64_t k, int32_t nprobe, int32_t krefine,
                       const uint8_t* bitset, ovvsDType lut_dtype, Io io, void* scratch,
                       size_t scratch_bytes, int64_t* neighbors, float* distances) {
  const auto started = Clock::now();
  if (!res || !index || !queries || !neighbors || !distances || nq <= 0 || k <= 0 ||
      k > std::numeric_limits<int32_t>::max()) {
    return OVVS_STATUS_INVALID_ARGUMENT;
  }
  if (nq > std::numeric_limits<int64_t>::max() / k ||
      static_cast<uint64_t>(nq) >
          static_cast<uint64_t>(std::numeric_limits<size_t>::max() / sizeof(int64_t)) /
              static_cast<uint64_t>(k)) {
    return OVVS_STATUS_SHAPE_MISMATCH;
  }
  ovvsIvfPqIndexImpl& ix = *index;
  if (ix.n <= 0 || ix.dim <= 0 || ix.nlist <= 0 || ix.pq_m <= 0 || ix.pq_ks <= 0 ||
      ix.lists.size() != static_cast<size_t>(ix.nlist) ||
      ix.codes.size() != static_cast<size_t>(ix.n) * static_cast<size_t>(ix.pq_m) ||
      static_cast<uint64_t>(nq) >
          static_cast<uint64_t>(std::numeric_limits<size_t>::max() / sizeof(float)) /
              static_cast<uint64_t>(ix.dim) ||
      static_cast<uint64_t>(nq) >
          static_cast<uint64_t>(std::numeric_limits<size_t>::max() / sizeof(int64_t)) /
              static_cast<uint64_t>(ix.nlist)) {
    return OVVS_STATUS_INVALID_ARGUMENT;
  }
  // Table precision: the scan stores no table (each entry is computed in registers
  // where a row uses it), so a binary16 table would save no memory traffic or
  // storage, only rank candidates differently from the reference. Both accepted
  // precisions are served with fp32 entries, the reference's arithmetic.
  if (lut_dtype != OVVS_DTYPE_F32 && lut_dtype != OVVS_DTYPE_F16) return OVVS_STATUS_UNSUPPORTED;
  const int32_t P = std::max(1, std::min(nprobe, ix.nlist));
  const int32_t R = krefine < static_cast<int32_t>(k) ? static_cast<int32_t>(k) : krefine;
  // Fixed limits of the kernels: fail closed, as the reference's GPU route does
  // for krefine > 128 (indexes.cpp:576-584).
  // OVVS_HIP_MAX_REFINE bounds krefine and k.
  if (R > OVVS_HIP_MAX_REFINE || P > OVVS_HIP_MAX_PROBES ||
      ovvs_hip_scan_lds_bytes(ix.pq_m, ix.pq_ks, static_cast<int32_t>(ix.dim), R, P) == 0 ||
      nq > 0x7fffffff || ix.n > 0x7fffffff) {
    return OVVS_STATUS_DEVICE_UNAVAILABLE;
  }

  try {
    std::lock_guard<std::mutex> lock(res->call_mutex);
    SEARCH_TRY(res->ensure_gpu());
    GpuWork work;
    if (io == Io::kScratch) {
      // Nothing may be allocated: the device mirror of the index must exist.
      std::lock_guard<std::mutex> dev_lock(ix.device_mutex);
      if (!ix.dev || ix.dev->device != res->device) return OVVS_STATUS_INVALID_ARGUMENT;
    } else {
      SEARCH_TRY(ix.ensure_device(*res, work));
    }
    const ovvs::IndexDevice& dv = *ix.dev;
    hipStream_t s = res->stream;
    const int32_t dim = static_cast<int32_t>(ix.dim);
    const bool device_io = io != Io::kHost;

    const size_t nqk = static_cast<size_t>(nq) * static_cast<size_t>(k);
    const size_t bitset_bytes = static_cast<size_t>((ix.n + 7) / 8);
    const size_t qbytes = static_cast<size_t>(nq) * dim * 4;

    // Every workspace buffer but the coarse score chunk.
    size_t fixed = 0;
    fixed += device_io ? 0 : align256(qbytes);                          // queries
    fixed += align256(static_cast<size_t>(nq) * 4);                     // query norms
    fixed += align256(static_cast<size_t>(nq) * P * 4);                 // probes
    fixed += align256(static_cast<size_t>(nq) * 4);                     // probe fallback flags
    fixed += 2 * align256(static_cast<size_t>(nq) * 4);                 // scan query order, keys
    fixed += align256(static_cast<size_t>(nq) * R * 8);                 // shortlist keys
    fixed += align256(static_cast<size_t>(nq) * R * 4);                 // shortlist positions
    fixed += align256(static_cast<size_t>(nq) * 4);                     // shortlist counts
    fixed += align256(static_cast<size_t>(nq) * 16);                    // scan statistics
    fixed += align256(static_cast<size_t>(nq) * 4);                     // full-table handoffs
    fixed += device_io ? 0 : align256(nqk * 8) + align256(nqk * 4);     // staged outputs
    fixed += align256(16 * 8);                                          // counters, stamps
    fixed += (!device_io && bitset) ? align256(bitset_bytes) : 0;
    // Query chunk of the coarse score matrix (the exact route and the probe's
    // fallback work through it chunk by chunk).
    const size_t row_bytes = static_cast<size_t>(ix.nlist) * 4;
    int64_t qc = static_cast<int64_t>(kScoreChunkBytes / row_bytes);
    unsigned char* base = nullptr;
    if (io == Io::kScratch) {
      if (fixed > scratch_bytes || (scratch_bytes - fixed) / row_bytes < 1 ||
          reinterpret_cast<uintptr_t>(scratch) % 256 != 0) {
        return OVVS_STATUS_SHAPE_MISMATCH;
      }
      qc = std::min<int64_t>(qc, static_cast<int64_t>(((scratch_bytes - fixed) & ~size_t(255)) / row_bytes));
      qc = std::max<int64_t>(1, std::min<int64_t>(qc, nq));
      base = static_cast<unsigned char*>(scratch);
    } else {
      qc = std::max<int64_t>(1, std::min<int64_t>(qc, nq));
      SEARCH_TRY(res->reserve_workspace(fixed + align256(static_cast<size_t>(qc) * row_bytes), work));
      base = static_cast<unsigned char*>(res->workspace.get());
    }
    // Pinned host staging: [counters 32 B | ids | distances | queries | bitset] with
    // host buffers, the counters alone with device buffers, none with the scratch.
    const size_t pin_ids = 256, pin_dist = pin_ids + align256(nqk * 8);
    const size_t pin_q = pin_dist + align256(nqk * 4), pin_bits = pin_q + align256(qbytes);
    if (io == Io::kHost) {
      SEARCH_TRY(res->reserve_pinned(pin_bits + (bitset ? bitset_bytes : 0)));
    } else if (io == Io::kDevice) {
      SEARCH_TRY(res->reserve_pinned(16 * 8));
    }
    unsigned long long scratch_counters[16] = {};
    unsigned char* pin = io == Io::kScratch ? reinterpret_cast<unsigned char*>(scratch_counters)
                                            : static_cast<unsigned char*>(res->pinned);

    Carver cv{base};
    const float* d_q = device_io ? queries : nullptr;
    if (!device_io) d_q = cv.take<float>(static_cast<size_t>(nq) * dim);
    float* d_qn = cv.take<float>(static_cast<size_t>(nq));
    int32_t* d_probes = cv.take<int32_t>(static_cast<size_t>(nq) * P);
    int32_t* d_flags = cv.take<int32_t>(static_cast<size_t>(nq));
    int32_t* d_order = cv.take<int32_t>(static_cast<size_t>(nq));
    int32_t* d_okeys = cv.take<int32_t>(static_cast<size_t>(nq));
    uint64_t* d_skeys = cv.take<uint64_t>(static_cast<size_t>(nq) * R);
    int32_t* d_spos = cv.take<int32_t>(static_cast<size_t>(nq) * R);
    int32_t* d_scnt = cv.take<int32_t>(static_cast<size_t>(nq));
    int32_t* d_sstats = cv.take<int32_t>(static_cast<size_t>(nq) * 4);
    int32_t* d_punt = cv.take<int32_t>(static_cast<size_t>(nq));
    // Device outputs are written by the refine kernel in place; host outputs are
    // staged and copied only after the search has succeeded.
    int64_t* d_oid = device_io ? neighbors : cv.take<int64_t>(nqk);
    float* d_odist = device_io ? distances : cv.take<float>(nqk);
    // Host outputs: the refine kernel writes straight into the pinned staging buffer
    // (mapped into the device's address space), which replaces two device-to-host
    // copies; they reach the caller's arrays only after the checks below.
    // Small batches take the search counters the same way (the refine launch's last
    // workgroup writes them); the scratch entry's counters land in host stack memory
    // by a copy.
    const bool small = nq < kSmallBatch;
    bool direct_out = false;
    unsigned long long* d_cnt_out = nullptr;
    if (io != Io::kScratch) {
      void* pdev = nullptr;
      if (hipHostGetDevicePointer(&pdev, res->pinned, 0) == hipSuccess && pdev) {
        if (small) d_cnt_out = static_cast<unsigned long long*>(pdev);
        if (io == Io::kHost) {
          d_oid = reinterpret_cast<int64_t*>(static_cast<unsigned char*>(pdev) + pin_ids);
          d_odist = reinterpret_cast<float*>(static_cast<unsigned char*>(pdev) + pin_dist);
          direct_out = true;
        }
      } else {
        (void)hipGetLastError();
      }
    }
    // counters: [0] candidate rows, [1] non-empty probed lists, [2] shortlist entries,
    // [3] out-of-range probe ids or shortlist positions, [4] queries handed off to the
    // full-table scan (as unsigned int), [5] the refine launch's finished workgroups (as
    // unsigned int); [6, 8) unused; [8, 13) the device wall clock when the probe, its
    // fallback, the scan and the refine start and when the refine ends (the stage times
    // of small batches on the matrix-core route; the first four are written by those
    // launches, the end by the refine's last workgroup with the counters).
    unsigned long long* d_counters = cv.take<unsigned long long>(16);
    unsigned long long* d_stamps = d_counters + 8;
    const uint8_t* d_bitset = device_io ? bitset : nullptr;
    if (!device_io && bitset) d_bitset = cv.take<uint8_t>(bitset_bytes);
    float* d_scores = cv.take<float>(static_cast<size_t>(qc) * ix.nlist);

    if (!device_io) {
      // Host inputs go through the pinned staging buffer in pieces, so that the
      // DMA of one piece overlaps the host copy of the next.
      if (bitset) {
        ovvs::parallel_copy(pin + pin_bits, bitset, bitset_bytes);
        SEARCH_HIP(hipMemcpyAsync(const_cast<uint8_t*>(d_bitset), pin + pin_bits, bitset_bytes,
                                  hipMemcpyHostToDevice, s));
        ovvs::saturating_add(work.h2d_calls, 1);
        ovvs::saturating_add(work.h2d_bytes, static_cast<int64_t>(bitset_bytes));
      }
      constexpr size_t kPiece = size_t(1) << 20;
      const unsigned char* src = reinterpret_cast<const unsigned char*>(queries);
      unsigned char* dst = reinterpret_cast<unsigned char*>(const_cast<float*>(d_q));
      for (size_t off = 0; off < qbytes; off += kPiece) {
        const size_t len = std::min(kPiece, qbytes - off);
        ovvs::parallel_copy(pin + pin_q + off, src + off, len);
        SEARCH_HIP(hipMemcpyAsync(dst + off, pin + pin_q + off, len, hipMemcpyHostToDevice, s));
        ovvs::saturating_add(work.h2d_calls, 1);
      }
      ovvs::saturating_add(work.h2d_bytes, static_cast<int64_t>(qbytes));
    }
    const bool mfma_probe =
        dv.cmfma.get() != nullptr && ovvs_hip_probe_mfma_supported(dim, ix.nlist, P) != 0;
    // The matrix-core probe computes the query norms and clears the counters itself.
    if (!mfma_probe) SEARCH_HIP(hipMemsetAsync(d_counters, 0, 8 * 8, s));

    // Stage times: small batches on the matrix-core route read the launches' stamps
    // (each event recorded between launches adds a few microseconds to a chain that
    // then lasts about 85 us); other searches record a HIP event at every stage
    // boundary on the search's stream.
    hipEvent_t* ev = res->events;
    const bool stamped = mfma_probe && d_cnt_out != nullptr;
    if (!stamped) SEARCH_HIP(hipEventRecord(ev[0], s));
    if (!mfma_probe) SEARCH_HIP(ovvs_hip_row_norms(d_q, nq, dim, d_qn, s));
    int64_t chunks = 0;
    if (mfma_probe) {
      // Matrix-core probe with exact re-score; flagged queries take the exact route.
      OvvsProbeArgs pa{};
      pa.queries = d_q;
      pa.qnorm = nullptr;
      pa.qnorm_out = d_qn;
      pa.zero = d_counters;
      pa.list_rank = dv.list_rank.as<int32_t>();
      pa.key_shift = ovvs_hip_query_key_shift(ix.nlist);
      pa.order_keys = d_okeys;
      pa.nq = nq;
      pa.dim = dim;
      pa.nlist = ix.nlist;
      pa.P = P;
      pa.centroids = dv.centroids.as<float>();
      pa.cnorm = dv.cnorm.as<float>();
      pa.cnorm_max = dv.cnorm_max;
      pa.cmfma = dv.cmfma.as<uint32_t>();
      pa.cmu = dv.cmu.as<float>();
      pa.cnc = dv.cnc.as<float>();
      pa.cnc_max = dv.cnc_max;
      pa.probes = d_probes;
      pa.fallback = d_flags;
      pa.stamp = stamped ? d_stamps : nullptr;
      SEARCH_HIP(ovvs_hip_probe_mfma(&pa, s));
      if (!stamped) SEARCH_HIP(hipEventRecord(ev[1], s));
      for (int64_t q0 = 0; q0 < nq; q0 += qc) {
        const int64_t cnt = std::min(qc, nq - q0);
        SEARCH_HIP(ovvs_hip_probe_fallback(d_q + q0 * dim, d_qn + q0, cnt,
                                           dv.centroids.as<float>(), dv.cnorm.as<float>(),
                                           ix.nlist, dim, d_flags + q0, d_scores, P,
                                           d_probes + q0 * P,
                                           stamped && q0 == 0 ? d_stamps + 1 : nullptr, s));
        ++chunks;
      }
      work.kernel_launches += 1;
    } else {
      for (int64_t q0 = 0; q0 < nq; q0 += qc) {
        const int64_t cnt = std::min(qc, nq - q0);
        SEARCH_HIP(ovvs_hip_coarse_scores(d_q + q0 * dim, d_qn + q0, cnt,
                                          dv.centroids.as<float>(), dv.cnorm.as<float>(),
                                          ix.nlist, dim, d_scores, ix.nlist, s));
        if (q0 == 0) SEARCH_HIP(hipEventRecord(ev[1], s));
        SEARCH_HIP(
            ovvs_hip_select_topk(d_scores, ix.nlist, cnt, ix.nlist, P, d_probes + q0 * P, s));
        ++chunks;
      }
    }
    // The scan's query order (counted in the probe-selection stage, so that the scan
    // stage times the scan kernel alone); small batches skip it.
    const bool ordered = !small;
    if (ordered)
      SEARCH_HIP(ovvs_hip_query_order(d_probes, nq, P, dv.list_rank.as<int32_t>(), ix.nlist,
                                      d_okeys, mfma_probe ? 1 : 0, d_order, s));
    if (!stamped) SEARCH_HIP(hipEventRecord(ev[2], s));

    OvvsScanArgs sa{};
    sa.queries = d_q;
    sa.nq = nq;
    sa.dim = dim;
    sa.P = P;
    sa.probes = d_probes;
    sa.centroids = dv.centroids.as<float>();
    sa.codebooks = dv.codebooks.as<float>();
    sa.pq_m = ix.pq_m;
    sa.ks = ix.pq_ks;
    sa.dsub = ix.dsub;
    sa.code_blocks = dv.code_blocks;
    sa.nlist = ix.nlist;
    sa.list_offsets = dv.offsets.as<int64_t>();
    sa.list_seg = dv.list_seg.as<int32_t>();
    sa.seg_start = dv.seg_start.as<int32_t>();
    sa.seg_len = dv.seg_len.as<int32_t>();
    sa.seg_box = dv.box_dims > 0 ? dv.seg_box.as<uint32_t>() : nullptr;
    sa.list_box = dv.box_dims > 0 ? dv.list_box.as<uint32_t>() : nullptr;
    sa.box_cmax = dv.box_cmax;
    sa.list_grp = dv.list_grp.as<int32_t>();
    sa.grp_seg = dv.grp_seg.as<int32_t>();
    sa.grp_box = dv.box_dims > 0 ? dv.grp_box.as<uint32_t>() : nullptr;
    sa.order = ordered ? d_order : nullptr;
    sa.positions = dv.positions;
    sa.codes = dv.codes.as<uint8_t>();
    sa.ids = dv.ids.as<int64_t>();
    sa.rord = dv.rord.as<int32_t>();
    sa.bitset = d_bitset;
    sa.K = R;
    sa.out_keys = d_skeys;
    sa.out_pos = d_spos;
    sa.out_count = d_scnt;
    sa.out_stats = d_sstats;
    // Queries whose bounds do not prune go to the full-table scan when its table fits.
    const bool table_ok =
        ovvs_hip_scan_table_lds_bytes(ix.pq_m, ix.pq_ks, dim, R, P) != 0;
    sa.punt = table_ok ? d_punt : nullptr;
    sa.punt_count = reinterpret_cast<unsigned int*>(d_counters + 4);
    sa.stamp = stamped ? d_stamps + 2 : nullptr;
    SEARCH_HIP(ovvs_hip_scan(&sa, s));
    if (table_ok) SEARCH_HIP(ovvs_hip_scan_table(&sa, s));
    if (!stamped) SEARCH_HIP(hipEventRecord(ev[3], s));

    OvvsRefineArgs ra{};
    ra.queries = d_q;
    ra.qnorm = d_qn;
    ra.nq = nq;
    ra.dim = dim;
    ra.metric = static_cast<int32_t>(ix.metric);
    ra.dataset = dv.dataset.as<float>();
    ra.xnorm = dv.xnorm.as<float>();
    ra.n = ix.n;
    ra.positions = dv.positions;
    ra.ids = dv.ids.as<int64_t>();
    ra.K = R;
    ra.short_pos = d_spos;
    ra.short_count = d_scnt;
    ra.k = k;
    ra.out_ids = d_oid;
    ra.out_dist = d_odist;
    ra.invalid = d_counters + 3;
    ra.stats = d_sstats;  // the scan's per-query statistics, summed by the same launch
    ra.counters = d_counters;
    ra.counters_out = d_cnt_out;
    ra.done = reinterpret_cast<unsigned int*>(d_counters + 5);
    ra.stamps = stamped ? d_stamps : nullptr;
    SEARCH_HIP(ovvs_hip_refine(&ra, s));
    if (!stamped) SEARCH_HIP(hipEventRecord(ev[4], s));
    work.kernel_launches +=
        (mfma_probe ? 3 + chunks : 5 + 2 * chunks) + (table_ok ? 1 : 0) - (ordered ? 0 : 1);

    if (!d_cnt_out) {
      SEARCH_HIP(hipMemcpyAsync(pin, d_counters, 5 * 8, hipMemcpyDeviceToHost, s));
      ovvs::saturating_add(work.d2h_calls, 1);
      ovvs::saturating_add(work.d2h_bytes, 40);
    }
    if (!device_io && !direct_out) {
      SEARCH_HIP(hipMemcpyAsync(pin + pin_ids, d_oid, nqk * 8, hipMemcpyDeviceToHost, s));
      SEARCH_HIP(hipMemcpyAsync(pin + pin_dist, d_odist, nqk * 4, hipMemcpyDeviceToHost, s));
      ovvs::saturating_add(work.d2h_calls, 2);
      ovvs::saturating_add(work.d2h_bytes, static_cast<int64_t>(nqk * 12));
    }
    ovvs::saturating_add(work.wait_calls, 1);
    SEARCH_HIP(hipStreamSynchronize(s));
    unsigned long long counters[13];
    std::memcpy(counters, pin, sizeof(counters));
    // A probe id or shortlist position out of range is an internal error: the
    // kernels count it instead of dereferencing it, and nothing is published.
    if (counters[3] != 0) return OVVS_STATUS_ERROR;

    // Success: publish the host outputs (device outputs already hold the results).
    if (!device_io) {
      ovvs::parallel_copy(neighbors, pin + pin_ids, nqk * 8);
      ovvs::parallel_copy(distances, pin + pin_dist, nqk * 4);
    }

    ovvsIvfPqSearchStatsV1 d{};
    d.successful_calls = 1;
    d.blocks = chunks;
    d.queries = nq;
    d.tasks = static_cast<int64_t>(std::min<unsigned long long>(counters[1], INT64_MAX));
    d.candidate_rows = static_cast<int64_t>(std::min<unsigned long long>(counters[0], INT64_MAX));
    d.selected_rows = static_cast<int64_t>(std::min<unsigned long long>(counters[2], INT64_MAX));
    if (stamped) {
      // Stamps are wall-clock ticks of the device; a stage is the time from its first
      // launch's start to the next stage's (the refine: to its last workgroup's end).
      const unsigned long long* t = counters + 8;
      auto span = [&](unsigned long long a, unsigned long long b) -> int64_t {
        return b > a ? static_cast<int64_t>(static_cast<double>(b - a) * 1e6 / res->wall_khz) : 0;
      };
      d.coarse_pairwise_ns = span(t[0], t[1]);
      d.coarse_topk_ns = span(t[1], t[2]);
      d.adc_scan_select_ns = span(t[2], t[3]);
      d.refine_distance_ns = span(t[3], t[4]);
    } else if (chunks == 1) {
      d.coarse_pairwise_ns = event_ns(ev[0], ev[1]);
      d.coarse_topk_ns = event_ns(ev[1], ev[2]);
      d.adc_scan_select_ns = event_ns(ev[2], ev[3]);
      d.refine_distance_ns = event_ns(ev[3], ev[4]);
    } else {
      d.coarse_pairwise_ns = event_ns(ev[0], ev[2]);
      d.adc_scan_select_ns = event_ns(ev[2], ev[3]);
      d.refine_distance_ns = event_ns(ev[3], ev[4]);
    }
    d.total_wall_ns = elapsed_ns(started, Clock::now());
    int64_t named = 0;
    ovvs::saturating_add(named, d.coarse_pairwise_ns);
    ovvs::saturating_add(named, d.coarse_topk_ns);
    ovvs::saturating_add(named, d.adc_scan_select_ns);
    ovvs::saturating_add(named, d.refine_distance_ns);
    d.planning_ns = d.total_wall_ns > named ? d.total_wall_ns - named : 0;
    d.gpu_allocation_calls = work.allocation_calls;
    d.gpu_allocation_bytes = work.allocation_bytes;
    d.gpu_h2d_calls = work.h2d_calls;
    d.gpu_h2d_bytes = work.h2d_bytes;
    d.gpu_d2h_calls = work.d2h_calls;
    d.gpu_d2h_bytes = work.d2h_bytes;
    d.gpu_kernel_launches = work.kernel_launches;
    d.gpu_wait_calls = work.wait_calls;
    {
      std::lock_guard<std::mutex> stats_lock(res->stats_mutex);
      ovvsIvfPqSearchStatsV1& t = res->stats;
      t.abi_version = OVVS_IVF_PQ_SEARCH_STATS_ABI_V1;
      t.struct_size = sizeof(t);
      int64_t* dst = &t.successful_calls;
      const int64_t* src = &d.successful_calls;
      for (int i = 0; i < 24; ++i) ovvs::saturating_add(dst[i], src[i]);
    }
    res->table_queries += static_cast<int64_t>(counters[4] & 0xffffffffull);
    res->last_device = OVVS_DEVICE_GPU;
    res->last_compute_dtype = OVVS_DTYPE_F32;
    return OVVS_STATUS_SUCCESS;
  } catch (const std::bad_alloc&) {
    return OVVS_STATUS_OOM;
  } catch (...) {
    return OVVS_STATUS_ERROR;
  }
}

}  // namespace

ovvsStatus ovvs::ivf_pq_search_scratch(ovvsResources_t res, ovvsIvfPqIndex_t index,
                                       const float* queries, int64_t nq, int64_t k,
                                       int32_t nprobe, int32_t krefine, const uint8_t* bitset,
                                       ovvsDType lut_dtype, int64_t* neighbors, float* distances,
                                       void* scratch, size_t scratch_bytes) {
  if (!scratch) return OVVS_STATUS_INVALID_ARGUMENT;
  return search_impl(res, index, queries, nq, k, nprobe, krefine, bitset, lut_dtype, Io::kScratch,
                     scratch, scratch_bytes, neighbors, distances);
}

extern "C" {

OVVS_API ovvsStatus ovvsIvfPqSearch(ovvsResources_t res, ovvsIvfPqIndex_t index,
                                    const float* queries, int64_t nq, int64_t k, int32_t nprobe,
                                    int32_t krefine, const uint8_t* bitset, int64_t* neighbors,
                                    float* distances) {
  return search_impl(res, index, queries, nq, k, nprobe, krefine, bitset, OVVS_DTYPE_F32, Io::kHost,
                     nullptr, 0, neighbors, distances);
}

OVVS_API ovvsStatus ovvsIvfPqSearchEx(ovvsResources_t res, ovvsIvfPqIndex_t index,
                                      const float* queries, int64_t nq, int64_t k,
                                      int32_t nprobe, int32_t krefine, const uint8_t* bitset,
                                      ovvsDType lut_dtype, int64_t* neighbors,
                                      float* distances) {
  return search_impl(res, index, queries, nq, k, nprobe, krefine, bitset, lut_dtype, Io::kHost,
                     nullptr, 0, neighbors, distances);
}

OVVS_API ovvsStatus ovvsIvfPqSearchDevice(ovvsResources_t res, ovvsIvfPqIndex_t index,
                                          const float* queries, int64_t nq, int64_t k,
                                          int32_t nprobe, int32_t krefine,
                                          const uint8_t* bitset, ovvsDType lut_dtype,
                                          int64_t* neighbors, float* distances) {
  return search_impl(res, index, queries, nq, k, nprobe, krefine, bitset, lut_dtype, Io::kDevice,
                     nullptr, 0, neighbors, distances);
}

}  // extern "C"
