// internal.hpp — host-side objects behind the libovvs C ABI.
//
// ovvsResourcesImpl  one HIP stream, a grow-only device workspace, pinned host
//                    staging and the IVF-PQ telemetry of one caller thread
//                    (counterpart of the reference ResourcesData,
//                    src/internal.hpp:459-562, minus everything that is not
//                    IVF-PQ).
// ovvsIvfPqIndexImpl the index in the reference's logical form (reference
//                    src/neighbors/indexes.cpp:34-48): a host copy that serializes
//                    byte-identically to IPQ1, plus a device mirror laid out for
//                    the scan kernel and created on first GPU use.
#pragma once

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <vector>

#include "kernels.hpp"
#include "ovvs/ovvs.h"

namespace ovvs {

// Owning device allocation.
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  ~DeviceBuffer() { reset(); }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  hipError_t allocate(size_t bytes);
  void reset();
  void* get() const { return ptr_; }
  size_t size() const { return bytes_; }
  template <class T>
  T* as() const {
    return static_cast<T*>(ptr_);
  }

 private:
  void* ptr_ = nullptr;
  size_t bytes_ = 0;
};

// Host form of the scan order (scan_layout.cpp): each list's rows split into
// segments of rows with nearby reconstructions, every segment starting at a
// 64-row code tile (the tail of its last tile is padding).
struct ScanLayoutHost {
  int64_t positions = 0;           // scan positions: rows plus padding, a multiple of 64
  int32_t box_dims = 0;            // pq_m * dsub
  std::vector<int32_t> list_seg;   // [nlist + 1] segment CSR
  std::vector<int32_t> list_grp;   // [nlist + 1] group CSR (groups of consecutive segments)
  std::vector<int32_t> grp_seg;    // [ngrp + 1] first segment of each group
  std::vector<uint32_t> grp_box;   // [ngrp * box_dims] union of the group's segment boxes
  std::vector<int32_t> seg_start;  // [nseg] first scan position
  std::vector<int32_t> seg_len;    // [nseg] rows
  std::vector<uint32_t> seg_box;   // [nseg * box_dims] (lo, hi) of the rows' reconstructions
                                   // plus the list centroid (absolute coordinates), as
                                   // binary16 rounded outward, packed lo | hi << 16
  std::vector<uint32_t> list_box;  // [nlist * box_dims] the same over each whole list
  float cmax = 0.f;                // max |centroid coordinate| (+inf if any is not finite)
  std::vector<int32_t> list_rank;  // [nlist] spatial order of the lists (a permutation)
  std::vector<int64_t> ids;        // [positions] row id, -1 for padding
  std::vector<int32_t> rord;       // [positions] index of the row within its list, -1 padding
  std::vector<uint8_t> codes;      // tiled codes by scan position (kernels.hpp)
};

// Segments of at most seg_rows rows. Fails with DEVICE_UNAVAILABLE when the scan
// positions or segments exceed 32-bit indexing.
ovvsStatus make_scan_layout(const ovvsIvfPqIndexImpl& ix, int seg_rows, ScanLayoutHost& out);
// Largest binary16 <= lo and smallest >= hi, packed lo | hi << 16 (lo, hi not NaN),
// and the inverse of one half of it.
uint32_t pack_box_fp16(float lo, float hi);
float unpack_box_fp16(uint32_t b, int hi);
// The range [c + lo, c + hi], rounded outward, packed the same way.
uint32_t pack_abs_box_fp16(float c, float lo, float hi);

// Device copy of an index. Codes, ids and in-list row indices are in scan order
// (ScanLayoutHost); offsets are the reference's list CSR (rows per list and the
// ordinal base of each list); dataset rows are by id.
struct IndexDevice {
  int device = -1;
  int32_t code_blocks = 0;
  int64_t positions = 0;   // scan positions
  int32_t box_dims = 0;    // dimensions of each segment box (0: no boxes)
  float box_cmax = 0.f;    // max |centroid coordinate| (ScanLayoutHost::cmax)
  DeviceBuffer centroids;  // [nlist * dim] f32
  DeviceBuffer cnorm;      // [nlist] f32
  float cnorm_max = 0.f;   // max of cnorm, +inf if any is NaN or inf
  DeviceBuffer cmfma;      // centred centroids as bf16 matrix-core operands (empty when the
                           // probe cannot take the dimension)
  DeviceBuffer cmu;        // [dim] f32 centring vector of the probe operands
  DeviceBuffer cnc;        // [nlist] f32 centred squared norms
  float cnc_max = 0.f;     // max of cnc, +inf if any is NaN or inf
  DeviceBuffer codebooks;  // [pq_m * ks * dsub] f32
  DeviceBuffer codes;      // [positions / 64 * code_blocks * 512] u8
  DeviceBuffer ids;        // [positions] i64
  DeviceBuffer rord;       // [positions] i32
  DeviceBuffer offsets;    // [nlist + 1] i64
  DeviceBuffer list_seg;   // [nlist + 1] i32
  DeviceBuffer seg_start;  // [nseg] i32
  DeviceBuffer seg_len;    // [nseg] i32
  DeviceBuffer seg_box;    // [nseg * box_dims] packed binary16 (lo, hi)
  DeviceBuffer list_box;   // [nlist * box_dims] packed binary16 (lo, hi)
  DeviceBuffer list_rank;  // [nlist] i32 spatial order of the lists
  DeviceBuffer list_grp;   // [nlist + 1] i32
  DeviceBuffer grp_seg;    // [ngrp + 1] i32
  DeviceBuffer grp_box;    // [ngrp * box_dims] packed binary16 (lo, hi)
  DeviceBuffer dataset;    // [n * dim] f32
  DeviceBuffer xnorm;      // [n] f32
};

// Work counters of one call, merged into the telemetry on success.
struct GpuWork {
  int64_t allocation_calls = 0;
  int64_t allocation_bytes = 0;
  int64_t h2d_calls = 0;
  int64_t h2d_bytes = 0;
  int64_t d2h_calls = 0;
  int64_t d2h_bytes = 0;
  int64_t kernel_launches = 0;
  int64_t wait_calls = 0;
};

void saturating_add(int64_t& value, int64_t delta) noexcept;

// True when a HIP device is present (probed once; no context is created when
// there is none).
bool gpu_present();

// Copies bytes from src to dst (host memory) with a small pool of worker threads
// shared by the library (one copy at a time; a copy that finds the pool busy, or
// that is too small to split, runs on the calling thread).
void parallel_copy(void* dst, const void* src, size_t bytes);

// ovvsIvfPqSearchDevice with every workspace buffer carved from the caller's
// scratch (device memory of scratch_bytes bytes) instead of the Resources'
// workspace: no device or host memory is allocated. The index must already be
// resident on the device (INVALID_ARGUMENT otherwise); a batch whose buffers do
// not fit the scratch returns SHAPE_MISMATCH.
ovvsStatus ivf_pq_search_scratch(ovvsResources_t res, ovvsIvfPqIndex_t index,
                                 const float* queries, int64_t nq, int64_t k, int32_t nprobe,
                                 int32_t krefine, const uint8_t* bitset, ovvsDType lut_dtype,
                                 int64_t* neighbors, float* distances, void* scratch,
                                 size_t scratch_bytes);

// Maps a HIP error to the ABI status.
ovvsStatus status_from_hip(hipError_t e);

}  // namespace ovvs

struct ovvsResourcesImpl {
  ovvsPolicy policy = OVVS_POLICY_AUTO;
  std::atomic<ovvsDevice> last_device{OVVS_DEVICE_CPU};
  std::atomic<ovvsDType> last_compute_dtype{OVVS_DTYPE_F32};

  std::mutex stats_mutex;
  ovvsIvfPqSearchStatsV1 stats{};
  // Queries the bounded scan handed off to the full-table scan, over all searches.
  std::atomic<int64_t> table_queries{0};

  // One call at a time per Resources (the documented model is one Resources
  // per thread; this keeps accidental sharing safe instead of racy).
  std::mutex call_mutex;
  bool gpu_ready = false;
  int device = -1;
  hipStream_t stream = nullptr;
  static constexpr int kEvents = 6;
  hipEvent_t events[kEvents] = {};
  // Rate of the device wall clock (wall_clock64) the kernels' stage stamps read, kHz.
  double wall_khz = 1e5;
  ovvs::DeviceBuffer workspace;
  void* pinned = nullptr;
  size_t pinned_bytes = 0;
  // Entry points built on other entry points (the ScaNN search around the
  // IVF-PQ search) hold outer_mutex for the whole call and keep their own
  // buffers in outer_workspace, which the inner call does not touch.
  std::mutex outer_mutex;
  ovvs::DeviceBuffer outer_workspace;

  ~ovvsResourcesImpl();
  // Opens the current HIP device, its stream and events. Returns
  // DEVICE_UNAVAILABLE without a GPU or when the policy forces another device.
  ovvsStatus ensure_gpu();
  // Grows the device workspace (the outer workspace) to at least `bytes`.
  ovvsStatus reserve_workspace(size_t bytes, ovvs::GpuWork& work);
  ovvsStatus reserve_outer_workspace(size_t bytes, ovvs::GpuWork& work);
  // Grows the pinned host staging buffer to at least `bytes`.
  ovvsStatus reserve_pinned(size_t bytes);
};

struct ovvsIvfPqIndexImpl {
  int64_t n = 0;
  int64_t dim = 0;
  int32_t nlist = 0;
  int32_t pq_m = 0;
  int32_t pq_ks = 256;
  int32_t dsub = 0;
  ovvsMetric metric = OVVS_METRIC_L2_EXPANDED;
  std::vector<float> centroids;               // [nlist * dim]
  std::vector<float> codebooks;               // [pq_m * pq_ks * dsub]
  std::vector<uint8_t> codes;                 // [n * pq_m], by id
  std::vector<float> dataset;                 // [n * dim], by id
  std::vector<int32_t> assign;                // [n]
  std::vector<std::vector<int64_t>> lists;    // [nlist], ids in list order

  std::mutex device_mutex;
  std::unique_ptr<ovvs::IndexDevice> dev;     // created on first GPU use

  // Uploads the device mirror once (thread-safe). Validates the packed
  // invariants first (reference make_ivf_pq_packed, indexes.cpp:59-114).
  ovvsStatus ensure_device(ovvsResourcesImpl& res, ovvs::GpuWork& work);
};

namespace ovvs {
// Argument checks of ovvsIvfPqBuild after the null checks, in its order:
// INVALID_ARGUMENT for non-positive sizes or an unknown metric, SHAPE_MISMATCH
// when pq_m does not divide dim or the sizes overflow.
ovvsStatus ivf_pq_build_arg_status(int64_t n, int64_t dim, ovvsMetric metric, int32_t nlist,
                                   int32_t pq_m);
// Checks the invariants of a list layout: every id in [0, n) exactly once,
// listed under its own assignment, codes < ks (reference indexes.cpp:59-114).
bool lists_valid(const ovvsIvfPqIndexImpl& ix);
}  // namespace ovvs
