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

// Device copy of an index. Codes are list-major in the tiled block layout of
// kernels.hpp (OVVS_CODE_TILE_ROWS); ids are list-major; offsets are the list
// CSR; dataset rows are by id.
struct IndexDevice {
  int device = -1;
  int32_t code_blocks = 0;
  DeviceBuffer centroids;  // [nlist * dim] f32
  DeviceBuffer cnorm;      // [nlist] f32
  DeviceBuffer cmfma;      // centroids as split-bf16 matrix-core operands (empty if dim > 128)
  float cnorm_max = 0.f;   // max of cnorm, +inf if any is NaN or inf
  DeviceBuffer codebooks;  // [pq_m * ks * dsub] f32
  DeviceBuffer codes;      // [ceil(n / 64) * code_blocks * 512] u8
  DeviceBuffer ids;        // [n] i64
  DeviceBuffer offsets;    // [nlist + 1] i64
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

// Maps a HIP error to the ABI status.
ovvsStatus status_from_hip(hipError_t e);

}  // namespace ovvs

struct ovvsResourcesImpl {
  ovvsPolicy policy = OVVS_POLICY_AUTO;
  std::atomic<ovvsDevice> last_device{OVVS_DEVICE_CPU};
  std::atomic<ovvsDType> last_compute_dtype{OVVS_DTYPE_F32};

  std::mutex stats_mutex;
  ovvsIvfPqSearchStatsV1 stats{};

  // One call at a time per Resources (the documented model is one Resources
  // per thread; this keeps accidental sharing safe instead of racy).
  std::mutex call_mutex;
  bool gpu_ready = false;
  int device = -1;
  hipStream_t stream = nullptr;
  static constexpr int kEvents = 6;
  hipEvent_t events[kEvents] = {};
  ovvs::DeviceBuffer workspace;
  void* pinned = nullptr;
  size_t pinned_bytes = 0;

  ~ovvsResourcesImpl();
  // Opens the current HIP device, its stream and events. Returns
  // DEVICE_UNAVAILABLE without a GPU or when the policy forces another device.
  ovvsStatus ensure_gpu();
  // Grows the device workspace to at least `bytes`.
  ovvsStatus reserve_workspace(size_t bytes, ovvs::GpuWork& work);
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
// Checks the invariants of a list layout: every id in [0, n) exactly once,
// listed under its own assignment, codes < ks (reference indexes.cpp:59-114).
bool lists_valid(const ovvsIvfPqIndexImpl& ix);
}  // namespace ovvs
