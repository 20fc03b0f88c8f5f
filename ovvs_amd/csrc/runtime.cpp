// runtime.cpp — Resources, status strings, version, bitset helper and the
// device-memory plumbing shared by the IVF-PQ entry points.
//
// Reference counterparts: src/rt/resources.cpp:14-147,218-229 and
// src/rt/status.cpp:1-29. The reference's Resources carries SYCL queues, NPU
// state, probe tables and CAGRA counters; this one carries what the IVF-PQ path
// on one MI355X needs: a HIP stream, a grow-only device workspace, pinned host
// staging, timing events and the IVF-PQ telemetry.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <limits>
#include <mutex>
#include <new>
#include <thread>

#include "internal.hpp"

namespace ovvs {

hipError_t DeviceBuffer::allocate(size_t bytes) {
  reset();
  if (bytes == 0) return hipSuccess;
  void* p = nullptr;
  const hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) return e;
  ptr_ = p;
  bytes_ = bytes;
  return hipSuccess;
}

void DeviceBuffer::reset() {
  if (ptr_) (void)hipFree(ptr_);
  ptr_ = nullptr;
  bytes_ = 0;
}

void saturating_add(int64_t& value, int64_t delta) noexcept {
  if (delta <= 0) return;
  if (value > std::numeric_limits<int64_t>::max() - delta) {
    value = std::numeric_limits<int64_t>::max();
  } else {
    value += delta;
  }
}

bool gpu_present() {
  static const bool present = [] {
    int count = 0;
    return hipGetDeviceCount(&count) == hipSuccess && count > 0;
  }();
  return present;
}

namespace {

// Worker threads that split host copies between them. A copy is cut into parts;
// the caller and the workers claim parts from one counter that also carries the
// copy's sequence number, so a worker that wakes late cannot claim a part of a
// copy that has already finished.
class CopyPool {
 public:
  static CopyPool& instance() {
    // Never destroyed: its detached workers may be blocked on the condition
    // variable when the process exits.
    static CopyPool* pool = new CopyPool();
    return *pool;
  }

  void copy(void* dst, const void* src, size_t bytes) {
    if (bytes < kMinSplit || workers_ == 0) {
      std::memcpy(dst, src, bytes);
      return;
    }
    std::unique_lock<std::mutex> one(busy_, std::try_to_lock);
    if (!one.owns_lock()) {
      std::memcpy(dst, src, bytes);
      return;
    }
    const size_t parts = std::min<size_t>(4 * (workers_ + 1), (bytes + kMinPart - 1) / kMinPart);
    {
      std::lock_guard<std::mutex> lk(m_);
      job_.dst = static_cast<unsigned char*>(dst);
      job_.src = static_cast<const unsigned char*>(src);
      job_.bytes = bytes;
      job_.parts = static_cast<uint32_t>(parts);
      job_.part = (bytes + parts - 1) / parts;
      ++seq_;
      job_.seq = seq_;
      left_.store(static_cast<uint32_t>(parts));
      next_.store(static_cast<uint64_t>(seq_) << 32);
    }
    wake_.notify_all();
    Job mine;
    {
      std::lock_guard<std::mutex> lk(m_);
      mine = job_;
    }
    run(mine);
    std::unique_lock<std::mutex> lk(m_);
    done_.wait(lk, [&] { return left_.load() == 0; });
  }

 private:
  static constexpr size_t kMinSplit = size_t(256) << 10;
  static constexpr size_t kMinPart = size_t(64) << 10;

  struct Job {
    unsigned char* dst = nullptr;
    const unsigned char* src = nullptr;
    size_t bytes = 0;
    size_t part = 0;
    uint32_t parts = 0;
    uint32_t seq = 0;
  };

  CopyPool() {
    const unsigned hw = std::thread::hardware_concurrency();
    workers_ = hw > 1 ? std::min(6u, hw - 1) : 0u;
    for (unsigned i = 0; i < workers_; ++i) std::thread([this] { loop(); }).detach();
  }

  void loop() {
    uint32_t seen = 0;
    for (;;) {
      Job j;
      {
        std::unique_lock<std::mutex> lk(m_);
        wake_.wait(lk, [&] { return seq_ != seen; });
        seen = seq_;
        j = job_;
      }
      run(j);
    }
  }

  // Claims and copies parts of copy j until none is left (or j has ended).
  void run(const Job& j) {
    for (;;) {
      uint64_t v = next_.load();
      uint32_t i;
      do {
        if (static_cast<uint32_t>(v >> 32) != j.seq) return;
        i = static_cast<uint32_t>(v);
        if (i >= j.parts) return;
      } while (!next_.compare_exchange_weak(v, v + 1));
      const size_t off = static_cast<size_t>(i) * j.part;
      if (off < j.bytes) std::memcpy(j.dst + off, j.src + off, std::min(j.part, j.bytes - off));
      if (left_.fetch_sub(1) == 1) {
        std::lock_guard<std::mutex> lk(m_);
        done_.notify_all();
      }
    }
  }

  unsigned workers_ = 0;
  std::mutex busy_;  // one copy at a time
  std::mutex m_;
  std::condition_variable wake_, done_;
  Job job_;
  uint32_t seq_ = 0;
  std::atomic<uint64_t> next_{0};  // sequence << 32 | next part
  std::atomic<uint32_t> left_{0};  // parts not yet copied
};

}  // namespace

void parallel_copy(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return;
  CopyPool::instance().copy(dst, src, bytes);
}

ovvsStatus status_from_hip(hipError_t e) {
  switch (e) {
    case hipSuccess:
      return OVVS_STATUS_SUCCESS;
    case hipErrorOutOfMemory:
      return OVVS_STATUS_OOM;
    case hipErrorNoDevice:
    case hipErrorInvalidDevice:
      return OVVS_STATUS_DEVICE_UNAVAILABLE;
    default:
      return OVVS_STATUS_ERROR;
  }
}

}  // namespace ovvs

ovvsResourcesImpl::~ovvsResourcesImpl() {
  if (gpu_ready) {
    (void)hipStreamSynchronize(stream);
    for (hipEvent_t& e : events) {
      if (e) (void)hipEventDestroy(e);
    }
    workspace.reset();
    outer_workspace.reset();
    if (pinned) (void)hipHostFree(pinned);
    (void)hipStreamDestroy(stream);
  }
}

ovvsStatus ovvsResourcesImpl::ensure_gpu() {
  if (policy == OVVS_POLICY_FORCE_CPU || policy == OVVS_POLICY_FORCE_NPU) {
    return OVVS_STATUS_DEVICE_UNAVAILABLE;
  }
  if (gpu_ready) return OVVS_STATUS_SUCCESS;
  if (!ovvs::gpu_present()) return OVVS_STATUS_DEVICE_UNAVAILABLE;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return OVVS_STATUS_DEVICE_UNAVAILABLE;
  hipStream_t s = nullptr;
  // Default stream priority, non-blocking with respect to the null stream.
  if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
    return OVVS_STATUS_DEVICE_UNAVAILABLE;
  }
  hipEvent_t ev[kEvents] = {};
  for (int i = 0; i < kEvents; ++i) {
    // Stage timing only (read after the stream is synchronized): no system-scope
    // fence when recorded, which would write back and invalidate caches mid-search.
    if (hipEventCreateWithFlags(&ev[i], hipEventDisableSystemFence) != hipSuccess) {
      for (int j = 0; j < i; ++j) (void)hipEventDestroy(ev[j]);
      (void)hipStreamDestroy(s);
      return OVVS_STATUS_DEVICE_UNAVAILABLE;
    }
  }
  int khz = 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) == hipSuccess && khz > 0) {
    wall_khz = khz;
  } else {
    (void)hipGetLastError();
  }
  device = dev;
  stream = s;
  for (int i = 0; i < kEvents; ++i) events[i] = ev[i];
  gpu_ready = true;
  return OVVS_STATUS_SUCCESS;
}

namespace {

ovvsStatus grow_buffer(ovvs::DeviceBuffer& buf, size_t bytes, hipStream_t stream,
                       ovvs::GpuWork& work) {
  if (buf.size() >= bytes) return OVVS_STATUS_SUCCESS;
  (void)hipStreamSynchronize(stream);
  // Grow geometrically so repeated calls with slowly growing batches settle.
  size_t want = buf.size() * 2;
  if (want < bytes) want = bytes;
  hipError_t e = buf.allocate(want);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    e = buf.allocate(bytes);
    want = bytes;
  }
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return OVVS_STATUS_OOM;
  }
  ovvs::saturating_add(work.allocation_calls, 1);
  ovvs::saturating_add(work.allocation_bytes, static_cast<int64_t>(want));
  return OVVS_STATUS_SUCCESS;
}

}  // namespace

ovvsStatus ovvsResourcesImpl::reserve_workspace(size_t bytes, ovvs::GpuWork& work) {
  return grow_buffer(workspace, bytes, stream, work);
}

ovvsStatus ovvsResourcesImpl::reserve_outer_workspace(size_t bytes, ovvs::GpuWork& work) {
  return grow_buffer(outer_workspace, bytes, stream, work);
}

ovvsStatus ovvsResourcesImpl::reserve_pinned(size_t bytes) {
  if (pinned_bytes >= bytes) return OVVS_STATUS_SUCCESS;
  (void)hipStreamSynchronize(stream);
  if (pinned) (void)hipHostFree(pinned);
  pinned = nullptr;
  pinned_bytes = 0;
  size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
  void* p = nullptr;
  if (hipHostMalloc(&p, want, hipHostMallocDefault) != hipSuccess) {
    (void)hipGetLastError();
    return OVVS_STATUS_OOM;
  }
  pinned = p;
  pinned_bytes = want;
  return OVVS_STATUS_SUCCESS;
}

extern "C" {

OVVS_API const char* ovvsGetVersion(void) { return OVVS_VERSION_STRING; }

OVVS_API const char* ovvsStatusString(ovvsStatus status) {
  switch (status) {
    case OVVS_STATUS_SUCCESS:
      return "success";
    case OVVS_STATUS_ERROR:
      return "error";
    case OVVS_STATUS_INVALID_ARGUMENT:
      return "invalid argument";
    case OVVS_STATUS_UNSUPPORTED:
      return "unsupported";
    case OVVS_STATUS_OOM:
      return "out of memory";
    case OVVS_STATUS_COMPILE_FAIL:
      return "compile fail";
    case OVVS_STATUS_SHAPE_MISMATCH:
      return "shape mismatch";
    case OVVS_STATUS_DEVICE_UNAVAILABLE:
      return "device unavailable";
    case OVVS_STATUS_IO:
      return "io error";
  }
  return "unknown";
}

OVVS_API ovvsStatus ovvsResourcesCreate(ovvsResources_t* res) {
  if (!res) return OVVS_STATUS_INVALID_ARGUMENT;
  auto* r = new (std::nothrow) ovvsResourcesImpl();
  if (!r) return OVVS_STATUS_OOM;
  *res = r;
  return OVVS_STATUS_SUCCESS;
}

OVVS_API ovvsStatus ovvsResourcesDestroy(ovvsResources_t res) {
  delete res;
  return OVVS_STATUS_SUCCESS;
}

OVVS_API ovvsStatus ovvsResourcesSetPolicy(ovvsResources_t res, ovvsPolicy policy) {
  if (!res) return OVVS_STATUS_INVALID_ARGUMENT;
  res->policy = policy;
  return OVVS_STATUS_SUCCESS;
}

OVVS_API ovvsStatus ovvsResourcesGetPolicy(ovvsResources_t res, ovvsPolicy* policy) {
  if (!res || !policy) return OVVS_STATUS_INVALID_ARGUMENT;
  *policy = res->policy;
  return OVVS_STATUS_SUCCESS;
}

OVVS_API ovvsStatus ovvsResourcesNpuAvailable(ovvsResources_t res, int32_t* available) {
  if (!res || !available) return OVVS_STATUS_INVALID_ARGUMENT;
  *available = 0;
  return OVVS_STATUS_SUCCESS;
}

OVVS_API ovvsStatus ovvsResourcesGpuAvailable(ovvsResources_t res, int32_t* available) {
  if (!res || !available) return OVVS_STATUS_INVALID_ARGUMENT;
  *available = ovvs::gpu_present() ? 1 : 0;
  return OVVS_STATUS_SUCCESS;
}

OVVS_API ovvsStatus ovvsResourcesSku(ovvsResources_t res, char* buf, int32_t len) {
  if (!res || !buf || len <= 0) return OVVS_STATUS_INVALID_ARGUMENT;
  const char* sku = "generic-cpu";
  char name[256] = {0};
  if (ovvs::gpu_present()) {
    hipDeviceProp_t prop;
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess) {
      std::snprintf(name, sizeof(name), "%s", prop.gcnArchName);
      sku = name;
    }
  }
  std::snprintf(buf, static_cast<size_t>(len), "%s", sku);
  return OVVS_STATUS_SUCCESS;
}

OVVS_API ovvsStatus ovvsResourcesLastDevice(ovvsResources_t res, ovvsDevice* device) {
  if (!res || !device) return OVVS_STATUS_INVALID_ARGUMENT;
  *device = res->last_device.load();
  return OVVS_STATUS_SUCCESS;
}

OVVS_API ovvsStatus ovvsResourcesLastComputeDtype(ovvsResources_t res, ovvsDType* dtype) {
  if (!res || !dtype) return OVVS_STATUS_INVALID_ARGUMENT;
  *dtype = res->last_compute_dtype.load();
  return OVVS_STATUS_SUCCESS;
}

OVVS_API ovvsStatus ovvsResourcesIvfPqSearchStatsV1(ovvsResources_t res,
                                                    ovvsIvfPqSearchStatsV1* stats) {
  if (!res || !stats) return OVVS_STATUS_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lock(res->stats_mutex);
  *stats = res->stats;
  stats->abi_version = OVVS_IVF_PQ_SEARCH_STATS_ABI_V1;
  stats->struct_size = static_cast<uint32_t>(sizeof(*stats));
  return OVVS_STATUS_SUCCESS;
}

OVVS_API ovvsStatus ovvsResourcesIvfPqTableQueries(ovvsResources_t res, int64_t* count) {
  if (!res || !count) return OVVS_STATUS_INVALID_ARGUMENT;
  *count = res->table_queries.load();
  return OVVS_STATUS_SUCCESS;
}

OVVS_API ovvsStatus ovvsBitsetFromAllowList(int64_t n, const int64_t* ids, int64_t nids,
                                            uint8_t* bitset) {
  if (!bitset || n <= 0 || nids < 0) return OVVS_STATUS_INVALID_ARGUMENT;
  const int64_t nbytes = n / 8 + (n % 8 != 0 ? 1 : 0);
  std::memset(bitset, 0, static_cast<size_t>(nbytes));
  if (!ids) return OVVS_STATUS_SUCCESS;
  for (int64_t i = 0; i < nids; ++i) {
    const int64_t id = ids[i];
    if (id >= 0 && id < n) bitset[id / 8] = static_cast<uint8_t>(bitset[id / 8] | (1u << (id % 8)));
  }
  return OVVS_STATUS_SUCCESS;
}

}  // extern "C"

static_assert(sizeof(ovvsIvfPqSearchStatsV1) == 200, "ovvsIvfPqSearchStatsV1 is a 200-byte ABI");
