// noalloc.hip — ovvsIvfPqSearchDeviceNoAlloc: the device-pointer IVF-PQ search for
// callers that cannot allocate memory (no hipMalloc, hipFree or pinned host
// allocation on the call path).
//
// The search's workspace (query norms, probes, probe fallback flags, the scan's
// query order, shortlists, per-query statistics, counters and a chunk of coarse
// scores) is carved from `scratch`, a fixed device array of the library's code
// object: every GPU holds its own copy from the time the library's code is loaded
// on it until the process ends. Its device address is looked up once per device
// with hipGetSymbolAddress and used for every kernel argument; the array's name is
// never used in host code otherwise (in host code it names a host-side stand-in,
// not device memory).
//
// Calls on one GPU share that GPU's array: the library runs them one at a time
// (a per-device mutex held for the whole call, which returns only after the
// search's last kernel has finished). The array keeps the last call's contents;
// everything the search needs cleared (its counters) is cleared by the search's
// own first kernel.
#include <hip/hip_runtime.h>

#include <mutex>

#include "internal.hpp"

namespace {

constexpr size_t kScratchBytes = OVVS_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch must hold whole 256-byte slots");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;

struct DeviceScratch {
  std::once_flag once;
  void* ptr = nullptr;  // device address of this device's copy of scratch
  hipError_t lookup = hipSuccess;
  std::mutex call;      // one call at a time on this device
};

DeviceScratch g_scratch[kMaxDevices];

// Device address of `scratch` on device dev (looked up once, with dev current).
void* scratch_on(int dev, hipError_t* err) {
  DeviceScratch& d = g_scratch[dev];
  std::call_once(d.once, [&d, dev] {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) cur = -1;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) {
      d.lookup = hipErrorInvalidDevice;
      (void)hipGetLastError();
      return;
    }
    void* p = nullptr;
    d.lookup = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (d.lookup == hipSuccess && p != nullptr) {
      d.ptr = p;
    } else {
      if (d.lookup == hipSuccess) d.lookup = hipErrorInvalidSymbol;
      (void)hipGetLastError();
    }
    if (cur >= 0 && cur != dev) (void)hipSetDevice(cur);
  });
  *err = d.lookup;
  return d.ptr;
}

}  // namespace

extern "C" OVVS_API ovvsStatus ovvsIvfPqSearchDeviceNoAlloc(
    ovvsResources_t res, ovvsIvfPqIndex_t index, const float* queries, int64_t nq, int64_t k,
    int32_t nprobe, int32_t krefine, const uint8_t* bitset, ovvsDType lut_dtype,
    int64_t* neighbors, float* distances) {
  if (!res || !index || !queries || !neighbors || !distances || nq <= 0 || k <= 0) {
    return OVVS_STATUS_INVALID_ARGUMENT;
  }
  int dev = -1;
  {
    // First call on this Resources: open its stream and events (set-up, as on the
    // first call of every other entry point).
    std::lock_guard<std::mutex> lock(res->call_mutex);
    const ovvsStatus st = res->ensure_gpu();
    if (st != OVVS_STATUS_SUCCESS) return st;
    dev = res->device;
  }
  if (dev < 0 || dev >= kMaxDevices) return OVVS_STATUS_DEVICE_UNAVAILABLE;
  hipError_t err = hipSuccess;
  void* ptr = scratch_on(dev, &err);
  if (!ptr) return ovvs::status_from_hip(err) == OVVS_STATUS_OOM ? OVVS_STATUS_OOM
                                                                  : OVVS_STATUS_DEVICE_UNAVAILABLE;
  std::lock_guard<std::mutex> one(g_scratch[dev].call);
  return ovvs::ivf_pq_search_scratch(res, index, queries, nq, k, nprobe, krefine, bitset,
                                     lut_dtype, neighbors, distances, ptr, kScratchBytes);
}
