// C++ RAII wrappers over the libovvs C ABI (IVF-PQ subset of the reference's
// include/ovvs/ovvs.hpp:10-127: the same class names, constructors and method
// signatures). Failures throw std::runtime_error(ovvsStatusString(status)).
#pragma once

#include <stdexcept>

#include "ovvs.h"

namespace ovvs {

inline void check(ovvsStatus s) {
  if (s != OVVS_STATUS_SUCCESS) throw std::runtime_error(ovvsStatusString(s));
}

class Resources {
 public:
  Resources() { check(ovvsResourcesCreate(&res_)); }
  ~Resources() {
    if (res_) ovvsResourcesDestroy(res_);
  }
  Resources(const Resources&) = delete;
  Resources& operator=(const Resources&) = delete;
  ovvsResources_t get() const { return res_; }
  void set_policy(ovvsPolicy p) { check(ovvsResourcesSetPolicy(res_, p)); }
  ovvsDevice last_device() const {
    ovvsDevice d = OVVS_DEVICE_CPU;
    check(ovvsResourcesLastDevice(res_, &d));
    return d;
  }
  ovvsDType last_compute_dtype() const {
    ovvsDType t = OVVS_DTYPE_F32;
    check(ovvsResourcesLastComputeDtype(res_, &t));
    return t;
  }
  ovvsIvfPqSearchStatsV1 ivf_pq_search_stats() const {
    ovvsIvfPqSearchStatsV1 s{};
    check(ovvsResourcesIvfPqSearchStatsV1(res_, &s));
    return s;
  }

 private:
  ovvsResources_t res_ = nullptr;
};

class IvfPqIndex {
 public:
  IvfPqIndex(Resources& res, const float* dataset, int64_t n, int64_t dim, ovvsMetric metric,
             int32_t nlist, int32_t pq_m, int32_t pq_nbits)
      : res_(&res) {
    check(ovvsIvfPqBuild(res.get(), dataset, n, dim, metric, nlist, pq_m, pq_nbits, &ix_));
  }
  IvfPqIndex(Resources& res, const char* path) : res_(&res) {
    check(ovvsIvfPqDeserialize(res.get(), path, &ix_));
  }
  ~IvfPqIndex() {
    if (ix_) ovvsIvfPqDestroy(ix_);
  }
  IvfPqIndex(const IvfPqIndex&) = delete;
  IvfPqIndex& operator=(const IvfPqIndex&) = delete;

  void search(const float* queries, int64_t nq, int64_t k, int32_t nprobe, int32_t krefine,
              int64_t* neighbors, float* distances, const uint8_t* bitset = nullptr) {
    check(ovvsIvfPqSearch(res_->get(), ix_, queries, nq, k, nprobe, krefine, bitset, neighbors,
                          distances));
  }
  // Additive: lookup-table precision choice (OVVS_DTYPE_F32 or OVVS_DTYPE_F16).
  void search_ex(const float* queries, int64_t nq, int64_t k, int32_t nprobe, int32_t krefine,
                 ovvsDType lut_dtype, int64_t* neighbors, float* distances,
                 const uint8_t* bitset = nullptr) {
    check(ovvsIvfPqSearchEx(res_->get(), ix_, queries, nq, k, nprobe, krefine, bitset, lut_dtype,
                            neighbors, distances));
  }
  void serialize(const char* path) { check(ovvsIvfPqSerialize(ix_, path)); }
  void extend(const float* extra, int64_t nextra) {
    check(ovvsIvfPqExtend(res_->get(), ix_, extra, nextra));
  }
  ovvsIvfPqIndex_t get() const { return ix_; }

 private:
  Resources* res_ = nullptr;
  ovvsIvfPqIndex_t ix_ = nullptr;
};

// reference include/ovvs/ovvs.hpp:221-241
class ScannIndex {
 public:
  ScannIndex(Resources& res, const float* dataset, int64_t n, int64_t dim, ovvsMetric metric,
             int32_t nlist, int32_t pq_m)
      : res_(&res) {
    check(ovvsScannBuild(res.get(), dataset, n, dim, metric, nlist, pq_m, &ix_));
  }
  ~ScannIndex() {
    if (ix_) ovvsScannDestroy(ix_);
  }
  ScannIndex(const ScannIndex&) = delete;
  ScannIndex& operator=(const ScannIndex&) = delete;
  void search(const float* queries, int64_t nq, int64_t k, int32_t nprobe, int32_t krefine,
              int64_t* neighbors, float* distances) {
    check(ovvsScannSearch(res_->get(), ix_, queries, nq, k, nprobe, krefine, neighbors, distances));
  }

 private:
  Resources* res_ = nullptr;
  ovvsScannIndex_t ix_ = nullptr;
};

}  // namespace ovvs
