// scann_index.cpp — the ScaNN-style index of the C ABI: IVF-PQ trained on column-scaled
// rows, searched with scaled queries and re-ranked on the original rows
// (reference src/neighbors/graphs.cpp:474-478, 3286-3385).
//
// Build: the rows go to the device once; the column factors (k_column_aniso), the
// scaled rows and the row norms of the re-rank are computed there, and the scaled
// rows feed ovvsIvfPqBuild. Search: queries are scaled on the device, the IVF-PQ
// search runs on device buffers (ovvsIvfPqSearchDevice, krefine results), and the
// re-rank is the IVF-PQ refine kernel over the returned ids with the original rows.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstring>
#include <limits>
#include <memory>
#include <mutex>
#include <vector>

#include "internal.hpp"
#include "kernels.hpp"

using ovvs::DeviceBuffer;
using ovvs::GpuWork;

struct ovvsScannIndexImpl {
  int64_t n = 0;
  int64_t dim = 0;
  ovvsMetric metric = OVVS_METRIC_L2_EXPANDED;
  std::vector<float> rows;   // [n * dim] the original rows (reference Dataset copy)
  std::vector<float> aniso;  // [dim] column factors
  ovvsIvfPqIndex_t pq = nullptr;  // IVF-PQ over the scaled rows

  // Device mirror: original rows, their squared norms and the column factors.
  std::mutex device_mutex;
  int device = -1;
  DeviceBuffer d_rows, d_rnorm, d_aniso;

  ~ovvsScannIndexImpl() {
    if (pq) ovvsIvfPqDestroy(pq);
  }
  ovvsStatus ensure_device(ovvsResourcesImpl& res, GpuWork& work);
};

namespace {

#define SCANN_TRY(expr)                             \
  do {                                              \
    const ovvsStatus st_ = (expr);                  \
    if (st_ != OVVS_STATUS_SUCCESS) return st_;     \
  } while (0)

#define SCANN_HIP(expr)                             \
  do {                                              \
    const hipError_t hip_e_ = (expr);               \
    if (hip_e_ != hipSuccess) {                     \
      (void)hipGetLastError();                      \
      return ovvs::status_from_hip(hip_e_);         \
    }                                               \
  } while (0)

size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

ovvsStatus alloc(DeviceBuffer& b, size_t bytes, GpuWork& work) {
  if (b.allocate(bytes) != hipSuccess) {
    (void)hipGetLastError();
    return OVVS_STATUS_OOM;
  }
  ovvs::saturating_add(work.allocation_calls, 1);
  ovvs::saturating_add(work.allocation_bytes, static_cast<int64_t>(bytes));
  return OVVS_STATUS_SUCCESS;
}

struct Carver {
  unsigned char* p;
  template <class T>
  T* take(size_t count) {
    T* r = reinterpret_cast<T*>(p);
    p += align256(count * sizeof(T));
    return r;
  }
};

}  // namespace

ovvsStatus ovvsScannIndexImpl::ensure_device(ovvsResourcesImpl& res, GpuWork& work) {
  std::lock_guard<std::mutex> lock(device_mutex);
  if (device == res.device && d_rows.get()) return OVVS_STATUS_SUCCESS;
  hipStream_t s = res.stream;
  const size_t bytes = static_cast<size_t>(n) * static_cast<size_t>(dim) * 4;
  SCANN_TRY(alloc(d_rows, bytes, work));
  SCANN_TRY(alloc(d_rnorm, static_cast<size_t>(n) * 4, work));
  SCANN_TRY(alloc(d_aniso, static_cast<size_t>(dim) * 4, work));
  SCANN_HIP(hipMemcpyAsync(d_rows.get(), rows.data(), bytes, hipMemcpyHostToDevice, s));
  SCANN_HIP(hipMemcpyAsync(d_aniso.get(), aniso.data(), aniso.size() * 4, hipMemcpyHostToDevice, s));
  SCANN_HIP(ovvs_hip_row_norms(d_rows.as<float>(), n, static_cast<int32_t>(dim), d_rnorm.as<float>(), s));
  SCANN_HIP(hipStreamSynchronize(s));
  device = res.device;
  return OVVS_STATUS_SUCCESS;
}

extern "C" {

OVVS_API ovvsStatus ovvsScannBuild(ovvsResources_t res, const float* dataset, int64_t n,
                                   int64_t dim, ovvsMetric metric, int32_t nlist, int32_t pq_m,
                                   ovvsScannIndex_t* index) {
  if (!res || !dataset || !index) return OVVS_STATUS_INVALID_ARGUMENT;
  // The inner build's own argument checks, before any GPU work.
  SCANN_TRY(ovvs::ivf_pq_build_arg_status(n, dim, metric, nlist, pq_m));
  try {
    auto sx = std::make_unique<ovvsScannIndexImpl>();
    sx->n = n;
    sx->dim = dim;
    sx->metric = metric;
    const size_t count = static_cast<size_t>(n) * static_cast<size_t>(dim);
    sx->rows.assign(dataset, dataset + count);
    sx->aniso.resize(static_cast<size_t>(dim));
    std::vector<float> scaled(count);
    {
      std::lock_guard<std::mutex> lock(res->call_mutex);
      SCANN_TRY(res->ensure_gpu());
      GpuWork work;
      hipStream_t s = res->stream;
      const int32_t d32 = static_cast<int32_t>(dim);
      DeviceBuffer d_scaled;
      SCANN_TRY(alloc(sx->d_rows, count * 4, work));
      SCANN_TRY(alloc(sx->d_rnorm, static_cast<size_t>(n) * 4, work));
      SCANN_TRY(alloc(sx->d_aniso, static_cast<size_t>(dim) * 4, work));
      SCANN_TRY(alloc(d_scaled, count * 4, work));
      SCANN_HIP(hipMemcpyAsync(sx->d_rows.get(), dataset, count * 4, hipMemcpyHostToDevice, s));
      SCANN_HIP(ovvs_hip_column_aniso(sx->d_rows.as<float>(), n, d32, sx->d_aniso.as<float>(), s));
      SCANN_HIP(ovvs_hip_scale_columns(sx->d_rows.as<float>(), n, d32, sx->d_aniso.as<float>(),
                                       d_scaled.as<float>(), s));
      SCANN_HIP(ovvs_hip_row_norms(sx->d_rows.as<float>(), n, d32, sx->d_rnorm.as<float>(), s));
      SCANN_HIP(hipMemcpyAsync(sx->aniso.data(), sx->d_aniso.get(), sx->aniso.size() * 4,
                               hipMemcpyDeviceToHost, s));
      SCANN_HIP(hipMemcpyAsync(scaled.data(), d_scaled.get(), count * 4, hipMemcpyDeviceToHost, s));
      SCANN_HIP(hipStreamSynchronize(s));
      sx->device = res->device;
    }
    SCANN_TRY(ovvsIvfPqBuild(res, scaled.data(), n, dim, metric, nlist, pq_m, 8, &sx->pq));
    *index = sx.release();
    return OVVS_STATUS_SUCCESS;
  } catch (const std::bad_alloc&) {
    return OVVS_STATUS_OOM;
  } catch (...) {
    return OVVS_STATUS_ERROR;
  }
}

OVVS_API ovvsStatus ovvsScannSearch(ovvsResources_t res, ovvsScannIndex_t index,
                                    const float* queries, int64_t nq, int64_t k, int32_t nprobe,
                                    int32_t krefine, int64_t* neighbors, float* distances) {
  if (!res || !index || !queries || !neighbors || !distances) return OVVS_STATUS_INVALID_ARGUMENT;
  // krefine := max(krefine, (int32)k) (reference graphs.cpp:3323); the inner search
  // is asked for krefine results, so its checks apply to nq and krefine.
  if (k > std::numeric_limits<int32_t>::max()) return OVVS_STATUS_INVALID_ARGUMENT;
  const int32_t R = std::max(krefine, static_cast<int32_t>(k));
  if (nq <= 0 || R <= 0) return OVVS_STATUS_INVALID_ARGUMENT;
  if (R > OVVS_HIP_MAX_REFINE || nq > 0x7fffffff) return OVVS_STATUS_DEVICE_UNAVAILABLE;
  ovvsScannIndexImpl& sx = *index;
  const int32_t dim = static_cast<int32_t>(sx.dim);
  const int64_t kk = k > 0 ? k : 0;
  try {
    std::lock_guard<std::mutex> outer(res->outer_mutex);
    GpuWork work;
    float *d_q, *d_qs, *d_qn, *d_cdist, *d_odist;
    int64_t *d_cid, *d_oid;
    int32_t *d_spos, *d_scnt;
    unsigned long long* d_bad;
    const size_t nqR = static_cast<size_t>(nq) * static_cast<size_t>(R);
    const size_t nqk = static_cast<size_t>(nq) * static_cast<size_t>(kk);
    {
      std::lock_guard<std::mutex> lock(res->call_mutex);
      SCANN_TRY(res->ensure_gpu());
      SCANN_TRY(sx.ensure_device(*res, work));
      hipStream_t s = res->stream;
      const size_t qf = static_cast<size_t>(nq) * static_cast<size_t>(dim);
      const size_t need = 2 * align256(qf * 4) + align256(static_cast<size_t>(nq) * 4) +
                          align256(nqR * 8) + align256(nqR * 4) + align256(nqR * 4) +
                          align256(static_cast<size_t>(nq) * 4) + align256(nqk * 8) +
                          align256(nqk * 4) + align256(8);
      SCANN_TRY(res->reserve_outer_workspace(need, work));
      Carver cv{static_cast<unsigned char*>(res->outer_workspace.get())};
      d_q = cv.take<float>(qf);
      d_qs = cv.take<float>(qf);
      d_qn = cv.take<float>(static_cast<size_t>(nq));
      d_cid = cv.take<int64_t>(nqR);
      d_cdist = cv.take<float>(nqR);
      d_spos = cv.take<int32_t>(nqR);
      d_scnt = cv.take<int32_t>(static_cast<size_t>(nq));
      d_oid = cv.take<int64_t>(nqk);
      d_odist = cv.take<float>(nqk);
      d_bad = cv.take<unsigned long long>(1);
      SCANN_HIP(hipMemcpyAsync(d_q, queries, qf * 4, hipMemcpyHostToDevice, s));
      SCANN_HIP(ovvs_hip_scale_columns(d_q, nq, dim, sx.d_aniso.as<float>(), d_qs, s));
      SCANN_HIP(ovvs_hip_row_norms(d_q, nq, dim, d_qn, s));
    }
    // IVF-PQ search of the scaled queries (its own lock, workspace and telemetry).
    SCANN_TRY(ovvsIvfPqSearchDevice(res, sx.pq, d_qs, nq, R, nprobe, R, nullptr, OVVS_DTYPE_F32,
                                    d_cid, d_cdist));
    if (kk == 0) return OVVS_STATUS_SUCCESS;

    std::lock_guard<std::mutex> lock(res->call_mutex);
    hipStream_t s = res->stream;
    SCANN_HIP(hipMemsetAsync(d_bad, 0, 8, s));
    // Shortlist positions are int32 flat indexes into each chunk's results.
    const int64_t qc = std::max<int64_t>(1, 0x7fffffff / R);
    for (int64_t q0 = 0; q0 < nq; q0 += qc) {
      const int64_t cnt = std::min(qc, nq - q0);
      SCANN_HIP(ovvs_hip_ids_shortlist(d_cid + q0 * R, cnt, R, sx.n, d_spos + q0 * R, d_scnt + q0, s));
      OvvsRefineArgs ra{};
      ra.queries = d_q + q0 * dim;
      ra.qnorm = d_qn + q0;
      ra.nq = cnt;
      ra.dim = dim;
      ra.metric = static_cast<int32_t>(sx.metric);
      ra.dataset = sx.d_rows.as<float>();
      ra.xnorm = sx.d_rnorm.as<float>();
      ra.n = sx.n;
      ra.positions = cnt * R;
      ra.ids = d_cid + q0 * R;
      ra.K = R;
      ra.short_pos = d_spos + q0 * R;
      ra.short_count = d_scnt + q0;
      ra.k = kk;
      ra.out_ids = d_oid + q0 * kk;
      ra.out_dist = d_odist + q0 * kk;
      ra.invalid = d_bad;
      SCANN_HIP(ovvs_hip_refine(&ra, s));
    }
    std::vector<int64_t> ids(nqk);
    std::vector<float> dist(nqk);
    unsigned long long bad = 0;
    SCANN_HIP(hipMemcpyAsync(ids.data(), d_oid, nqk * 8, hipMemcpyDeviceToHost, s));
    SCANN_HIP(hipMemcpyAsync(dist.data(), d_odist, nqk * 4, hipMemcpyDeviceToHost, s));
    SCANN_HIP(hipMemcpyAsync(&bad, d_bad, 8, hipMemcpyDeviceToHost, s));
    SCANN_HIP(hipStreamSynchronize(s));
    if (bad != 0) return OVVS_STATUS_ERROR;
    std::memcpy(neighbors, ids.data(), nqk * 8);
    std::memcpy(distances, dist.data(), nqk * 4);
    res->last_device = OVVS_DEVICE_GPU;
    return OVVS_STATUS_SUCCESS;
  } catch (const std::bad_alloc&) {
    return OVVS_STATUS_OOM;
  } catch (...) {
    return OVVS_STATUS_ERROR;
  }
}

OVVS_API ovvsStatus ovvsScannDestroy(ovvsScannIndex_t index) {
  delete index;
  return OVVS_STATUS_SUCCESS;
}

}  // extern "C"
