// knn_graph_index.cpp — the IVF-PQ k-nearest-neighbour graph of the C ABI (additive): the
// CAGRA build's IVF-PQ initializer (reference src/neighbors/graphs.cpp:767-797).
//
// The reference builds a small IVF-PQ index over the rows (nlist = max(2, min(8, n/4)),
// pq_m = the largest divisor of dim not above 4, 8-bit codes) and searches every row on
// its own for degree + 1 neighbours with every list probed and krefine = degree + 1,
// then keeps the results other than the row itself and -1. Here the same build runs
// on the GPU and the searches run as batches of rows taken from the index's device copy
// of the dataset (a batch's results are those of the same rows searched one at a time),
// followed by the list assembly kernel.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstring>
#include <limits>
#include <mutex>
#include <vector>

#include "internal.hpp"
#include "kernels.hpp"

namespace {

#define KNN_TRY(expr)                               \
  do {                                              \
    const ovvsStatus st_ = (expr);                  \
    if (st_ != OVVS_STATUS_SUCCESS) return st_;     \
  } while (0)

#define KNN_HIP(expr)                               \
  do {                                              \
    const hipError_t hip_e_ = (expr);               \
    if (hip_e_ != hipSuccess) {                     \
      (void)hipGetLastError();                      \
      return ovvs::status_from_hip(hip_e_);         \
    }                                               \
  } while (0)

constexpr int64_t kRowsPerBatch = 65536;

size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

struct IndexGuard {
  ovvsIvfPqIndex_t value = nullptr;
  ~IndexGuard() {
    if (value) (void)ovvsIvfPqDestroy(value);
  }
};

}  // namespace

extern "C" {

OVVS_API ovvsStatus ovvsIvfPqKnnGraph(ovvsResources_t res, const float* dataset, int64_t n,
                                      int64_t dim, ovvsMetric metric, int32_t degree,
                                      int32_t* graph) {
  if (!res || !dataset || !graph || degree < 0) return OVVS_STATUS_INVALID_ARGUMENT;
  // reference graphs.cpp:770-777
  const int32_t nlist = static_cast<int32_t>(std::max<int64_t>(2, std::min<int64_t>(8, n / 4)));
  int32_t pq_m = 1;
  for (int64_t c = std::min<int64_t>(4, dim); c >= 1; --c) {
    if (dim % c == 0) {
      pq_m = static_cast<int32_t>(c);
      break;
    }
  }
  if (degree >= OVVS_HIP_MAX_REFINE) return OVVS_STATUS_DEVICE_UNAVAILABLE;
  if (n > 0 && static_cast<uint64_t>(n) >
                   std::numeric_limits<size_t>::max() / 8 / (static_cast<uint64_t>(degree) + 1))
    return OVVS_STATUS_SHAPE_MISMATCH;
  try {
    std::lock_guard<std::mutex> outer(res->outer_mutex);
    IndexGuard pq;
    KNN_TRY(ovvsIvfPqBuild(res, dataset, n, dim, metric, nlist, pq_m, 8, &pq.value));
    if (degree == 0) return OVVS_STATUS_SUCCESS;
    const int64_t k = static_cast<int64_t>(degree) + 1;
    const int64_t qc = std::min(kRowsPerBatch, n);
    const float* rows = nullptr;
    int64_t* d_nb = nullptr;
    float* d_ds = nullptr;
    int32_t* d_graph = nullptr;
    const size_t gcount = static_cast<size_t>(n) * static_cast<size_t>(degree);
    {
      std::lock_guard<std::mutex> lock(res->call_mutex);
      KNN_TRY(res->ensure_gpu());
      ovvs::GpuWork work;
      KNN_TRY(pq.value->ensure_device(*res, work));
      rows = pq.value->dev->dataset.as<float>();
      const size_t nk = static_cast<size_t>(qc) * static_cast<size_t>(k);
      KNN_TRY(res->reserve_outer_workspace(align256(nk * 8) + align256(nk * 4) + align256(gcount * 4),
                                           work));
      unsigned char* p = static_cast<unsigned char*>(res->outer_workspace.get());
      d_nb = reinterpret_cast<int64_t*>(p);
      d_ds = reinterpret_cast<float*>(p + align256(nk * 8));
      d_graph = reinterpret_cast<int32_t*>(p + align256(nk * 8) + align256(nk * 4));
    }
    for (int64_t q0 = 0; q0 < n; q0 += qc) {
      const int64_t cnt = std::min(qc, n - q0);
      KNN_TRY(ovvsIvfPqSearchDevice(res, pq.value, rows + q0 * dim, cnt, k, nlist,
                                    static_cast<int32_t>(k), nullptr, OVVS_DTYPE_F32, d_nb, d_ds));
      std::lock_guard<std::mutex> lock(res->call_mutex);
      KNN_HIP(ovvs_hip_knn_graph_rows(d_nb, cnt, q0, degree, d_graph, res->stream));
    }
    std::vector<int32_t> out(gcount);
    {
      std::lock_guard<std::mutex> lock(res->call_mutex);
      KNN_HIP(hipMemcpyAsync(out.data(), d_graph, gcount * 4, hipMemcpyDeviceToHost, res->stream));
      KNN_HIP(hipStreamSynchronize(res->stream));
    }
    std::memcpy(graph, out.data(), gcount * 4);
    res->last_device = OVVS_DEVICE_GPU;
    return OVVS_STATUS_SUCCESS;
  } catch (const std::bad_alloc&) {
    return OVVS_STATUS_OOM;
  } catch (...) {
    return OVVS_STATUS_ERROR;
  }
}

}  // extern "C"
