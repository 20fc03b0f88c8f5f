// ivf_pq_index.cpp — IVF-PQ index lifecycle: build and extend on the GPU,
// IPQ1 v1 serialize/deserialize, destroy, and the device mirror.
//
// Reference counterparts (src/neighbors/indexes.cpp):
//   ovvsIvfPqBuild        :459-536  (k-means 12 iterations, L2 assignment,
//                                    residuals, per-subspace PQ k-means 8
//                                    iterations, first-minimum encoding)
//   kmeans_fit_impl       src/prim/mixer.cpp:866-921 (mt19937(42) seeding,
//                                    exact L2 assignment, row-order mean update)
//   ovvsIvfPqSerialize    :1145-1178, ovvsIvfPqDeserialize :1180-1318 (IPQ1 v1)
//   ovvsIvfPqExtend       :1320-1427 (transactional append)
//   make_ivf_pq_packed    :59-114    (list-major layout and its invariants)
// The arithmetic-heavy steps (distances, assignment, mean update, encoding) run
// as HIP kernels (build.hip, coarse.hip); the host keeps the reference's
// control flow and its seeding, which uses the same libstdc++ distribution.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <limits>
#include <new>
#include <random>
#include <unordered_set>

#include "internal.hpp"

using ovvs::DeviceBuffer;
using ovvs::GpuWork;

namespace {

#define OVVS_HIP_TRY(expr)                          \
  do {                                              \
    const hipError_t hip_e_ = (expr);               \
    if (hip_e_ != hipSuccess) {                     \
      (void)hipGetLastError();                      \
      return ovvs::status_from_hip(hip_e_);         \
    }                                               \
  } while (0)

#define OVVS_TRY(expr)                    \
  do {                                    \
    const ovvsStatus st_ = (expr);        \
    if (st_ != OVVS_STATUS_SUCCESS) return st_; \
  } while (0)

constexpr uint32_t kIpq1Magic = 0x31515049u;  // "IPQ1", little-endian
constexpr uint64_t kIpq1HeaderBytes = 4 + 4 + 8 + 8 + 5 * 4;

ovvsStatus alloc(DeviceBuffer& b, size_t bytes, GpuWork& work) {
  const hipError_t e = b.allocate(bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return OVVS_STATUS_OOM;
  }
  ovvs::saturating_add(work.allocation_calls, 1);
  ovvs::saturating_add(work.allocation_bytes, static_cast<int64_t>(bytes));
  return OVVS_STATUS_SUCCESS;
}

ovvsStatus h2d(void* dst, const void* src, size_t bytes, hipStream_t s, GpuWork& work) {
  if (bytes == 0) return OVVS_STATUS_SUCCESS;
  OVVS_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
  ovvs::saturating_add(work.h2d_calls, 1);
  ovvs::saturating_add(work.h2d_bytes, static_cast<int64_t>(bytes));
  return OVVS_STATUS_SUCCESS;
}

ovvsStatus d2h(void* dst, const void* src, size_t bytes, hipStream_t s, GpuWork& work) {
  if (bytes == 0) return OVVS_STATUS_SUCCESS;
  OVVS_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
  ovvs::saturating_add(work.d2h_calls, 1);
  ovvs::saturating_add(work.d2h_bytes, static_cast<int64_t>(bytes));
  return OVVS_STATUS_SUCCESS;
}

ovvsStatus sync(hipStream_t s, GpuWork& work) {
  ovvs::saturating_add(work.wait_calls, 1);
  OVVS_HIP_TRY(hipStreamSynchronize(s));
  return OVVS_STATUS_SUCCESS;
}

// Seed rows of the reference k-means (mixer.cpp:881-890): k draws of a
// uniform_int_distribution<int64_t>(0, n-1) over mt19937(42), each redrawn up
// to 8 times while it repeats an earlier seed.
std::vector<int64_t> kmeans_seeds(int64_t n, int32_t k) {
  std::mt19937 rng(42u);
  std::uniform_int_distribution<int64_t> pick(0, n - 1);
  std::vector<int64_t> used;
  used.reserve(static_cast<size_t>(k));
  std::unordered_set<int64_t> seen;
  for (int32_t c = 0; c < k; ++c) {
    int64_t i = pick(rng);
    for (int t = 0; t < 8 && seen.count(i) != 0; ++t) i = pick(rng);
    used.push_back(i);
    seen.insert(i);
  }
  return used;
}

// Device k-means over x [n x dim] (row norms xn precomputed); centroids_out
// receives min(k, n) centroids. Follows kmeans_fit_impl exactly.
ovvsStatus kmeans_fit(hipStream_t s, const float* x, const float* xn, int64_t n, int32_t dim,
                      int32_t k_req, int32_t iters, const std::vector<int64_t>& seeds,
                      std::vector<float>& centroids_out, GpuWork& work) {
  const int32_t k = std::max<int32_t>(1, static_cast<int32_t>(std::min<int64_t>(k_req, n)));
  DeviceBuffer C, cn, rows, labels, sorted, order, offsets, temp;
  const size_t temp_bytes = ovvs_hip_group_temp_bytes(n);
  if (temp_bytes == 0) return OVVS_STATUS_SHAPE_MISMATCH;
  OVVS_TRY(alloc(C, static_cast<size_t>(k) * dim * 4, work));
  OVVS_TRY(alloc(cn, static_cast<size_t>(k) * 4, work));
  OVVS_TRY(alloc(rows, static_cast<size_t>(k) * 8, work));
  OVVS_TRY(alloc(labels, static_cast<size_t>(n) * 4, work));
  OVVS_TRY(alloc(sorted, static_cast<size_t>(n) * 4, work));
  OVVS_TRY(alloc(order, static_cast<size_t>(n) * 4, work));
  OVVS_TRY(alloc(offsets, (static_cast<size_t>(k) + 1) * 8, work));
  OVVS_TRY(alloc(temp, temp_bytes, work));
  OVVS_TRY(h2d(rows.get(), seeds.data(), static_cast<size_t>(k) * 8, s, work));
  OVVS_HIP_TRY(ovvs_hip_gather_rows(x, dim, rows.as<int64_t>(), k, C.as<float>(), s));
  ++work.kernel_launches;
  for (int32_t it = 0; it < iters; ++it) {
    OVVS_HIP_TRY(ovvs_hip_row_norms(C.as<float>(), k, dim, cn.as<float>(), s));
    OVVS_HIP_TRY(ovvs_hip_coarse_argmin(x, xn, n, C.as<float>(), cn.as<float>(), k, dim,
                                        labels.as<int32_t>(), s));
    OVVS_HIP_TRY(ovvs_hip_group_by_label(labels.as<int32_t>(), n, k, sorted.as<int32_t>(),
                                         order.as<int32_t>(), offsets.as<int64_t>(), temp.get(),
                                         temp_bytes, s));
    OVVS_HIP_TRY(ovvs_hip_kmeans_update(x, dim, order.as<int32_t>(), offsets.as<int64_t>(), k,
                                        C.as<float>(), s));
    work.kernel_launches += 6;
  }
  centroids_out.assign(static_cast<size_t>(k) * dim, 0.f);
  OVVS_TRY(d2h(centroids_out.data(), C.get(), centroids_out.size() * 4, s, work));
  return sync(s, work);
}

// Assignment + residual + encoding of rows x [n x dim] against an existing
// coarse quantizer and codebooks (shared by build and extend).
struct Encoded {
  std::vector<int32_t> labels;
  std::vector<uint8_t> codes;
};

ovvsStatus assign_and_encode(hipStream_t s, const float* x, const float* xn, int64_t n,
                             const ovvsIvfPqIndexImpl& ix, const float* dC, const float* dcn,
                             const float* dCB, Encoded& out, GpuWork& work) {
  DeviceBuffer labels, resid, codes;
  OVVS_TRY(alloc(labels, static_cast<size_t>(n) * 4, work));
  OVVS_TRY(alloc(resid, static_cast<size_t>(n) * ix.dim * 4, work));
  OVVS_TRY(alloc(codes, static_cast<size_t>(n) * ix.pq_m, work));
  const int32_t dim = static_cast<int32_t>(ix.dim);
  OVVS_HIP_TRY(ovvs_hip_coarse_argmin(x, xn, n, dC, dcn, ix.nlist, dim, labels.as<int32_t>(), s));
  OVVS_HIP_TRY(ovvs_hip_residuals(x, n, dim, labels.as<int32_t>(), dC, resid.as<float>(), s));
  OVVS_HIP_TRY(ovvs_hip_pq_encode(resid.as<float>(), n, dim, ix.pq_m, ix.pq_ks, ix.dsub, dCB,
                                  codes.as<uint8_t>(), s));
  work.kernel_launches += 3;
  out.labels.resize(static_cast<size_t>(n));
  out.codes.resize(static_cast<size_t>(n) * ix.pq_m);
  OVVS_TRY(d2h(out.labels.data(), labels.get(), out.labels.size() * 4, s, work));
  OVVS_TRY(d2h(out.codes.data(), codes.get(), out.codes.size(), s, work));
  return sync(s, work);
}

ovvsStatus build_on_gpu(ovvsResourcesImpl& res, ovvsIvfPqIndexImpl& ix, GpuWork& work) {
  hipStream_t s = res.stream;
  const int64_t n = ix.n;
  const int32_t dim = static_cast<int32_t>(ix.dim);
  DeviceBuffer x, xn, C, cn, resid, sub, subn, CB;
  OVVS_TRY(alloc(x, static_cast<size_t>(n) * dim * 4, work));
  OVVS_TRY(alloc(xn, static_cast<size_t>(n) * 4, work));
  OVVS_TRY(h2d(x.get(), ix.dataset.data(), ix.dataset.size() * 4, s, work));
  OVVS_HIP_TRY(ovvs_hip_row_norms(x.as<float>(), n, dim, xn.as<float>(), s));
  ++work.kernel_launches;

  const std::vector<int64_t> seeds = kmeans_seeds(n, std::max(ix.nlist, ix.pq_ks));
  OVVS_TRY(kmeans_fit(s, x.as<float>(), xn.as<float>(), n, dim, ix.nlist, 12, seeds, ix.centroids,
                      work));

  // Assignment, residuals, and PQ training per subspace.
  OVVS_TRY(alloc(C, ix.centroids.size() * 4, work));
  OVVS_TRY(alloc(cn, static_cast<size_t>(ix.nlist) * 4, work));
  OVVS_TRY(h2d(C.get(), ix.centroids.data(), ix.centroids.size() * 4, s, work));
  OVVS_HIP_TRY(ovvs_hip_row_norms(C.as<float>(), ix.nlist, dim, cn.as<float>(), s));
  DeviceBuffer labels;
  OVVS_TRY(alloc(labels, static_cast<size_t>(n) * 4, work));
  OVVS_HIP_TRY(ovvs_hip_coarse_argmin(x.as<float>(), xn.as<float>(), n, C.as<float>(),
                                      cn.as<float>(), ix.nlist, dim, labels.as<int32_t>(), s));
  OVVS_TRY(alloc(resid, static_cast<size_t>(n) * dim * 4, work));
  OVVS_HIP_TRY(ovvs_hip_residuals(x.as<float>(), n, dim, labels.as<int32_t>(), C.as<float>(),
                                  resid.as<float>(), s));
  work.kernel_launches += 3;
  x.reset();  // the dataset copy is no longer needed on the device

  ix.codebooks.assign(static_cast<size_t>(ix.pq_m) * ix.pq_ks * ix.dsub, 0.f);
  OVVS_TRY(alloc(sub, static_cast<size_t>(n) * ix.dsub * 4, work));
  OVVS_TRY(alloc(subn, static_cast<size_t>(n) * 4, work));
  std::vector<float> cents;
  for (int32_t m = 0; m < ix.pq_m; ++m) {
    OVVS_HIP_TRY(ovvs_hip_gather_sub(resid.as<float>(), n, dim, m, ix.dsub, sub.as<float>(), s));
    OVVS_HIP_TRY(ovvs_hip_row_norms(sub.as<float>(), n, ix.dsub, subn.as<float>(), s));
    work.kernel_launches += 2;
    OVVS_TRY(kmeans_fit(s, sub.as<float>(), subn.as<float>(), n, ix.dsub, ix.pq_ks, 8, seeds, cents,
                        work));
    std::memcpy(ix.codebooks.data() + static_cast<size_t>(m) * ix.pq_ks * ix.dsub, cents.data(),
                cents.size() * 4);
  }
  sub.reset();
  subn.reset();

  OVVS_TRY(alloc(CB, ix.codebooks.size() * 4, work));
  OVVS_TRY(h2d(CB.get(), ix.codebooks.data(), ix.codebooks.size() * 4, s, work));
  DeviceBuffer codes;
  OVVS_TRY(alloc(codes, static_cast<size_t>(n) * ix.pq_m, work));
  OVVS_HIP_TRY(ovvs_hip_pq_encode(resid.as<float>(), n, dim, ix.pq_m, ix.pq_ks, ix.dsub,
                                  CB.as<float>(), codes.as<uint8_t>(), s));
  ++work.kernel_launches;
  ix.assign.resize(static_cast<size_t>(n));
  ix.codes.resize(static_cast<size_t>(n) * ix.pq_m);
  OVVS_TRY(d2h(ix.assign.data(), labels.get(), ix.assign.size() * 4, s, work));
  OVVS_TRY(d2h(ix.codes.data(), codes.get(), ix.codes.size(), s, work));
  OVVS_TRY(sync(s, work));

  ix.lists.assign(static_cast<size_t>(ix.nlist), {});
  for (int64_t i = 0; i < n; ++i) {
    const int32_t a = ix.assign[static_cast<size_t>(i)];
    if (a < 0 || a >= ix.nlist) return OVVS_STATUS_ERROR;
    ix.lists[static_cast<size_t>(a)].push_back(i);
  }
  return OVVS_STATUS_SUCCESS;
}

bool fits_size(uint64_t a, uint64_t b) {
  return b == 0 || a <= std::numeric_limits<size_t>::max() / b;
}

}  // namespace

namespace ovvs {

ovvsStatus ivf_pq_build_arg_status(int64_t n, int64_t dim, ovvsMetric metric, int32_t nlist,
                                   int32_t pq_m) {
  if (n <= 0 || dim <= 0 || nlist <= 0 || pq_m <= 0) return OVVS_STATUS_INVALID_ARGUMENT;
  if (metric < OVVS_METRIC_L2_EXPANDED || metric > OVVS_METRIC_LP_UNEXPANDED) {
    return OVVS_STATUS_INVALID_ARGUMENT;
  }
  if (dim % pq_m != 0) return OVVS_STATUS_SHAPE_MISMATCH;
  if (n > std::numeric_limits<int32_t>::max() || dim > std::numeric_limits<int32_t>::max() ||
      !fits_size(static_cast<uint64_t>(n), static_cast<uint64_t>(dim) * 4)) {
    return OVVS_STATUS_SHAPE_MISMATCH;
  }
  return OVVS_STATUS_SUCCESS;
}

bool lists_valid(const ovvsIvfPqIndexImpl& ix) {
  if (ix.n <= 0 || ix.nlist <= 0 || ix.pq_m <= 0 || ix.pq_ks <= 0 || ix.pq_ks > 256 ||
      ix.lists.size() != static_cast<size_t>(ix.nlist) ||
      ix.assign.size() != static_cast<size_t>(ix.n) ||
      ix.codes.size() != static_cast<size_t>(ix.n) * static_cast<size_t>(ix.pq_m)) {
    return false;
  }
  std::vector<uint8_t> seen(static_cast<size_t>(ix.n), 0);
  int64_t total = 0;
  for (int32_t c = 0; c < ix.nlist; ++c) {
    for (const int64_t id : ix.lists[static_cast<size_t>(c)]) {
      if (id < 0 || id >= ix.n || seen[static_cast<size_t>(id)] ||
          ix.assign[static_cast<size_t>(id)] != c) {
        return false;
      }
      seen[static_cast<size_t>(id)] = 1;
      const uint8_t* code = ix.codes.data() + static_cast<size_t>(id) * ix.pq_m;
      for (int32_t m = 0; m < ix.pq_m; ++m) {
        if (code[m] >= ix.pq_ks) return false;
      }
      ++total;
    }
  }
  return total == ix.n;
}

}  // namespace ovvs

ovvsStatus ovvsIvfPqIndexImpl::ensure_device(ovvsResourcesImpl& res, GpuWork& work) {
  std::lock_guard<std::mutex> lock(device_mutex);
  if (dev && dev->device == res.device) return OVVS_STATUS_SUCCESS;
  if (!ovvs::lists_valid(*this)) return OVVS_STATUS_ERROR;
  auto d = std::make_unique<ovvs::IndexDevice>();
  d->device = res.device;
  constexpr size_t kB = OVVS_CODE_BLOCK;
  d->code_blocks = static_cast<int32_t>((static_cast<size_t>(pq_m) + kB - 1) / kB);
  std::vector<int64_t> offsets(static_cast<size_t>(nlist) + 1, 0);
  for (int32_t c = 0; c < nlist; ++c) {
    offsets[static_cast<size_t>(c) + 1] =
        offsets[static_cast<size_t>(c)] + static_cast<int64_t>(lists[static_cast<size_t>(c)].size());
  }
  ovvs::ScanLayoutHost lay;
  OVVS_TRY(ovvs::make_scan_layout(*this, OVVS_SEGMENT_ROWS, lay));
  d->positions = lay.positions;
  // The scan's bound arithmetic covers boxes of up to OVVS_MAX_BOX_DIMS dimensions.
  d->box_dims = lay.box_dims <= OVVS_MAX_BOX_DIMS ? lay.box_dims : 0;
  d->box_cmax = lay.cmax;
  const size_t nseg = lay.seg_start.size();
  hipStream_t s = res.stream;
  OVVS_TRY(alloc(d->centroids, centroids.size() * 4, work));
  OVVS_TRY(alloc(d->cnorm, static_cast<size_t>(nlist) * 4, work));
  OVVS_TRY(alloc(d->codebooks, codebooks.size() * 4, work));
  OVVS_TRY(alloc(d->codes, lay.codes.size(), work));
  OVVS_TRY(alloc(d->ids, lay.ids.size() * 8, work));
  OVVS_TRY(alloc(d->rord, lay.rord.size() * 4, work));
  OVVS_TRY(alloc(d->offsets, offsets.size() * 8, work));
  OVVS_TRY(alloc(d->list_seg, lay.list_seg.size() * 4, work));
  OVVS_TRY(alloc(d->seg_start, std::max<size_t>(nseg, 1) * 4, work));
  OVVS_TRY(alloc(d->seg_len, std::max<size_t>(nseg, 1) * 4, work));
  if (d->box_dims > 0) {
    OVVS_TRY(alloc(d->seg_box, std::max<size_t>(lay.seg_box.size(), 1) * 4, work));
    OVVS_TRY(alloc(d->list_box, lay.list_box.size() * 4, work));
    OVVS_TRY(h2d(d->list_box.get(), lay.list_box.data(), lay.list_box.size() * 4, s, work));
    OVVS_TRY(alloc(d->grp_box, std::max<size_t>(lay.grp_box.size(), 1) * 4, work));
    OVVS_TRY(h2d(d->grp_box.get(), lay.grp_box.data(), lay.grp_box.size() * 4, s, work));
  }
  OVVS_TRY(alloc(d->list_rank, lay.list_rank.size() * 4, work));
  OVVS_TRY(h2d(d->list_rank.get(), lay.list_rank.data(), lay.list_rank.size() * 4, s, work));
  OVVS_TRY(alloc(d->list_grp, lay.list_grp.size() * 4, work));
  OVVS_TRY(h2d(d->list_grp.get(), lay.list_grp.data(), lay.list_grp.size() * 4, s, work));
  OVVS_TRY(alloc(d->grp_seg, lay.grp_seg.size() * 4, work));
  OVVS_TRY(h2d(d->grp_seg.get(), lay.grp_seg.data(), lay.grp_seg.size() * 4, s, work));
  OVVS_TRY(alloc(d->dataset, dataset.size() * 4, work));
  OVVS_TRY(alloc(d->xnorm, static_cast<size_t>(n) * 4, work));
  OVVS_TRY(h2d(d->centroids.get(), centroids.data(), centroids.size() * 4, s, work));
  OVVS_TRY(h2d(d->codebooks.get(), codebooks.data(), codebooks.size() * 4, s, work));
  OVVS_TRY(h2d(d->codes.get(), lay.codes.data(), lay.codes.size(), s, work));
  OVVS_TRY(h2d(d->ids.get(), lay.ids.data(), lay.ids.size() * 8, s, work));
  OVVS_TRY(h2d(d->rord.get(), lay.rord.data(), lay.rord.size() * 4, s, work));
  OVVS_TRY(h2d(d->offsets.get(), offsets.data(), offsets.size() * 8, s, work));
  OVVS_TRY(h2d(d->list_seg.get(), lay.list_seg.data(), lay.list_seg.size() * 4, s, work));
  if (nseg > 0) {
    OVVS_TRY(h2d(d->seg_start.get(), lay.seg_start.data(), nseg * 4, s, work));
    OVVS_TRY(h2d(d->seg_len.get(), lay.seg_len.data(), nseg * 4, s, work));
    if (d->box_dims > 0)
      OVVS_TRY(h2d(d->seg_box.get(), lay.seg_box.data(), lay.seg_box.size() * 4, s, work));
  }
  OVVS_TRY(h2d(d->dataset.get(), dataset.data(), dataset.size() * 4, s, work));
  OVVS_HIP_TRY(ovvs_hip_row_norms(d->centroids.as<float>(), nlist, static_cast<int32_t>(dim),
                                  d->cnorm.as<float>(), s));
  OVVS_HIP_TRY(ovvs_hip_row_norms(d->dataset.as<float>(), n, static_cast<int32_t>(dim),
                                  d->xnorm.as<float>(), s));
  work.kernel_launches += 2;
  std::vector<uint32_t> cmfma(ovvs_hip_probe_cmfma_words(static_cast<int32_t>(dim), nlist));
  std::vector<float> cmu, cnc;
  if (!cmfma.empty()) {
    cmu.resize(static_cast<size_t>(dim));
    cnc.resize(static_cast<size_t>(nlist));
    ovvs_probe_prepare(centroids.data(), nlist, static_cast<int32_t>(dim), cmfma.data(), cmu.data(),
                       cnc.data(), &d->cnc_max);
    OVVS_TRY(alloc(d->cmfma, cmfma.size() * 4, work));
    OVVS_TRY(h2d(d->cmfma.get(), cmfma.data(), cmfma.size() * 4, s, work));
    OVVS_TRY(alloc(d->cmu, cmu.size() * 4, work));
    OVVS_TRY(h2d(d->cmu.get(), cmu.data(), cmu.size() * 4, s, work));
    OVVS_TRY(alloc(d->cnc, cnc.size() * 4, work));
    OVVS_TRY(h2d(d->cnc.get(), cnc.data(), cnc.size() * 4, s, work));
  }
  std::vector<float> cnorm(static_cast<size_t>(nlist));
  OVVS_TRY(d2h(cnorm.data(), d->cnorm.get(), cnorm.size() * 4, s, work));
  OVVS_TRY(sync(s, work));
  for (const float v : cnorm) {
    if (!(v <= d->cnorm_max)) d->cnorm_max = std::isfinite(v) ? v : INFINITY;
    if (std::isinf(d->cnorm_max)) break;
  }
  dev = std::move(d);
  return OVVS_STATUS_SUCCESS;
}

extern "C" {

OVVS_API ovvsStatus ovvsIvfPqBuild(ovvsResources_t res, const float* dataset, int64_t n,
                                   int64_t dim, ovvsMetric metric, int32_t nlist, int32_t pq_m,
                                   int32_t pq_nbits, ovvsIvfPqIndex_t* index) {
  if (index) *index = nullptr;
  if (!res || !dataset || !index) return OVVS_STATUS_INVALID_ARGUMENT;
  OVVS_TRY(ovvs::ivf_pq_build_arg_status(n, dim, metric, nlist, pq_m));
  nlist = static_cast<int32_t>(std::min<int64_t>(nlist, n));
  const int32_t ks = 1 << std::min(std::max(pq_nbits, 4), 8);
  try {
    std::lock_guard<std::mutex> lock(res->call_mutex);
    OVVS_TRY(res->ensure_gpu());
    auto ix = std::make_unique<ovvsIvfPqIndexImpl>();
    ix->n = n;
    ix->dim = dim;
    ix->metric = metric;
    ix->nlist = nlist;
    ix->pq_m = pq_m;
    ix->pq_ks = ks;
    ix->dsub = static_cast<int32_t>(dim / pq_m);
    ix->dataset.assign(dataset, dataset + n * dim);
    GpuWork work;
    OVVS_TRY(build_on_gpu(*res, *ix, work));
    if (!ovvs::lists_valid(*ix)) return OVVS_STATUS_ERROR;
    res->last_device = OVVS_DEVICE_GPU;
    *index = ix.release();
    return OVVS_STATUS_SUCCESS;
  } catch (const std::bad_alloc&) {
    return OVVS_STATUS_OOM;
  } catch (...) {
    return OVVS_STATUS_ERROR;
  }
}

OVVS_API ovvsStatus ovvsIvfPqDestroy(ovvsIvfPqIndex_t index) {
  delete index;
  return OVVS_STATUS_SUCCESS;
}

OVVS_API ovvsStatus ovvsIvfPqSerialize(ovvsIvfPqIndex_t index, const char* path) {
  if (!index || !path) return OVVS_STATUS_INVALID_ARGUMENT;
  const ovvsIvfPqIndexImpl& ix = *index;
  FILE* f = std::fopen(path, "wb");
  if (!f) return OVVS_STATUS_IO;
  bool ok = true;
  auto put = [&](const void* p, size_t bytes) {
    if (ok && bytes > 0) ok = std::fwrite(p, 1, bytes, f) == bytes;
  };
  const int32_t version = 1;
  const int32_t metric = static_cast<int32_t>(ix.metric);
  put(&kIpq1Magic, 4);
  put(&version, 4);
  put(&ix.n, 8);
  put(&ix.dim, 8);
  put(&ix.nlist, 4);
  put(&ix.pq_m, 4);
  put(&ix.pq_ks, 4);
  put(&ix.dsub, 4);
  put(&metric, 4);
  put(ix.centroids.data(), ix.centroids.size() * 4);
  put(ix.codebooks.data(), ix.codebooks.size() * 4);
  put(ix.codes.data(), ix.codes.size());
  put(ix.dataset.data(), ix.dataset.size() * 4);
  put(ix.assign.data(), ix.assign.size() * 4);
  for (const auto& list : ix.lists) {
    const int32_t size = static_cast<int32_t>(list.size());
    put(&size, 4);
    put(list.data(), list.size() * 8);
  }
  if (std::fclose(f) != 0) ok = false;
  return ok ? OVVS_STATUS_SUCCESS : OVVS_STATUS_IO;
}

OVVS_API ovvsStatus ovvsIvfPqDeserialize(ovvsResources_t res, const char* path,
                                         ovvsIvfPqIndex_t* index) {
  if (index) *index = nullptr;
  if (!res || !path || !index) return OVVS_STATUS_INVALID_ARGUMENT;
  try {
    FILE* f = std::fopen(path, "rb");
    if (!f) return OVVS_STATUS_IO;
    struct Closer {
      FILE* f;
      ~Closer() { std::fclose(f); }
    } closer{f};
    if (fseeko(f, 0, SEEK_END) != 0) return OVVS_STATUS_IO;
    const off_t end = ftello(f);
    if (end < 0 || fseeko(f, 0, SEEK_SET) != 0) return OVVS_STATUS_IO;
    const uint64_t file_bytes = static_cast<uint64_t>(end);
    auto get = [&](void* p, size_t bytes) {
      return bytes == 0 || std::fread(p, 1, bytes, f) == bytes;
    };
    uint32_t magic = 0;
    int32_t version = 0;
    if (!get(&magic, 4) || !get(&version, 4) || magic != kIpq1Magic) return OVVS_STATUS_IO;
    if (version != 1) return OVVS_STATUS_UNSUPPORTED;
    auto ix = std::make_unique<ovvsIvfPqIndexImpl>();
    int32_t metric = 0;
    if (!get(&ix->n, 8) || !get(&ix->dim, 8) || !get(&ix->nlist, 4) || !get(&ix->pq_m, 4) ||
        !get(&ix->pq_ks, 4) || !get(&ix->dsub, 4) || !get(&metric, 4)) {
      return OVVS_STATUS_IO;
    }
    if (ix->n <= 0 || ix->n > std::numeric_limits<int32_t>::max() || ix->dim <= 0 ||
        ix->nlist <= 0 || ix->nlist > ix->n || ix->pq_m <= 0 || ix->pq_ks < 16 ||
        ix->pq_ks > 256 || (ix->pq_ks & (ix->pq_ks - 1)) != 0 || ix->dsub <= 0 ||
        ix->dim % ix->pq_m != 0 || ix->dsub != ix->dim / ix->pq_m ||
        metric < OVVS_METRIC_L2_EXPANDED || metric > OVVS_METRIC_LP_UNEXPANDED ||
        ix->dim > std::numeric_limits<int32_t>::max()) {
      return OVVS_STATUS_IO;
    }
    ix->metric = static_cast<ovvsMetric>(metric);
    const uint64_t n = static_cast<uint64_t>(ix->n), dim = static_cast<uint64_t>(ix->dim);
    const uint64_t nlist = static_cast<uint64_t>(ix->nlist);
    const uint64_t cb = static_cast<uint64_t>(ix->pq_m) * ix->pq_ks * ix->dsub;
    if (!fits_size(n, dim * 4) || !fits_size(nlist, dim * 4)) return OVVS_STATUS_IO;
    using u128 = unsigned __int128;
    const u128 expected = static_cast<u128>(kIpq1HeaderBytes) + static_cast<u128>(nlist) * dim * 4 +
                          static_cast<u128>(cb) * 4 + static_cast<u128>(n) * ix->pq_m +
                          static_cast<u128>(n) * dim * 4 + static_cast<u128>(n) * 4 +
                          static_cast<u128>(nlist) * 4 + static_cast<u128>(n) * 8;
    if (static_cast<u128>(file_bytes) != expected) return OVVS_STATUS_IO;
    ix->centroids.resize(nlist * dim);
    ix->codebooks.resize(cb);
    ix->codes.resize(n * static_cast<uint64_t>(ix->pq_m));
    ix->dataset.resize(n * dim);
    ix->assign.resize(n);
    if (!get(ix->centroids.data(), ix->centroids.size() * 4) ||
        !get(ix->codebooks.data(), ix->codebooks.size() * 4) ||
        !get(ix->codes.data(), ix->codes.size()) ||
        !get(ix->dataset.data(), ix->dataset.size() * 4) ||
        !get(ix->assign.data(), ix->assign.size() * 4)) {
      return OVVS_STATUS_IO;
    }
    ix->lists.resize(nlist);
    int64_t total = 0;
    for (uint64_t c = 0; c < nlist; ++c) {
      int32_t size = 0;
      if (!get(&size, 4) || size < 0 || size > ix->n - total) return OVVS_STATUS_IO;
      total += size;
      ix->lists[c].resize(static_cast<size_t>(size));
      if (!get(ix->lists[c].data(), static_cast<size_t>(size) * 8)) return OVVS_STATUS_IO;
    }
    if (total != ix->n || !ovvs::lists_valid(*ix)) return OVVS_STATUS_IO;
    *index = ix.release();
    return OVVS_STATUS_SUCCESS;
  } catch (const std::bad_alloc&) {
    return OVVS_STATUS_OOM;
  } catch (...) {
    return OVVS_STATUS_ERROR;
  }
}

OVVS_API ovvsStatus ovvsIvfPqExtend(ovvsResources_t res, ovvsIvfPqIndex_t index,
                                    const float* extra, int64_t nextra) {
  if (!res || !index || !extra || nextra <= 0) return OVVS_STATUS_INVALID_ARGUMENT;
  ovvsIvfPqIndexImpl& ix = *index;
  const int64_t old_n = ix.n;
  if (old_n <= 0 || ix.dim <= 0 || ix.nlist <= 0 || ix.pq_m <= 0 || ix.pq_ks <= 0 ||
      ix.dsub <= 0 || nextra > std::numeric_limits<int64_t>::max() - old_n ||
      nextra > std::numeric_limits<int64_t>::max() / ix.dim) {
    return OVVS_STATUS_SHAPE_MISMATCH;
  }
  const int64_t new_n = old_n + nextra;
  if (new_n > std::numeric_limits<int32_t>::max() ||
      !fits_size(static_cast<uint64_t>(new_n), static_cast<uint64_t>(ix.dim) * 4)) {
    return OVVS_STATUS_SHAPE_MISMATCH;
  }
  if (ix.dataset.size() != static_cast<size_t>(old_n * ix.dim) ||
      ix.assign.size() != static_cast<size_t>(old_n) ||
      ix.codes.size() != static_cast<size_t>(old_n) * ix.pq_m ||
      ix.lists.size() != static_cast<size_t>(ix.nlist)) {
    return OVVS_STATUS_ERROR;
  }
  try {
    std::lock_guard<std::mutex> lock(res->call_mutex);
    OVVS_TRY(res->ensure_gpu());
    GpuWork work;
    hipStream_t s = res->stream;
    const int32_t dim = static_cast<int32_t>(ix.dim);
    DeviceBuffer x, xn, C, cn, CB;
    OVVS_TRY(alloc(x, static_cast<size_t>(nextra) * dim * 4, work));
    OVVS_TRY(alloc(xn, static_cast<size_t>(nextra) * 4, work));
    OVVS_TRY(alloc(C, ix.centroids.size() * 4, work));
    OVVS_TRY(alloc(cn, static_cast<size_t>(ix.nlist) * 4, work));
    OVVS_TRY(alloc(CB, ix.codebooks.size() * 4, work));
    OVVS_TRY(h2d(x.get(), extra, static_cast<size_t>(nextra) * dim * 4, s, work));
    OVVS_TRY(h2d(C.get(), ix.centroids.data(), ix.centroids.size() * 4, s, work));
    OVVS_TRY(h2d(CB.get(), ix.codebooks.data(), ix.codebooks.size() * 4, s, work));
    OVVS_HIP_TRY(ovvs_hip_row_norms(x.as<float>(), nextra, dim, xn.as<float>(), s));
    OVVS_HIP_TRY(ovvs_hip_row_norms(C.as<float>(), ix.nlist, dim, cn.as<float>(), s));
    Encoded enc;
    OVVS_TRY(assign_and_encode(s, x.as<float>(), xn.as<float>(), nextra, ix, C.as<float>(),
                               cn.as<float>(), CB.as<float>(), enc, work));

    // Stage the new state, validate it, then commit with no-throw swaps.
    ovvsIvfPqIndexImpl next;
    next.n = new_n;
    next.dim = ix.dim;
    next.nlist = ix.nlist;
    next.pq_m = ix.pq_m;
    next.pq_ks = ix.pq_ks;
    next.assign = ix.assign;
    next.assign.insert(next.assign.end(), enc.labels.begin(), enc.labels.end());
    next.codes = ix.codes;
    next.codes.insert(next.codes.end(), enc.codes.begin(), enc.codes.end());
    next.lists = ix.lists;
    for (int64_t i = 0; i < nextra; ++i) {
      const int32_t a = enc.labels[static_cast<size_t>(i)];
      if (a < 0 || a >= ix.nlist) return OVVS_STATUS_ERROR;
      next.lists[static_cast<size_t>(a)].push_back(old_n + i);
    }
    if (!ovvs::lists_valid(next)) return OVVS_STATUS_ERROR;
    std::vector<float> next_dataset;
    next_dataset.reserve(static_cast<size_t>(new_n) * dim);
    next_dataset.insert(next_dataset.end(), ix.dataset.begin(), ix.dataset.end());
    next_dataset.insert(next_dataset.end(), extra, extra + nextra * dim);

    std::lock_guard<std::mutex> dev_lock(ix.device_mutex);
    ix.dataset.swap(next_dataset);
    ix.assign.swap(next.assign);
    ix.codes.swap(next.codes);
    ix.lists.swap(next.lists);
    ix.n = new_n;
    ix.dev.reset();
    res->last_device = OVVS_DEVICE_GPU;
    return OVVS_STATUS_SUCCESS;
  } catch (const std::bad_alloc&) {
    return OVVS_STATUS_OOM;
  } catch (...) {
    return OVVS_STATUS_ERROR;
  }
}

}  // extern "C"
