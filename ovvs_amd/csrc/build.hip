// build.hip — gfx950 kernels behind ovvsIvfPqBuild / ovvsIvfPqExtend.
//
// Reference behaviour (src/neighbors/indexes.cpp:192-229,459-536,
// src/prim/mixer.cpp:866-921): Lloyd k-means whose assignment step is the exact
// expanded-L2 argmin (ovvs_hip_coarse_argmin) and whose update step sums each
// cluster's rows left to right in row order and multiplies by 1/count; PQ
// training runs that k-means per subspace on the residuals; encoding picks the
// first codeword with the smallest direct L2 distance.
//
// Grouping rows by label uses hipCUB's LSD radix sort, which is stable, so each
// cluster's rows come out in ascending row order, the order the reference sums
// them in (and the order build_ivf_lists, indexes.cpp:50-57, lists them in).
#include <hipcub/hipcub.hpp>

#include "device_common.hpp"
#include "kernels.hpp"

using namespace ovvs_dev;

namespace {

constexpr int kThreads = 256;

__global__ void k_gather_sub(const float* __restrict__ x, int64_t n, int dim, int m, int dsub,
                             float* __restrict__ out) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= n * dsub) return;
  const int64_t i = e / dsub;
  const int u = static_cast<int>(e % dsub);
  out[e] = x[i * dim + static_cast<int64_t>(m) * dsub + u];
}

__global__ void k_residuals(const float* __restrict__ x, int64_t n, int dim,
                            const int32_t* __restrict__ labels, const float* __restrict__ C,
                            float* __restrict__ out) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= n * dim) return;
  const int64_t i = e / dim;
  const int t = static_cast<int>(e % dim);
  out[e] = x[e] - C[static_cast<int64_t>(labels[i]) * dim + t];
}

__global__ void k_gather_rows(const float* __restrict__ x, int dim, const int64_t* __restrict__ rows,
                              int count, float* __restrict__ out) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= static_cast<int64_t>(count) * dim) return;
  const int64_t c = e / dim;
  const int t = static_cast<int>(e % dim);
  out[e] = x[rows[c] * dim + t];
}

__global__ void k_iota(int32_t* __restrict__ out, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i < n) out[i] = static_cast<int32_t>(i);
}

// offsets[c] = first index of sorted_labels with value >= c, for c in [0, k].
__global__ void k_segment_offsets(const int32_t* __restrict__ sorted_labels, int64_t n, int k,
                                  int64_t* __restrict__ offsets) {
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c > k) return;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = lo + ((hi - lo) >> 1);
    if (sorted_labels[mid] < c) {
      lo = mid + 1;
    } else {
      hi = mid;
    }
  }
  offsets[c] = lo;
}

__global__ void k_kmeans_update(const float* __restrict__ x, int dim,
                                const int32_t* __restrict__ order,
                                const int64_t* __restrict__ offsets, int k, float* __restrict__ C) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= static_cast<int64_t>(k) * dim) return;
  const int64_t c = e / dim;
  const int t = static_cast<int>(e % dim);
  const int64_t b = offsets[c], end = offsets[c + 1];
  if (end <= b) return;
  float s = 0.f;
  for (int64_t r = b; r < end; ++r) s = s + x[static_cast<int64_t>(order[r]) * dim + t];
  const float inv = 1.f / static_cast<float>(end - b);
  C[e] = s * inv;
}

__global__ void k_pq_encode(const float* __restrict__ resid, int64_t n, int dim, int pq_m, int ks,
                            int dsub, const float* __restrict__ codebooks,
                            uint8_t* __restrict__ codes) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= n * pq_m) return;
  const int64_t i = e / pq_m;
  const int m = static_cast<int>(e % pq_m);
  const float* sub = resid + i * dim + static_cast<int64_t>(m) * dsub;
  const float* cb = codebooks + static_cast<int64_t>(m) * ks * dsub;
  int best = 0;
  float best_d = __builtin_inff();
  for (int c = 0; c < ks; ++c) {
    const float d = seq_l2sq(sub, cb + static_cast<int64_t>(c) * dsub, dsub);
    if (d < best_d) {
      best_d = d;
      best = c;
    }
  }
  codes[e] = static_cast<uint8_t>(best);
}

inline uint32_t blocks_for(int64_t work) { return static_cast<uint32_t>((work + kThreads - 1) / kThreads); }
inline bool grid_ok(int64_t work) { return work >= 0 && (work + kThreads - 1) / kThreads <= 0x7fffffff; }
inline size_t round256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

size_t cub_sort_bytes(int64_t n) {
  size_t bytes = 0;
  const hipError_t e = hipcub::DeviceRadixSort::SortPairs(
      nullptr, bytes, static_cast<const int32_t*>(nullptr), static_cast<int32_t*>(nullptr),
      static_cast<const int32_t*>(nullptr), static_cast<int32_t*>(nullptr), static_cast<int>(n), 0,
      32);
  return e == hipSuccess ? bytes : 0;
}

}  // namespace

extern "C" hipError_t ovvs_hip_gather_sub(const float* x, int64_t n, int32_t dim, int32_t m,
                                          int32_t dsub, float* out, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (!x || !out || dim <= 0 || dsub <= 0 || m < 0 || (m + 1) * dsub > dim || !grid_ok(n * dsub))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gather_sub, dim3(blocks_for(n * dsub)), dim3(kThreads), 0, stream, x, n,
                     dim, m, dsub, out);
  return hipGetLastError();
}

extern "C" hipError_t ovvs_hip_residuals(const float* x, int64_t n, int32_t dim,
                                         const int32_t* labels, const float* C, float* out,
                                         hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (!x || !labels || !C || !out || dim <= 0 || !grid_ok(n * dim)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_residuals, dim3(blocks_for(n * dim)), dim3(kThreads), 0, stream, x, n, dim,
                     labels, C, out);
  return hipGetLastError();
}

extern "C" hipError_t ovvs_hip_gather_rows(const float* x, int32_t dim, const int64_t* rows,
                                           int32_t count, float* out, hipStream_t stream) {
  if (count <= 0) return hipSuccess;
  if (!x || !rows || !out || dim <= 0 || !grid_ok(static_cast<int64_t>(count) * dim))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gather_rows, dim3(blocks_for(static_cast<int64_t>(count) * dim)),
                     dim3(kThreads), 0, stream, x, dim, rows, count, out);
  return hipGetLastError();
}

extern "C" size_t ovvs_hip_group_temp_bytes(int64_t n) {
  if (n <= 0 || n > 0x7fffffff) return 0;
  return round256(static_cast<size_t>(n) * 4) + round256(cub_sort_bytes(n));
}

extern "C" hipError_t ovvs_hip_group_by_label(const int32_t* labels, int64_t n, int32_t k,
                                              int32_t* sorted_labels, int32_t* order,
                                              int64_t* offsets, void* temp, size_t temp_bytes,
                                              hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (!labels || !sorted_labels || !order || !offsets || !temp || k <= 0 || n > 0x7fffffff ||
      temp_bytes < ovvs_hip_group_temp_bytes(n))
    return hipErrorInvalidValue;
  int32_t* iota = static_cast<int32_t*>(temp);
  void* cub_temp = static_cast<unsigned char*>(temp) + round256(static_cast<size_t>(n) * 4);
  size_t cub_bytes = temp_bytes - round256(static_cast<size_t>(n) * 4);
  hipLaunchKernelGGL(k_iota, dim3(blocks_for(n)), dim3(kThreads), 0, stream, iota, n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // Labels are in [0, k): sorting only the significant bits keeps the passes few.
  int bits = 1;
  while (bits < 32 && (static_cast<int64_t>(1) << bits) < k) ++bits;
  size_t cub_need = 0;
  e = hipcub::DeviceRadixSort::SortPairs(nullptr, cub_need, labels, sorted_labels, iota, order,
                                         static_cast<int>(n), 0, bits, stream);
  if (e != hipSuccess) return e;
  if (cub_need > cub_bytes) return hipErrorInvalidValue;
  e = hipcub::DeviceRadixSort::SortPairs(cub_temp, cub_bytes, labels, sorted_labels, iota, order,
                                         static_cast<int>(n), 0, bits, stream);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_segment_offsets, dim3(blocks_for(static_cast<int64_t>(k) + 1)),
                     dim3(kThreads), 0, stream, sorted_labels, n, k, offsets);
  return hipGetLastError();
}

extern "C" hipError_t ovvs_hip_kmeans_update(const float* x, int32_t dim, const int32_t* order,
                                             const int64_t* offsets, int32_t k, float* C,
                                             hipStream_t stream) {
  if (k <= 0) return hipSuccess;
  if (!x || !order || !offsets || !C || dim <= 0 || !grid_ok(static_cast<int64_t>(k) * dim))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_kmeans_update, dim3(blocks_for(static_cast<int64_t>(k) * dim)),
                     dim3(kThreads), 0, stream, x, dim, order, offsets, k, C);
  return hipGetLastError();
}

extern "C" hipError_t ovvs_hip_pq_encode(const float* resid, int64_t n, int32_t dim, int32_t pq_m,
                                         int32_t ks, int32_t dsub, const float* codebooks,
                                         uint8_t* codes, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (!resid || !codebooks || !codes || pq_m <= 0 || ks <= 0 || ks > 256 || dsub <= 0 ||
      static_cast<int64_t>(pq_m) * dsub > dim || !grid_ok(n * pq_m))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_pq_encode, dim3(blocks_for(n * pq_m)), dim3(kThreads), 0, stream, resid, n,
                     dim, pq_m, ks, dsub, codebooks, codes);
  return hipGetLastError();
}
