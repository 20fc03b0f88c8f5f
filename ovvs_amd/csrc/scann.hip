// scann.hip — device steps of the ScaNN-style index on gfx950: the per-column
// scale factors of the build, the column scaling of rows and queries, and the
// candidate lists of the original-space re-rank.
//
// Reference behaviour (src/neighbors/graphs.cpp:3286-3374): the build scales
// column d of every row by aniso[d] = sqrt(var_d + 1e-6), var_d the population
// variance of the column (left-to-right fp32 sums over the rows: the mean, then
// the squared deviations), trains IVF-PQ on the scaled rows, and the search runs
// IVF-PQ on scaled queries, then re-ranks the returned ids on the original rows.
#include "device_common.hpp"
#include "kernels.hpp"

namespace {

constexpr int kColThreads = 64;
constexpr int kColBatch = 16;  // loads in flight per thread

// Left-to-right fp32 sum over the rows of column d of f(x[i*dim + d]).
template <class F>
__device__ float column_sum(const float* __restrict__ x, int64_t n, int32_t dim, int32_t d, F f) {
  float s = 0.f;
  int64_t i = 0;
  for (; i + kColBatch <= n; i += kColBatch) {
    float v[kColBatch];
#pragma unroll
    for (int u = 0; u < kColBatch; ++u) v[u] = x[(i + u) * dim + d];
#pragma unroll
    for (int u = 0; u < kColBatch; ++u) s = s + f(v[u]);
  }
  for (; i < n; ++i) s = s + f(x[i * dim + d]);
  return s;
}

// One thread per column (reference graphs.cpp:3291-3301): mean = sum / n, then
// var = sum of (x - mean)^2, aniso = sqrt(var / max(n, 1) + 1e-6). Division and
// sqrt are the correctly rounded lowerings (no fast-math flags), as the host's
// divss/sqrtss are.
__global__ __launch_bounds__(kColThreads) void k_column_aniso(const float* __restrict__ x,
                                                              int64_t n, int32_t dim,
                                                              float* __restrict__ aniso) {
  const int32_t d = static_cast<int32_t>(blockIdx.x) * kColThreads + static_cast<int32_t>(threadIdx.x);
  if (d >= dim) return;
  const float mean = column_sum(x, n, dim, d, [](float v) { return v; }) / static_cast<float>(n);
  const float var = column_sum(x, n, dim, d, [mean](float v) {
    const float t = v - mean;
    return t * t;
  });
  const float cnt = static_cast<float>(n > 1 ? n : 1);
  aniso[d] = __builtin_sqrtf(var / cnt + 1e-6f);
}

// out[i*dim + d] = x[i*dim + d] * s[d] (reference graphs.cpp:3304-3307, 3326-3328).
__global__ __launch_bounds__(256) void k_scale_columns(const float* __restrict__ x, int64_t count,
                                                       int32_t dim, const float* __restrict__ s,
                                                       float* __restrict__ out) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; e < count; e += stride) {
    out[e] = x[e] * s[e % dim];
  }
}

// The re-rank's candidate list of each query (reference graphs.cpp:3334-3340):
// the ids in [0, n) among the query's R IVF-PQ results, in result order. pos[q*R+j]
// is the flat index q*R + t of the j-th kept result; count[q] = j.
__global__ __launch_bounds__(256) void k_ids_shortlist(const int64_t* __restrict__ ids, int64_t nq,
                                                       int32_t R, int64_t n,
                                                       int32_t* __restrict__ pos,
                                                       int32_t* __restrict__ count) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (q >= nq) return;
  const int64_t base = q * R;
  int32_t j = 0;
  for (int32_t t = 0; t < R; ++t) {
    const int64_t id = ids[base + t];
    if (id >= 0 && id < n) pos[base + j++] = static_cast<int32_t>(base + t);
  }
  count[q] = j;
}

}  // namespace

extern "C" hipError_t ovvs_hip_column_aniso(const float* x, int64_t n, int32_t dim, float* aniso,
                                            hipStream_t stream) {
  if (!x || !aniso || n <= 0 || dim <= 0) return hipErrorInvalidValue;
  const uint32_t blocks = static_cast<uint32_t>((dim + kColThreads - 1) / kColThreads);
  hipLaunchKernelGGL(k_column_aniso, dim3(blocks), dim3(kColThreads), 0, stream, x, n, dim, aniso);
  return hipGetLastError();
}

extern "C" hipError_t ovvs_hip_scale_columns(const float* x, int64_t rows, int32_t dim,
                                             const float* s, float* out, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  if (!x || !s || !out || dim <= 0) return hipErrorInvalidValue;
  const int64_t count = rows * dim;
  const int64_t want = (count + 255) / 256;
  const uint32_t blocks = static_cast<uint32_t>(want < 16384 ? want : 16384);
  hipLaunchKernelGGL(k_scale_columns, dim3(blocks), dim3(256), 0, stream, x, count, dim, s, out);
  return hipGetLastError();
}

extern "C" hipError_t ovvs_hip_ids_shortlist(const int64_t* ids, int64_t nq, int32_t R, int64_t n,
                                             int32_t* pos, int32_t* count, hipStream_t stream) {
  if (nq <= 0) return hipSuccess;
  if (!ids || !pos || !count || R <= 0 || nq > 0x7fffffff / R) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_ids_shortlist, dim3(static_cast<uint32_t>((nq + 255) / 256)), dim3(256), 0,
                     stream, ids, nq, R, n, pos, count);
  return hipGetLastError();
}
