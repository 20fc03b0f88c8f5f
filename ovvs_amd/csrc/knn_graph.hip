// knn_graph.hip — neighbour-list assembly of the IVF-PQ k-nearest-neighbour graph
// (the CAGRA build's IVF-PQ initializer, reference src/neighbors/graphs.cpp:767-797)
// on gfx950.
#include "device_common.hpp"
#include "kernels.hpp"

namespace {

// Row i's list (reference graphs.cpp:788-795): its search results in rank order,
// skipping i itself and -1, at most `degree` of them, the rest -1. One thread per row.
__global__ __launch_bounds__(256) void k_knn_graph_rows(const int64_t* __restrict__ nb, int64_t n,
                                                        int64_t row0, int32_t degree,
                                                        int32_t* __restrict__ graph) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (r >= n) return;
  const int64_t self = row0 + r;
  const int64_t* in = nb + r * (degree + 1);
  int32_t* out = graph + self * degree;
  int32_t filled = 0;
  for (int32_t t = 0; t < degree + 1 && filled < degree; ++t) {
    const int64_t id = in[t];
    if (id == self || id < 0) continue;
    out[filled++] = static_cast<int32_t>(id);
  }
  for (; filled < degree; ++filled) out[filled] = -1;
}

}  // namespace

extern "C" hipError_t ovvs_hip_knn_graph_rows(const int64_t* nb, int64_t n, int64_t row0,
                                              int32_t degree, int32_t* graph,
                                              hipStream_t stream) {
  if (n <= 0 || degree <= 0) return hipSuccess;
  if (!nb || !graph || row0 < 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_knn_graph_rows, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0,
                     stream, nb, n, row0, degree, graph);
  return hipGetLastError();
}
