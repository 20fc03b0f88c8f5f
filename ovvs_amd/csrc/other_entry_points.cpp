// other_entry_points.cpp — the reference's entry points for algorithms outside the
// IVF-PQ path (brute force, IVF-Flat, IVF-RaBitQ, CAGRA, HNSW, Vamana, k-means, the
// batcher, the dense primitives, SYCL and energy queries). The reference's own
// callers bind them when they load the library (its Python package does so at
// import), so libovvs exports each with the reference's name and signature and
// answers OVVS_STATUS_UNSUPPORTED, writing nothing; destroying a NULL handle
// succeeds, as it does in the reference.
#include "ovvs/ovvs.h"

namespace {
constexpr ovvsStatus kNo = OVVS_STATUS_UNSUPPORTED;
ovvsStatus destroy_none(const void* handle) {
  return handle ? OVVS_STATUS_INVALID_ARGUMENT : OVVS_STATUS_SUCCESS;
}
}  // namespace

extern "C" {

OVVS_API int32_t ovvsSyclEnabled(void) { return 0; }
OVVS_API ovvsStatus ovvsResourcesEnergyUj(ovvsResources_t, int64_t*) { return kNo; }
OVVS_API ovvsStatus ovvsGemm(ovvsResources_t, const float*, const float*, float*, int64_t, int64_t,
                             int64_t, int32_t) {
  return kNo;
}
OVVS_API ovvsStatus ovvsGemmEx(ovvsResources_t, const float*, const float*, float*, int64_t,
                               int64_t, int64_t, int32_t, ovvsDType) {
  return kNo;
}
OVVS_API ovvsStatus ovvsTopk(ovvsResources_t, const float*, int64_t, int64_t, int64_t, int64_t*,
                             float*, int32_t) {
  return kNo;
}
OVVS_API ovvsStatus ovvsGatherRows(ovvsResources_t, const float*, int64_t, int64_t,
                                   const int64_t*, int64_t, float*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsBruteForceBuild(ovvsResources_t, const float*, int64_t, int64_t,
                                        ovvsMetric, ovvsBruteForceIndex_t*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsBruteForceSearch(ovvsResources_t, ovvsBruteForceIndex_t, const float*,
                                         int64_t, int64_t, const uint8_t*, int64_t*, float*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsBruteForceDestroy(ovvsBruteForceIndex_t index) { return destroy_none(index); }
OVVS_API ovvsStatus ovvsIvfFlatBuild(ovvsResources_t, const float*, int64_t, int64_t, ovvsMetric,
                                     int32_t, ovvsIvfFlatIndex_t*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsIvfFlatSearch(ovvsResources_t, ovvsIvfFlatIndex_t, const float*, int64_t,
                                      int64_t, int32_t, const uint8_t*, int64_t*, float*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsIvfFlatDestroy(ovvsIvfFlatIndex_t index) { return destroy_none(index); }
OVVS_API ovvsStatus ovvsIvfRabitqBuild(ovvsResources_t, const float*, int64_t, int64_t,
                                       ovvsMetric, int32_t, ovvsIvfRabitqIndex_t*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsIvfRabitqSearch(ovvsResources_t, ovvsIvfRabitqIndex_t, const float*,
                                        int64_t, int64_t, int32_t, int32_t, const uint8_t*,
                                        int64_t*, float*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsIvfRabitqSerialize(ovvsIvfRabitqIndex_t, const char*) { return kNo; }
OVVS_API ovvsStatus ovvsIvfRabitqDeserialize(ovvsResources_t, const char*, ovvsIvfRabitqIndex_t*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsIvfRabitqExtend(ovvsResources_t, ovvsIvfRabitqIndex_t, const float*,
                                        int64_t) {
  return kNo;
}
OVVS_API ovvsStatus ovvsIvfRabitqDestroy(ovvsIvfRabitqIndex_t index) { return destroy_none(index); }
OVVS_API ovvsStatus ovvsCagraBuild(ovvsResources_t, const float*, int64_t, int64_t, ovvsMetric,
                                   int32_t, int32_t, ovvsCagraIndex_t*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsCagraSearch(ovvsResources_t, ovvsCagraIndex_t, const float*, int64_t,
                                    int64_t, int32_t, int32_t, const uint8_t*, int64_t*, float*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsCagraExtend(ovvsResources_t, ovvsCagraIndex_t, const float*, int64_t) {
  return kNo;
}
OVVS_API ovvsStatus ovvsCagraDestroy(ovvsCagraIndex_t index) { return destroy_none(index); }
OVVS_API ovvsStatus ovvsHnswFromCagra(ovvsResources_t, ovvsCagraIndex_t, ovvsHnswIndex_t*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsHnswSearch(ovvsResources_t, ovvsHnswIndex_t, const float*, int64_t,
                                   int64_t, int32_t, int64_t*, float*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsHnswSerialize(ovvsHnswIndex_t, const char*) { return kNo; }
OVVS_API ovvsStatus ovvsHnswDeserialize(ovvsResources_t, const char*, ovvsHnswIndex_t*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsHnswDestroy(ovvsHnswIndex_t index) { return destroy_none(index); }
OVVS_API ovvsStatus ovvsVamanaBuild(ovvsResources_t, const float*, int64_t, int64_t, ovvsMetric,
                                    int32_t, float, ovvsVamanaIndex_t*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsVamanaSearch(ovvsResources_t, ovvsVamanaIndex_t, const float*, int64_t,
                                     int64_t, int32_t, const uint8_t*, int64_t*, float*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsVamanaDestroy(ovvsVamanaIndex_t index) { return destroy_none(index); }
OVVS_API ovvsStatus ovvsKMeansFit(ovvsResources_t, const float*, int64_t, int64_t, int32_t,
                                  int32_t, ovvsKMeansModel_t*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsKMeansPredict(ovvsResources_t, ovvsKMeansModel_t, const float*, int64_t,
                                      int64_t*, float*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsKMeansDestroy(ovvsKMeansModel_t model) { return destroy_none(model); }
OVVS_API ovvsStatus ovvsBatcherCreate(ovvsResources_t, ovvsBruteForceIndex_t, int32_t, int32_t,
                                      ovvsBatcher_t*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsBatcherSearch(ovvsBatcher_t, const float*, int64_t, int64_t, int64_t*,
                                      float*) {
  return kNo;
}
OVVS_API ovvsStatus ovvsBatcherDestroy(ovvsBatcher_t batcher) { return destroy_none(batcher); }

}  // extern "C"
