/* C consumer of the libovvs ABI: compiles against include/ovvs/ovvs.h with a C
 * compiler and exercises the GPU-free part of the IVF-PQ lifecycle (the
 * reference's tests/consumer.c:8-9,65-68 pins the same stats layout).
 * Usage: consumer <ipq1 file> <output file>; exit status 0 on success. */
#include <ovvs/ovvs.h>

#include <assert.h>
#include <stddef.h>
#include <stdio.h>
#include <string.h>

_Static_assert(sizeof(ovvsIvfPqSearchStatsV1) == 200, "stats V1 is 200 bytes");
_Static_assert(offsetof(ovvsIvfPqSearchStatsV1, successful_calls) == 8, "stats V1 layout");
_Static_assert(offsetof(ovvsIvfPqSearchStatsV1, gpu_wait_calls) == 192, "stats V1 layout");
_Static_assert(OVVS_IVF_PQ_SEARCH_STATS_ABI_V1 == 1u, "stats V1 version");
_Static_assert(OVVS_STATUS_IO == 8 && OVVS_POLICY_FORCE_CPU == 6 && OVVS_METRIC_LP_UNEXPANDED == 5,
               "enum values");

int main(int argc, char** argv) {
  if (argc != 3) return 2;
  if (strcmp(ovvsGetVersion(), OVVS_VERSION_STRING) != 0) return 3;
  if (strcmp(ovvsStatusString(OVVS_STATUS_IO), "io error") != 0) return 4;
  ovvsResources_t res = NULL;
  if (ovvsResourcesCreate(&res) != OVVS_STATUS_SUCCESS) return 5;
  ovvsIvfPqSearchStatsV1 st;
  memset(&st, 0xff, sizeof(st));
  if (ovvsResourcesIvfPqSearchStatsV1(res, &st) != OVVS_STATUS_SUCCESS) return 6;
  if (st.abi_version != 1u || st.struct_size != 200u || st.successful_calls != 0) return 7;
  ovvsIvfPqIndex_t ix = NULL;
  if (ovvsIvfPqDeserialize(res, argv[1], &ix) != OVVS_STATUS_SUCCESS || !ix) return 8;
  if (ovvsIvfPqSerialize(ix, argv[2]) != OVVS_STATUS_SUCCESS) return 9;
  ovvsIvfPqDestroy(ix);
  uint8_t bits[2];
  const int64_t ids[3] = {0, 9, 42};
  if (ovvsBitsetFromAllowList(10, ids, 3, bits) != OVVS_STATUS_SUCCESS) return 10;
  if (bits[0] != 0x01 || bits[1] != 0x02) return 11;
  ovvsResourcesDestroy(res);
  puts("c consumer ok");
  return 0;
}
