// C++ consumer of include/ovvs/ovvs.hpp (the reference's tests/consumer.cpp:118
// drives ovvs::IvfPqIndex the same way). Usage: consumer_cpp <ipq1> [search];
// with "search" it runs the legacy-file query on the GPU and checks the
// reference's known answer (ids 1, 2; distances 0.01, 0.81), then builds and
// searches a small ovvs::ScannIndex.
#include <ovvs/ovvs.hpp>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  ovvs::Resources res;
  ovvs::IvfPqIndex ix(res, argv[1]);
  try {
    ovvs::IvfPqIndex bad(res, "/nonexistent/ipq1");
    return 3;
  } catch (const std::runtime_error& e) {
    if (std::strcmp(e.what(), "io error") != 0) return 4;
  }
  if (argc > 2 && std::strcmp(argv[2], "search") == 0) {
    const float q[2] = {1.1f, 0.f};
    int64_t ids[2] = {-1, -1};
    float d[2] = {0, 0};
    ix.search(q, 1, 2, 1, 4, ids, d);
    if (ids[0] != 1 || ids[1] != 2 || std::fabs(d[0] - 0.01f) > 1e-5f ||
        std::fabs(d[1] - 0.81f) > 1e-5f)
      return 5;
    if (res.last_device() != OVVS_DEVICE_GPU) return 6;
    // ScaNN-style index (the reference's tests/consumer.cpp:135 builds one the same
    // way): every list probed and krefine = n find a row itself at distance 0.
    float rows[40 * 8];
    for (int i = 0; i < 40 * 8; ++i) rows[i] = static_cast<float>((i * 7919) % 1009) * 0.01f - 5.f;
    ovvs::ScannIndex scann(res, rows, 40, 8, OVVS_METRIC_L2_EXPANDED, 4, 2);
    int64_t sid[3] = {-1, -1, -1};
    float sd[3] = {-1, -1, -1};
    scann.search(rows + 5 * 8, 1, 3, 4, 40, sid, sd);
    if (sid[0] != 5 || sd[0] != 0.f || !(sd[1] >= sd[0]) || !(sd[2] >= sd[1])) return 7;
  }
  std::puts("c++ consumer ok");
  return 0;
}
