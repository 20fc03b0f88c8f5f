// peaks.hip — micro-benchmarks of the MI355X ceilings the search kernels are
// measured against (bench.py loads ovvs_amd/lib/libovvs_peaks.so; libovvs does not
// use it):
//   peaks_hbm_read    streaming read of a device buffer (16-byte loads, four in
//                     flight per lane), GB/s
//   peaks_mfma_bf16   v_mfma_f32_16x16x32_bf16 on register operands, eight
//                     independent accumulators per wave, TFLOP/s (dense)
//   peaks_mfma_f32    v_mfma_f32_16x16x4_f32 the same way, TFLOP/s
//   peaks_valu        independent fp32 multiply and add chains (one wave64 VALU
//                     instruction each), giga wave64 instructions per second
// Each runs `reps` timed launches (HIP events on its own stream) after one
// warm-up launch and reports the best.
#include <hip/hip_runtime.h>

#include <stdint.h>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(256) void k_read(const uint4* __restrict__ src, size_t n16,
                                              uint32_t* __restrict__ out) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^
           d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const uint4 a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (acc == 0x9e3779b9u) out[blockIdx.x] = acc;  // keeps the loads live
}

__global__ __launch_bounds__(256) void k_mfma_bf16(int iters, float* __restrict__ out) {
  bf16x8 a, b;
  for (int j = 0; j < 8; ++j) {
    a[j] = static_cast<__bf16>(1.0f + 0.001f * static_cast<float>(threadIdx.x + j));
    b[j] = static_cast<__bf16>(0.5f - 0.001f * static_cast<float>(j));
  }
  f32x4 acc[8];
  for (int r = 0; r < 8; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[r], 0, 0, 0);
  }
  float s = 0.f;
  for (int r = 0; r < 8; ++r) s = s + acc[r][0] + acc[r][1] + acc[r][2] + acc[r][3];
  if (s == 12345.f) out[blockIdx.x] = s;
}

__global__ __launch_bounds__(256) void k_mfma_f32(int iters, float* __restrict__ out) {
  const float a = 1.0f + 0.001f * static_cast<float>(threadIdx.x);
  const float b = 0.5f;
  f32x4 acc[8];
  for (int r = 0; r < 8; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[r] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[r], 0, 0, 0);
  }
  float s = 0.f;
  for (int r = 0; r < 8; ++r) s = s + acc[r][0] + acc[r][1] + acc[r][2] + acc[r][3];
  if (s == 12345.f) out[blockIdx.x] = s;
}

// 8 independent chains, each step a multiply then an add (contraction is off for
// this file's build), 16 VALU instructions per iteration.
__global__ __launch_bounds__(256) void k_valu(int iters, float* __restrict__ out) {
  float x[8];
  for (int r = 0; r < 8; ++r) x[r] = 1.0f + 1e-3f * static_cast<float>(threadIdx.x + r);
  const float m = 0.9999f, c = 1e-4f;
#pragma unroll 4
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      x[r] = x[r] * m;
      x[r] = x[r] + c;
    }
  }
  float s = 0.f;
  for (int r = 0; r < 8; ++r) s = s + x[r];
  if (s == 12345.f) out[blockIdx.x] = s;
}

// Best of `reps` timed runs of launch() in milliseconds (0 on error).
template <class F>
double best_ms(int reps, F launch) {
  hipStream_t s = nullptr;
  if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return 0.0;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  double best = 0.0;
  if (hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) {
    launch(s);  // warm-up
    if (hipStreamSynchronize(s) == hipSuccess) {
      for (int r = 0; r < reps; ++r) {
        (void)hipEventRecord(e0, s);
        launch(s);
        (void)hipEventRecord(e1, s);
        if (hipEventSynchronize(e1) != hipSuccess) {
          best = 0.0;
          break;
        }
        float ms = 0.f;
        (void)hipEventElapsedTime(&ms, e0, e1);
        if (best == 0.0 || ms < best) best = ms;
      }
    }
  }
  if (hipGetLastError() != hipSuccess) best = 0.0;
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipStreamDestroy(s);
  return best;
}

int cu_count() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return cus;
}

}  // namespace

#define PEAKS_API __attribute__((visibility("default")))

extern "C" {

// src: device buffer of `bytes` (a multiple of 16); scratch: device, one uint32 per
// workgroup (gridDim <= 65536). Returns GB/s (1e9 bytes), 0 on error.
PEAKS_API double peaks_hbm_read(const void* src, size_t bytes, void* scratch, int reps) {
  const int cus = cu_count();
  if (!src || !scratch || bytes < 16 || cus <= 0) return 0.0;
  const unsigned grid = static_cast<unsigned>(cus) * 16u;
  const size_t n16 = bytes / 16;
  const double ms = best_ms(reps, [&](hipStream_t s) {
    hipLaunchKernelGGL(k_read, dim3(grid), dim3(256), 0, s, static_cast<const uint4*>(src), n16,
                       static_cast<uint32_t*>(scratch));
  });
  return ms > 0.0 ? static_cast<double>(n16 * 16) / (ms * 1e-3) / 1e9 : 0.0;
}

// scratch: device, one float per workgroup (8 workgroups of 4 waves per CU).
PEAKS_API double peaks_mfma_bf16(void* scratch, int iters, int reps) {
  const int cus = cu_count();
  if (!scratch || iters <= 0 || cus <= 0) return 0.0;
  const unsigned grid = static_cast<unsigned>(cus) * 8u;
  const double ms = best_ms(reps, [&](hipStream_t s) {
    hipLaunchKernelGGL(k_mfma_bf16, dim3(grid), dim3(256), 0, s, iters, static_cast<float*>(scratch));
  });
  const double flops = static_cast<double>(grid) * 4.0 * iters * 8.0 * (16.0 * 16.0 * 32.0 * 2.0);
  return ms > 0.0 ? flops / (ms * 1e-3) / 1e12 : 0.0;
}

PEAKS_API double peaks_mfma_f32(void* scratch, int iters, int reps) {
  const int cus = cu_count();
  if (!scratch || iters <= 0 || cus <= 0) return 0.0;
  const unsigned grid = static_cast<unsigned>(cus) * 8u;
  const double ms = best_ms(reps, [&](hipStream_t s) {
    hipLaunchKernelGGL(k_mfma_f32, dim3(grid), dim3(256), 0, s, iters, static_cast<float*>(scratch));
  });
  const double flops = static_cast<double>(grid) * 4.0 * iters * 8.0 * (16.0 * 16.0 * 4.0 * 2.0);
  return ms > 0.0 ? flops / (ms * 1e-3) / 1e12 : 0.0;
}

// Giga wave64 VALU instructions per second over the whole GPU.
PEAKS_API double peaks_valu(void* scratch, int iters, int reps) {
  const int cus = cu_count();
  if (!scratch || iters <= 0 || cus <= 0) return 0.0;
  const unsigned grid = static_cast<unsigned>(cus) * 8u;
  const double ms = best_ms(reps, [&](hipStream_t s) {
    hipLaunchKernelGGL(k_valu, dim3(grid), dim3(256), 0, s, iters, static_cast<float*>(scratch));
  });
  const double insts = static_cast<double>(grid) * 4.0 * iters * 16.0;
  return ms > 0.0 ? insts / (ms * 1e-3) / 1e9 : 0.0;
}

// Shader clock (MHz) and compute units of the current device.
PEAKS_API int peaks_device_info(int* clock_mhz, int* cus) {
  int dev = 0;
  if (!clock_mhz || !cus || hipGetDevice(&dev) != hipSuccess) return 1;
  int khz = 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeClockRate, dev) != hipSuccess) return 1;
  *clock_mhz = khz / 1000;
  *cus = cu_count();
  return 0;
}

}  // extern "C"
