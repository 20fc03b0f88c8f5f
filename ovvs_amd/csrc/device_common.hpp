// device_common.hpp — device helpers shared by the libovvs gfx950 kernels.
//
// Arithmetic rule for every kernel in this library: fp32 products and sums are
// rounded one operation at a time, in the reference's order (no FMA
// contraction: the kernels are compiled with -ffp-contract=off and this header
// turns contraction off again for the translation unit).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace ovvs_dev {

constexpr uint64_t kNoKey = ~0ull;

// Order-preserving 32-bit key of an fp32 score for the reference's total order
// (reference src/prim/cpu/cpu_prims.cpp:24-32): numbers ascending with -0 == +0,
// every NaN after +inf and equal to each other. Ties are broken by the low word
// the caller packs next to it.
__device__ __forceinline__ uint32_t score_key(float s) {
  if (s != s) return 0xffffffffu;
  uint32_t u = __float_as_uint(s);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t make_key(float s, uint32_t ordinal) {
  return (static_cast<uint64_t>(score_key(s)) << 32) | ordinal;
}

// Left-to-right fp32 sums from +0, one rounding per operation.
__device__ __forceinline__ float seq_dot(const float* a, const float* b, int d) {
  float s = 0.f;
  for (int i = 0; i < d; ++i) s = s + a[i] * b[i];
  return s;
}

__device__ __forceinline__ float seq_l2sq(const float* a, const float* b, int d) {
  float s = 0.f;
  for (int i = 0; i < d; ++i) {
    const float t = a[i] - b[i];
    s = s + t * t;
  }
  return s;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), mask, 64);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), mask, 64);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
  const uint32_t lo = __shfl(static_cast<uint32_t>(v), src, 64);
  const uint32_t hi = __shfl(static_cast<uint32_t>(v >> 32), src, 64);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x & 63u); }

}  // namespace ovvs_dev
