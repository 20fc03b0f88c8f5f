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

// seq_dot(q, x, d) for d % 4 == 0 with both rows 16-byte aligned: the same
// left-to-right sum, each row read 16 bytes at a time, four vectors ahead.
__device__ __forceinline__ float seq_dot_v4(const float* __restrict__ q,
                                            const float* __restrict__ x, int d) {
  const float4* q4 = reinterpret_cast<const float4*>(q);
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float s = 0.f;
  int i = 0;
  for (; i + 4 <= d / 4; i += 4) {
    float4 v[4], w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = x4[i + j];
      w[j] = q4[i + j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s = s + w[j].x * v[j].x;
      s = s + w[j].y * v[j].y;
      s = s + w[j].z * v[j].z;
      s = s + w[j].w * v[j].w;
    }
  }
  for (; i < d / 4; ++i) {
    const float4 v = x4[i], w = q4[i];
    s = s + w.x * v.x;
    s = s + w.y * v.y;
    s = s + w.z * v.z;
    s = s + w.w * v.w;
  }
  return s;
}

// seq_dot(q, x, d) for d % 4 == 0 with both rows 16-byte aligned (q typically in LDS,
// x a row in global memory): the same left-to-right sum from +0, x read kChunk 16-byte
// vectors at a time with all of a chunk's loads issued before its terms are added, so
// that a row costs a few memory round trips instead of one per four vectors.
template <int kChunk = 12>
__device__ __forceinline__ float seq_dot_v4_chunked(const float* q, const float* __restrict__ x, int d) {
  const float4* q4 = reinterpret_cast<const float4*>(q);
  const float4* x4 = reinterpret_cast<const float4*>(x);
  const int n4 = d >> 2;
  float s = 0.f;
  for (int i = 0; i < n4; i += kChunk) {
    float4 v[kChunk];
#pragma unroll
    for (int j = 0; j < kChunk; ++j) v[j] = x4[i + j < n4 ? i + j : n4 - 1];
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      if (i + j < n4) {
        const float4 w = q4[i + j];
        s = s + w.x * v[j].x;
        s = s + w.y * v[j].y;
        s = s + w.z * v[j].z;
        s = s + w.w * v[j].w;
      }
    }
  }
  return s;
}

// seq_dot_v4 with the row x (global memory) double-buffered: the next four
// vectors are requested before the current four are summed, so one memory round
// trip overlaps the next. q is read from LDS as it is consumed. Same sum, same
// order.
__device__ __forceinline__ float seq_dot_v4_ahead(const float* __restrict__ q,
                                                  const float* __restrict__ x, int d) {
  const float4* q4 = reinterpret_cast<const float4*>(q);
  const float4* x4 = reinterpret_cast<const float4*>(x);
  const int n4 = d / 4;
  float s = 0.f;
  int i = 0;
  if (n4 >= 4) {
    float4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = x4[j];
    for (i = 4; i + 4 <= n4; i += 4) {
      float4 nv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) nv[j] = x4[i + j];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 w = q4[i - 4 + j];
        s = s + w.x * v[j].x;
        s = s + w.y * v[j].y;
        s = s + w.z * v[j].z;
        s = s + w.w * v[j].w;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = nv[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 w = q4[i - 4 + j];
      s = s + w.x * v[j].x;
      s = s + w.y * v[j].y;
      s = s + w.z * v[j].z;
      s = s + w.w * v[j].w;
    }
  }
  for (; i < n4; ++i) {
    const float4 v = x4[i], w = q4[i];
    s = s + w.x * v.x;
    s = s + w.y * v.y;
    s = s + w.z * v.z;
    s = s + w.w * v.w;
  }
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
