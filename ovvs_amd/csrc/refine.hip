// refine.hip — exact re-rank of the IVF-PQ shortlist on gfx950.
//
// Reference behaviour (src/neighbors/indexes.cpp:1067-1096): gather the dataset
// rows of the shortlisted ids, compute the index metric exactly
// (src/prim/mixer.cpp:177-221 for the expanded metrics, src/internal.hpp:240-272
// for the others), keep the first min(k, kr) under the total order on
// (distance, shortlist rank), flip the sign back for inner product, and pad the
// remaining slots with (-1, +inf).
//
// One wave64 per query, or four per wave for shortlists of at most 16 (plus, when
// asked, up to 64 workgroups that sum the scan's per-query statistics into the
// search counters): the query row is staged in LDS, each lane scores
// shortlist entries i = lane, lane+64, ... with left-to-right fp32 sums (rows
// read 16 bytes at a time when dim % 4 == 0), the (key, rank) pairs are sorted in
// LDS by a single-wave bitonic network, and the first k slots are written. LDS is
// sized to the shortlist (a power of two >= krefine), so short shortlists keep
// many waves resident. Longer shortlists with dim % 4 == 0 stage their rows through
// LDS in chunks read by whole-row 16-byte loads (k_refine_staged).
#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"

using namespace ovvs_dev;

namespace {

enum { kL2 = 0, kL2Sqrt = 1, kIP = 2, kCosine = 3, kHamming = 4, kLp = 5 };

// std::max semantics for floats: keeps `a` unless a < b.
__device__ __forceinline__ float ref_max(float a, float b) { return (a < b) ? b : a; }

// Left-to-right dot product; q (LDS) and x are 16-byte aligned when dim % 4 == 0.
__device__ __forceinline__ float dot(const float* __restrict__ q, const float* __restrict__ x,
                                     int dim) {
  return (dim & 3) == 0 ? seq_dot_v4(q, x, dim) : seq_dot(q, x, dim);
}

__device__ float metric_value(int metric, const float* __restrict__ q,
                              const float* __restrict__ x, int dim, float qn, float xn) {
  switch (metric) {
    case kL2:
      return (qn + xn) - 2.f * dot(q, x, dim);
    case kIP:
      return -dot(q, x, dim);
    case kCosine: {
      // __builtin_sqrtf and '/' lower to correctly rounded sequences (no
      // fast-math, no approximate-sqrt flags), as x86 sqrtss/divss are.
      const float ip = dot(q, x, dim);
      const float a = __builtin_sqrtf(ref_max(qn, 1e-12f));
      const float b = __builtin_sqrtf(ref_max(xn, 1e-12f));
      return 1.f - ip / (a * b);
    }
    case kL2Sqrt:
      return __builtin_sqrtf(seq_l2sq(q, x, dim));
    case kHamming: {
      int s = 0;
      for (int i = 0; i < dim; ++i) s += static_cast<int>((q[i] >= 0.f) != (x[i] >= 0.f));
      return static_cast<float>(s);
    }
    case kLp: {
      // Minkowski p = 2 as the search passes it (reference indexes.cpp:1076):
      // (sum |q-x|^2)^(1/2). The reference evaluates both powers with powf;
      // |t|^2 and s^(1/2) are computed here as the correctly rounded t*t and
      // sqrt(s), which powf returns too except when its result lies within its
      // own error bound of a rounding midpoint.
      float s = 0.f;
      for (int i = 0; i < dim; ++i) {
        const float t = fabsf(q[i] - x[i]);
        s = s + t * t;
      }
      return __builtin_sqrtf(s);
    }
    default:
      return seq_l2sq(q, x, dim);
  }
}

constexpr size_t align16(size_t b) { return (b + 15) & ~static_cast<size_t>(15); }

// LDS: query row [round4(dim)] f32 | keys [M] u64 | vals [M] f32.
size_t refine_lds(int dim, int M) {
  return align16(static_cast<size_t>((dim + 3) & ~3) * 4) + static_cast<size_t>(M) * 12;
}

// Workgroups past the queries sum the scan's per-query statistics (a wave each,
// strided over the queries, one atomic per counter and workgroup).
__device__ void refine_stats(const OvvsRefineArgs& a, int64_t g, int64_t ng) {
  unsigned long long acc[4] = {0, 0, 0, 0};
  for (int64_t q = g * 64 + threadIdx.x; q < a.nq; q += ng * 64) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] += static_cast<uint32_t>(a.stats[q * 4 + i]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc[i] += shfl_xor_u64(acc[i], o);
  }
  if (threadIdx.x == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (acc[i]) atomicAdd(&a.counters[i], acc[i]);
  }
}

// Sorts the M keys in LDS (one wave's bitonic network) and writes the first k
// outputs of query q: (id, distance) of the smallest keys, (-1, +inf) past cnt.
// The id of entry i is lid[i] when lid is given, else looked up again.
__device__ void sort_and_publish(const OvvsRefineArgs& a, int64_t q, uint64_t* keys,
                                 const float* vals, int M, int cnt, const int64_t* lid) {
  const int lane = threadIdx.x;
  __syncthreads();
  for (int k = 2; k <= M; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = lane; i < M; i += 64) {
        const int p = i ^ j;
        if (p > i) {
          const uint64_t x = keys[i], y = keys[p];
          if ((x > y) == ((i & k) == 0)) {
            keys[i] = y;
            keys[p] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  const int64_t kk = a.k < cnt ? a.k : cnt;
  for (int64_t t = lane; t < a.k; t += 64) {
    int64_t id = -1;
    float d = __builtin_inff();
    if (t < kk && keys[t] != kNoKey) {
      const int i = static_cast<int>(keys[t] & 0xffffffffu);
      id = lid ? lid[i] : a.ids[a.short_pos[q * a.K + i]];
      d = a.metric == kIP ? -vals[i] : vals[i];
    }
    a.out_ids[q * a.k + t] = id;
    a.out_dist[q * a.k + t] = d;
  }
}

// With counters_out (host memory mapped into the device's address space), the last
// workgroup of the launch to finish copies the five search counters there once
// every other workgroup's atomics are done (each fences before taking its ticket),
// so the host reads them after its stream synchronization without a copy.
// With stamps, the last workgroup also copies the stage stamps and its end time to
// counters_out[8, 13).
__device__ void publish_counters(const OvvsRefineArgs& a) {
  if (!a.counters_out) return;
  __shared__ bool last;
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    last = atomicAdd(a.done, 1u) == gridDim.x - 1u;
  }
  __syncthreads();
  if (last) {
    __threadfence();
    if (threadIdx.x < 5)
      a.counters_out[threadIdx.x] =
          __hip_atomic_load(a.counters + threadIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (a.stamps && threadIdx.x >= 8 && threadIdx.x < 13)
      a.counters_out[threadIdx.x] =
          threadIdx.x == 12 ? wall_clock64()
                            : __hip_atomic_load(a.stamps + (threadIdx.x - 8), __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
  }
}

__device__ __forceinline__ void stamp_start(const OvvsRefineArgs& a) {
  if (a.stamps && blockIdx.x == 0 && threadIdx.x == 0) a.stamps[3] = wall_clock64();
}

__device__ void refine_one(const OvvsRefineArgs& a, int Mmax) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* qs = reinterpret_cast<float*>(smem);
  uint64_t* keys =
      reinterpret_cast<uint64_t*>(smem + align16(static_cast<size_t>((a.dim + 3) & ~3) * 4));
  float* vals = reinterpret_cast<float*>(keys + Mmax);
  const int64_t q = blockIdx.x;
  const int lane = threadIdx.x;
  for (int t = lane; t < a.dim; t += 64) qs[t] = a.queries[q * a.dim + t];
  __syncthreads();
  const float* __restrict__ qv = qs;
  int cnt = a.short_count[q];
  cnt = cnt < 0 ? 0 : (cnt > a.K ? a.K : cnt);
  int M = 1;
  while (M < cnt) M <<= 1;
  for (int i = lane; i < M; i += 64) {
    uint64_t key = kNoKey;
    if (i < cnt) {
      // Positions come from the scan; one out of range is reported (the search
      // then fails) instead of being dereferenced.
      const int32_t pos = a.short_pos[q * a.K + i];
      const int64_t id = (pos >= 0 && pos < a.positions) ? a.ids[pos] : -1;
      if (id >= 0 && id < a.n) {
        const float v = metric_value(a.metric, qv, a.dataset + id * a.dim, a.dim, a.qnorm[q],
                                     a.xnorm[id]);
        key = make_key(v, static_cast<uint32_t>(i));
        vals[i] = v;
      } else {
        atomicAdd(a.invalid, 1ull);
      }
    }
    keys[i] = key;
  }
  sort_and_publish(a, q, keys, vals, M, cnt, nullptr);
}

__global__ __launch_bounds__(64) void k_refine(const OvvsRefineArgs a, int Mmax) {
  stamp_start(a);
  if (static_cast<int64_t>(blockIdx.x) >= a.nq) {
    refine_stats(a, blockIdx.x - a.nq, gridDim.x - a.nq);
  } else {
    refine_one(a, Mmax);
  }
  publish_counters(a);
}

// Shortlists longer than 16 with dim % 4 == 0 (dim <= 4 * kStageVecMax): the rows
// of R entries at a time are read by the whole wave, consecutive lanes taking
// consecutive 16-byte vectors of a row (a load instruction covers whole rows instead
// of 64 scattered vectors), kStageLoads loads in flight per lane, into LDS rows
// padded by 16 bytes; each lane then scores its own entry from LDS with the same
// metric_value, so the sums and their order are those of k_refine.
constexpr int kStageRowsMax = 64;
constexpr int kStageLoads = 8;
// Rows staged per chunk: 8 KB per wave keeps more waves resident than 16 KB (C3's
// refine took 0.147 ms so against 0.175; 4 KB: 0.158, 24 KB: 0.232).
constexpr size_t kStageBytes = 8 * 1024;
constexpr int kStageVecMax = 255;

// LDS: query row [dim] f32 | keys [M] u64 | vals [M] f32 | ids of the entries [M]
// i64 | rows [R * stride] f32.
struct StagedCarve {
  size_t keys_off, vals_off, rid_off, rows_off, lds;
};

__host__ __device__ inline StagedCarve staged_carve(int dim, int M, int R, int stride) {
  StagedCarve c;
  c.keys_off = align16(static_cast<size_t>(dim) * 4);
  c.vals_off = c.keys_off + static_cast<size_t>(M) * 8;
  c.rid_off = align16(c.vals_off + static_cast<size_t>(M) * 4);
  c.rows_off = align16(c.rid_off + static_cast<size_t>(M) * 8);
  c.lds = c.rows_off + static_cast<size_t>(R) * stride * 4;
  return c;
}

__device__ void refine_staged_one(const OvvsRefineArgs& a, int Mmax, int R, int stride) {
  extern __shared__ __align__(16) unsigned char smem[];
  const StagedCarve L = staged_carve(a.dim, Mmax, R, stride);
  float* qs = reinterpret_cast<float*>(smem);
  uint64_t* keys = reinterpret_cast<uint64_t*>(smem + L.keys_off);
  float* vals = reinterpret_cast<float*>(smem + L.vals_off);
  int64_t* rid = reinterpret_cast<int64_t*>(smem + L.rid_off);
  float* rows = reinterpret_cast<float*>(smem + L.rows_off);
  const int64_t q = blockIdx.x;
  const int lane = threadIdx.x;
  for (int t = lane; t < a.dim; t += 64) qs[t] = a.queries[q * a.dim + t];
  int cnt = a.short_count[q];
  cnt = cnt < 0 ? 0 : (cnt > a.K ? a.K : cnt);
  int M = 1;
  while (M < cnt) M <<= 1;
  // Vector j = lane + 64 i of a chunk is vector j % nv of its row j / nv; the lane
  // steps (de, dv) per 64.
  const int nv = a.dim >> 2;
  const int de = 64 / nv, dv = 64 - de * nv;
  const int e0 = lane / nv, v0 = lane - e0 * nv;
  // The ids of all entries first (-1 for an invalid one). Positions come from the
  // scan; one out of range is reported (the search then fails) instead of being
  // dereferenced.
  for (int i = lane; i < cnt; i += 64) {
    const int32_t pos = a.short_pos[q * a.K + i];
    const int64_t id = (pos >= 0 && pos < a.positions) ? a.ids[pos] : -1;
    const bool ok = id >= 0 && id < a.n;
    if (!ok) atomicAdd(a.invalid, 1ull);
    rid[i] = ok ? id : -1;
  }
  __syncthreads();
  for (int c0 = 0; c0 < cnt; c0 += R) {
    const int n = cnt - c0 < R ? cnt - c0 : R;
    const int total = n * nv;
    int e = e0, v = v0;
    for (int base = 0; base < total; base += 64 * kStageLoads) {
      float4 x[kStageLoads];
      int at[kStageLoads];
#pragma unroll
      for (int u = 0; u < kStageLoads; ++u) {
        const bool in = base + 64 * u + lane < total;
        const int64_t id = in ? rid[c0 + e] : -1;
        x[u] = id >= 0 ? *reinterpret_cast<const float4*>(a.dataset + id * a.dim + 4 * v)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
        at[u] = in ? e * stride + 4 * v : -1;
        e += de;
        v += dv;
        if (v >= nv) {
          v -= nv;
          ++e;
        }
      }
#pragma unroll
      for (int u = 0; u < kStageLoads; ++u)
        if (at[u] >= 0) *reinterpret_cast<float4*>(rows + at[u]) = x[u];
    }
    __syncthreads();
    if (lane < n) {
      const int64_t id = rid[c0 + lane];
      uint64_t key = kNoKey;
      if (id >= 0) {
        const float val = metric_value(a.metric, qs, rows + lane * stride, a.dim, a.qnorm[q], a.xnorm[id]);
        key = make_key(val, static_cast<uint32_t>(c0 + lane));
        vals[c0 + lane] = val;
      }
      keys[c0 + lane] = key;
    }
    __syncthreads();
  }
  for (int i = cnt + lane; i < M; i += 64) keys[i] = kNoKey;
  sort_and_publish(a, q, keys, vals, M, cnt, rid);
}

__global__ __launch_bounds__(64) void k_refine_staged(const OvvsRefineArgs a, int Mmax, int R,
                                                      int stride) {
  stamp_start(a);
  if (static_cast<int64_t>(blockIdx.x) >= a.nq) {
    refine_stats(a, blockIdx.x - a.nq, gridDim.x - a.nq);
  } else {
    refine_staged_one(a, Mmax, R, stride);
  }
  publish_counters(a);
}

// Shortlists of at most 16 (M <= 16): four queries per wave64, 16 lanes each, so a
// batch needs a quarter of the waves. Lane i of a group scores entry i; the 16 keys
// of each group are sorted by the same bitonic network in LDS.
constexpr int kGroupLanes = 16;
constexpr int kGroups = 64 / kGroupLanes;

size_t refine4_lds(int dim) {
  return align16(static_cast<size_t>(kGroups) * ((dim + 3) & ~3) * 4) +
         static_cast<size_t>(64) * 12;
}

__device__ void refine4_one(const OvvsRefineArgs& a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int dq = (a.dim + 3) & ~3;
  float* qs_all = reinterpret_cast<float*>(smem);
  uint64_t* keys_all =
      reinterpret_cast<uint64_t*>(smem + align16(static_cast<size_t>(kGroups) * dq * 4));
  float* vals_all = reinterpret_cast<float*>(keys_all + 64);
  const int lane = threadIdx.x;
  const int grp = lane / kGroupLanes, i = lane % kGroupLanes;
  const int64_t q = static_cast<int64_t>(blockIdx.x) * kGroups + grp;
  const bool qok = q < a.nq;
  float* qs = qs_all + grp * dq;
  uint64_t* keys = keys_all + grp * kGroupLanes;
  float* vals = vals_all + grp * kGroupLanes;
  for (int t = i; t < a.dim; t += kGroupLanes) qs[t] = qok ? a.queries[q * a.dim + t] : 0.f;
  __syncthreads();
  int cnt = qok ? a.short_count[q] : 0;
  cnt = cnt < 0 ? 0 : (cnt > a.K ? a.K : cnt);
  uint64_t key = kNoKey;
  if (i < cnt) {
    const int32_t pos = a.short_pos[q * a.K + i];
    const int64_t id = (pos >= 0 && pos < a.positions) ? a.ids[pos] : -1;
    if (id >= 0 && id < a.n) {
      const float v = metric_value(a.metric, qs, a.dataset + id * a.dim, a.dim, a.qnorm[q],
                                   a.xnorm[id]);
      key = make_key(v, static_cast<uint32_t>(i));
      vals[i] = v;
    } else {
      atomicAdd(a.invalid, 1ull);
    }
  }
  keys[i] = key;
  __syncthreads();
  for (int k = 2; k <= kGroupLanes; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      const int p = i ^ j;
      if (p > i) {
        const uint64_t x = keys[i], y = keys[p];
        if ((x > y) == ((i & k) == 0)) {
          keys[i] = y;
          keys[p] = x;
        }
      }
      __syncthreads();
    }
  }
  if (!qok) return;
  const int64_t kk = a.k < cnt ? a.k : cnt;
  for (int64_t t = i; t < a.k; t += kGroupLanes) {
    int64_t id = -1;
    float d = __builtin_inff();
    if (t < kk && keys[t] != kNoKey) {
      const int e = static_cast<int>(keys[t] & 0xffffffffu);
      id = a.ids[a.short_pos[q * a.K + e]];
      d = a.metric == kIP ? -vals[e] : vals[e];
    }
    a.out_ids[q * a.k + t] = id;
    a.out_dist[q * a.k + t] = d;
  }
}

__global__ __launch_bounds__(64) void k_refine4(const OvvsRefineArgs a) {
  stamp_start(a);
  const int64_t nblk = (a.nq + kGroups - 1) / kGroups;
  if (static_cast<int64_t>(blockIdx.x) >= nblk) {
    refine_stats(a, blockIdx.x - nblk, gridDim.x - nblk);
  } else {
    refine4_one(a);
  }
  publish_counters(a);
}

}  // namespace

extern "C" hipError_t ovvs_hip_refine(const OvvsRefineArgs* args, hipStream_t stream) {
  if (!args) return hipErrorInvalidValue;
  const OvvsRefineArgs& a = *args;
  if (a.nq <= 0) return hipSuccess;
  if (!a.queries || !a.qnorm || !a.dataset || !a.xnorm || !a.ids || !a.short_pos ||
      !a.short_count || !a.out_ids || !a.out_dist || !a.invalid || a.n <= 0 || a.positions <= 0 ||
      a.dim <= 0 ||
      a.K <= 0 ||
      a.K > OVVS_HIP_MAX_REFINE || a.k <= 0 || a.nq > 0x7fffffff - 64 ||
      (a.stats == nullptr) != (a.counters == nullptr) ||
      (a.counters_out != nullptr && (a.counters == nullptr || a.done == nullptr)))
    return hipErrorInvalidValue;
  int M = 1;
  while (M < a.K) M <<= 1;
  const int64_t stat_groups = a.stats ? std::min<int64_t>(64, (a.nq + 63) / 64) : 0;
  if (M <= kGroupLanes) {
    const size_t lds4 = refine4_lds(a.dim);
    if (lds4 <= 65536) {
      const int64_t blocks = (a.nq + kGroups - 1) / kGroups + stat_groups;
      hipLaunchKernelGGL(k_refine4, dim3(static_cast<uint32_t>(blocks)), dim3(64), lds4, stream, a);
      return hipGetLastError();
    }
  }
  if ((a.dim & 3) == 0 && (a.dim >> 2) <= kStageVecMax) {
    const int stride = a.dim + 4;
    // At least four rows per chunk (dims up to 1020: 16 KB).
    const int R = static_cast<int>(std::min<size_t>(
        kStageRowsMax, std::max<size_t>(4, kStageBytes / (static_cast<size_t>(stride) * 4))));
    const StagedCarve c = staged_carve(a.dim, M, R, stride);
    if (R >= 4 && c.lds <= 65536) {
      hipLaunchKernelGGL(k_refine_staged, dim3(static_cast<uint32_t>(a.nq + stat_groups)), dim3(64),
                         c.lds, stream, a, M, R, stride);
      return hipGetLastError();
    }
  }
  const size_t lds = refine_lds(a.dim, M);
  if (lds > 160u * 1024u) return hipErrorInvalidValue;
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_refine),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(k_refine, dim3(static_cast<uint32_t>(a.nq + stat_groups)), dim3(64), lds,
                     stream, a, M);
  return hipGetLastError();
}
