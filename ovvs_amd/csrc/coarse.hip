// coarse.hip — coarse probe for IVF-PQ search on gfx950, plus the exact
// nearest-centroid assignment the index builder uses.
//
// Reference behaviour (src/neighbors/indexes.cpp:597-606, src/prim/mixer.cpp:174-199,
// src/prim/cpu/cpu_prims.cpp:24-106): the coarse score of query q and centroid c is
// (|q|^2 + |c|^2) - 2*(q.c), each term a left-to-right fp32 sum, and the probe set is
// the first nprobe centroids under the total order (score, centroid index).
//
// Kernels:
//   k_row_norms      64 rows per workgroup staged through LDS, one lane per row,
//                    sequential sum.
//   k_coarse_scores  64x64 register-tiled VALU GEMM (4x4 outputs per lane, operands
//                    staged through LDS, 16-deep K slices), sequential per output so
//                    every score is bit-identical to the reference's.
//   k_select_topk    one workgroup per query row: 4-pass 8-bit radix select of the
//                    P-th smallest score key, ordered compaction of the winners,
//                    bitonic sort of (key, column) in LDS.
//   k_probe_fallback the exact route for the queries the matrix-core probe flags:
//                    one workgroup per 16 queries, each flagged one scored against
//                    every centroid and selected as in k_select_topk.
//   k_coarse_argmin  the GEMM tile loop over all centroids for 64 rows with a
//                    running (key, column) minimum: the k-means / extend assignment.
#include "device_common.hpp"
#include "kernels.hpp"

using namespace ovvs_dev;

namespace {

constexpr int kTile = 64;    // rows (queries) and columns (centroids) per workgroup
constexpr int kSlice = 16;   // K-depth staged per LDS round
constexpr int kPad = 4;      // LDS row padding (floats) for the transposed tiles

// Norms of 64 rows per workgroup: 64-column slices of the rows are staged in LDS by
// all 256 threads (coalesced), then thread r sums row r's squares left to right.
constexpr int kNormRows = 64;
__global__ __launch_bounds__(256) void k_row_norms(const float* __restrict__ x, int64_t n,
                                                   int dim, float* __restrict__ out) {
  __shared__ float tile[kNormRows][kNormRows + 1];
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kNormRows;
  const int t = static_cast<int>(threadIdx.x);
  float s = 0.f;
  for (int d0 = 0; d0 < dim; d0 += kNormRows) {
    const int dc = dim - d0 < kNormRows ? dim - d0 : kNormRows;
    __syncthreads();  // the previous slice has been summed
    for (int e = t; e < kNormRows * kNormRows; e += 256) {
      const int rr = e / kNormRows, c = e % kNormRows;
      const int64_t row = r0 + rr;
      tile[rr][c] = (row < n && c < dc) ? x[row * dim + d0 + c] : 0.f;
    }
    __syncthreads();
    if (t < kNormRows) {
      for (int c = 0; c < dc; ++c) s = s + tile[t][c] * tile[t][c];
    }
  }
  if (t < kNormRows && r0 + t < n) out[r0 + t] = s;
}

// Stages the [64 x kSlice] slices of Q (rows q0..) and C (rows c0..) for depth
// k0..k0+kt into LDS, transposed to [t][row], zero-filled out of range.
__device__ __forceinline__ void stage_slices(const float* __restrict__ Q, int64_t nq, int64_t q0,
                                             const float* __restrict__ C, int64_t nc, int64_t c0,
                                             int dim, int k0, int kt,
                                             float (*Qs)[kTile + kPad], float (*Cs)[kTile + kPad]) {
  for (int e = threadIdx.x; e < kTile * kSlice; e += 256) {
    const int r = e / kSlice, t = e % kSlice;
    const int64_t q = q0 + r;
    Qs[t][r] = (q < nq && t < kt) ? Q[q * dim + k0 + t] : 0.f;
    const int64_t c = c0 + r;
    Cs[t][r] = (c < nc && t < kt) ? C[c * dim + k0 + t] : 0.f;
  }
}

// acc[i][j] += Qs[t][ty*4+i] * Cs[t][tx*4+j] for t in [0, kt), one rounding each.
__device__ __forceinline__ void tile_fma_free(float (&acc)[4][4], const float (*Qs)[kTile + kPad],
                                              const float (*Cs)[kTile + kPad], int kt, int tx,
                                              int ty) {
  for (int t = 0; t < kt; ++t) {
    const float4 a = *reinterpret_cast<const float4*>(&Qs[t][ty * 4]);
    const float4 b = *reinterpret_cast<const float4*>(&Cs[t][tx * 4]);
    const float av[4] = {a.x, a.y, a.z, a.w};
    const float bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = acc[i][j] + av[i] * bv[j];
  }
}

__global__ __launch_bounds__(256) void k_coarse_scores(const float* __restrict__ Q,
                                                       const float* __restrict__ qn, int64_t nq,
                                                       const float* __restrict__ C,
                                                       const float* __restrict__ cn, int nlist,
                                                       int dim, float* __restrict__ S,
                                                       int64_t ldS) {
  __shared__ __attribute__((aligned(16))) float Qs[kSlice][kTile + kPad];
  __shared__ __attribute__((aligned(16))) float Cs[kSlice][kTile + kPad];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t q0 = static_cast<int64_t>(blockIdx.y) * kTile;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kTile;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
  for (int k0 = 0; k0 < dim; k0 += kSlice) {
    const int kt = min(kSlice, dim - k0);
    stage_slices(Q, nq, q0, C, nlist, c0, dim, k0, kt, Qs, Cs);
    __syncthreads();
    tile_fma_free(acc, Qs, Cs, kt, tx, ty);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t q = q0 + ty * 4 + i;
    if (q >= nq) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t c = c0 + tx * 4 + j;
      if (c < nlist) S[q * ldS + c] = (qn[q] + cn[c]) - 2.f * acc[i][j];
    }
  }
}

__global__ __launch_bounds__(256) void k_coarse_argmin(const float* __restrict__ Q,
                                                       const float* __restrict__ qn, int64_t nq,
                                                       const float* __restrict__ C,
                                                       const float* __restrict__ cn, int nlist,
                                                       int dim, int32_t* __restrict__ labels) {
  __shared__ __attribute__((aligned(16))) float Qs[kSlice][kTile + kPad];
  __shared__ __attribute__((aligned(16))) float Cs[kSlice][kTile + kPad];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t q0 = static_cast<int64_t>(blockIdx.x) * kTile;
  uint64_t best[4] = {kNoKey, kNoKey, kNoKey, kNoKey};
  for (int64_t c0 = 0; c0 < nlist; c0 += kTile) {
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
    for (int k0 = 0; k0 < dim; k0 += kSlice) {
      const int kt = min(kSlice, dim - k0);
      stage_slices(Q, nq, q0, C, nlist, c0, dim, k0, kt, Qs, Cs);
      __syncthreads();
      tile_fma_free(acc, Qs, Cs, kt, tx, ty);
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + ty * 4 + i;
      if (q >= nq) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t c = c0 + tx * 4 + j;
        if (c >= nlist) continue;
        const float s = (qn[q] + cn[c]) - 2.f * acc[i][j];
        const uint64_t key = make_key(s, static_cast<uint32_t>(c));
        best[i] = key < best[i] ? key : best[i];
      }
    }
  }
  // The 16 lanes sharing ty hold the same four rows: reduce across tx.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint64_t b = best[i];
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
      const uint64_t o = shfl_xor_u64(b, m);
      b = o < b ? o : b;
    }
    const int64_t q = q0 + ty * 4 + i;
    if (tx == 0 && q < nq) labels[q] = static_cast<int32_t>(b & 0xffffffffu);
  }
}

// ---- per-row top-P selection ----

__device__ __forceinline__ void block_bitonic_sort(uint64_t* s, int M) {
  for (int k = 2; k <= M; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < M; i += blockDim.x) {
        const int p = i ^ j;
        if (p > i) {
          const uint64_t a = s[i], b = s[p];
          const bool up = (i & k) == 0;
          if ((a > b) == up) {
            s[i] = b;
            s[p] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Exclusive block scan of one value per thread (256 threads). Returns the
// prefix; *total receives the sum.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* scratch,
                                                         uint32_t* total) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) scratch[wave] = x;
  __syncthreads();
  uint32_t base = 0, sum = 0;
  for (int w = 0; w < 4; ++w) {
    if (w < wave) base += scratch[w];
    sum += scratch[w];
  }
  __syncthreads();
  *total = sum;
  return base + x - v;
}

// LDS of one row selection.
struct SelectLds {
  uint64_t* sel;  // [M]
  uint32_t* hist;
  uint32_t* scan_scratch;
  uint32_t* digit_need;  // [2]
};

// The first P columns of row `row` of S under the total order, in rank order, into
// out[row * P ...]. Called by the whole workgroup.
__device__ __forceinline__ void select_row(const float* __restrict__ S, int64_t ldS, int N, int P,
                                           int M, int64_t row, int32_t* __restrict__ out,
                                           const SelectLds& L) {
  uint64_t* sel = L.sel;
  uint32_t* hist = L.hist;
  uint32_t* scan_scratch = L.scan_scratch;
  uint32_t& s_digit = L.digit_need[0];
  uint32_t& s_need = L.digit_need[1];
  const float* r = S + row * ldS;

  // 1. Radix select of the P-th smallest 32-bit score key.
  uint32_t prefix = 0, mask = 0, need = static_cast<uint32_t>(P);
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    hist[threadIdx.x] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < N; i += 256) {
      const uint32_t key = score_key(r[i]);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t cum = 0;
      for (int d = 0; d < 256; ++d) {
        if (cum + hist[d] >= need) {
          s_digit = static_cast<uint32_t>(d);
          s_need = need - cum;
          break;
        }
        cum += hist[d];
      }
    }
    __syncthreads();
    prefix |= s_digit << shift;
    mask |= 255u << shift;
    need = s_need;
    __syncthreads();
  }
  const uint32_t thr = prefix;  // key of the P-th element; take `need` of the equal ones

  // 2. Ordered compaction: keys < thr anywhere, then the first `need` keys == thr
  //    in column order. Each thread owns one contiguous segment of columns.
  const int seg = (N + 255) / 256;
  const int b = threadIdx.x * seg, e = min(N, b + seg);
  uint32_t n_lt = 0, n_eq = 0;
  for (int i = b; i < e; ++i) {
    const uint32_t key = score_key(r[i]);
    n_lt += key < thr;
    n_eq += key == thr;
  }
  uint32_t tot_lt = 0, tot_eq = 0;
  const uint32_t off_lt = block_exclusive_scan(n_lt, scan_scratch, &tot_lt);
  uint32_t off_eq = block_exclusive_scan(n_eq, scan_scratch, &tot_eq);
  uint32_t w_lt = off_lt;
  for (int i = b; i < e; ++i) {
    const uint32_t key = score_key(r[i]);
    const uint64_t packed = (static_cast<uint64_t>(key) << 32) | static_cast<uint32_t>(i);
    if (key < thr) {
      sel[w_lt++] = packed;
    } else if (key == thr) {
      if (off_eq < need) sel[tot_lt + off_eq] = packed;
      ++off_eq;
    }
  }
  for (int i = P + threadIdx.x; i < M; i += 256) sel[i] = kNoKey;
  __syncthreads();

  // 3. Sort the P winners by (key, column) and emit them in rank order.
  block_bitonic_sort(sel, M);
  for (int i = threadIdx.x; i < P; i += 256) {
    out[row * P + i] = static_cast<int32_t>(sel[i] & 0xffffffffu);
  }
}

// Rows that flags marks (flags[row] != 0) among the workgroup's 256 rows
// [kFallbackRows * blockIdx.x, +kFallbackRows), compacted into rows[0, *count). Called
// by the whole workgroup; a workgroup without flagged rows returns count 0 after one
// load.
constexpr int kFallbackRows = 16;
__device__ __forceinline__ int flagged_rows(const int32_t* __restrict__ flags, int64_t nrows,
                                            int32_t* rows, int32_t* count) {
  if (threadIdx.x == 0) *count = 0;
  __syncthreads();
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kFallbackRows + threadIdx.x;
  if (threadIdx.x < kFallbackRows && row < nrows && flags[row] != 0)
    rows[atomicAdd(count, 1)] = static_cast<int32_t>(row);
  __syncthreads();
  return *count;
}

// One workgroup per row.
__global__ __launch_bounds__(256) void k_select_topk(const float* __restrict__ S, int64_t ldS,
                                                     int N, int P, int M,
                                                     int32_t* __restrict__ out) {
  extern __shared__ uint64_t sel[];  // [M]
  __shared__ uint32_t hist[256];
  __shared__ uint32_t scan_scratch[4];
  __shared__ uint32_t digit_need[2];
  select_row(S, ldS, N, P, M, blockIdx.x, out, SelectLds{sel, hist, scan_scratch, digit_need});
}

// The exact route for the queries the matrix-core probe flagged (usually none):
// one workgroup per kFallbackRows queries; for each flagged one, the exact score of
// every centroid into its row of S, then the row selection.
__global__ __launch_bounds__(256) void k_probe_fallback(
    const float* __restrict__ Q, const float* __restrict__ qn, int64_t nq,
    const float* __restrict__ C, const float* __restrict__ cn, int nlist, int dim,
    const int32_t* __restrict__ flags, float* __restrict__ S, int P, int M,
    int32_t* __restrict__ out, unsigned long long* stamp) {
  if (stamp && blockIdx.x == 0 && threadIdx.x == 0) *stamp = wall_clock64();
  extern __shared__ uint64_t sel[];  // [M]
  __shared__ uint32_t hist[256];
  __shared__ uint32_t scan_scratch[4];
  __shared__ uint32_t digit_need[2];
  __shared__ int32_t rows[kFallbackRows];
  __shared__ int32_t count;
  const SelectLds L{sel, hist, scan_scratch, digit_need};
  const int n = flagged_rows(flags, nq, rows, &count);
  for (int i = 0; i < n; ++i) {
    const int64_t q = rows[i];
    const float* qv = Q + q * dim;
    const float qnq = qn[q];
    for (int c = static_cast<int>(threadIdx.x); c < nlist; c += 256) {
      S[q * nlist + c] = (qnq + cn[c]) - 2.f * seq_dot(qv, C + static_cast<int64_t>(c) * dim, dim);
    }
    __syncthreads();  // the row of S is complete (workgroup-scope release/acquire)
    select_row(S, nlist, nlist, P, M, q, out, L);
    __syncthreads();  // sel is reused by the next row
  }
}

}  // namespace

extern "C" hipError_t ovvs_hip_row_norms(const float* x, int64_t n, int32_t dim, float* out,
                                         hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (!x || !out || dim <= 0) return hipErrorInvalidValue;
  const int64_t blocks = (n + kNormRows - 1) / kNormRows;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_row_norms, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream, x, n,
                     dim, out);
  return hipGetLastError();
}

extern "C" hipError_t ovvs_hip_coarse_scores(const float* Q, const float* qn, int64_t nq,
                                             const float* C, const float* cn, int32_t nlist,
                                             int32_t dim, float* S, int64_t ldS,
                                             hipStream_t stream) {
  if (nq <= 0) return hipSuccess;
  if (!Q || !qn || !C || !cn || !S || nlist <= 0 || dim <= 0 || ldS < nlist)
    return hipErrorInvalidValue;
  const int64_t gy = (nq + kTile - 1) / kTile, gx = (nlist + kTile - 1) / kTile;
  if (gy > 65535 || gx > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_coarse_scores, dim3(static_cast<uint32_t>(gx), static_cast<uint32_t>(gy)),
                     dim3(256), 0, stream, Q, qn, nq, C, cn, nlist, dim, S, ldS);
  return hipGetLastError();
}

extern "C" hipError_t ovvs_hip_coarse_argmin(const float* Q, const float* qn, int64_t nq,
                                             const float* C, const float* cn, int32_t nlist,
                                             int32_t dim, int32_t* labels, hipStream_t stream) {
  if (nq <= 0) return hipSuccess;
  if (!Q || !qn || !C || !cn || !labels || nlist <= 0 || dim <= 0) return hipErrorInvalidValue;
  const int64_t g = (nq + kTile - 1) / kTile;
  if (g > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_coarse_argmin, dim3(static_cast<uint32_t>(g)), dim3(256), 0, stream, Q, qn,
                     nq, C, cn, nlist, dim, labels);
  return hipGetLastError();
}

extern "C" hipError_t ovvs_hip_select_topk(const float* S, int64_t ldS, int64_t nrows, int32_t N,
                                           int32_t P, int32_t* out, hipStream_t stream) {
  if (nrows <= 0) return hipSuccess;
  if (!S || !out || N <= 0 || P <= 0 || P > N || P > OVVS_HIP_MAX_PROBES || ldS < N ||
      nrows > 0x7fffffff)
    return hipErrorInvalidValue;
  int M = 1;
  while (M < P) M <<= 1;
  hipLaunchKernelGGL(k_select_topk, dim3(static_cast<uint32_t>(nrows)), dim3(256),
                     static_cast<size_t>(M) * sizeof(uint64_t), stream, S, ldS, N, P, M, out);
  return hipGetLastError();
}

extern "C" hipError_t ovvs_hip_probe_fallback(const float* Q, const float* qn, int64_t nq,
                                              const float* C, const float* cn, int32_t nlist,
                                              int32_t dim, const int32_t* flags, float* S,
                                              int32_t P, int32_t* out, unsigned long long* stamp,
                                              hipStream_t stream) {
  if (nq <= 0) return hipSuccess;
  if (!Q || !qn || !C || !cn || !flags || !S || !out || nlist <= 0 || dim <= 0 || P <= 0 ||
      P > nlist || P > OVVS_HIP_MAX_PROBES || nq > 0x7fffffff)
    return hipErrorInvalidValue;
  int M = 1;
  while (M < P) M <<= 1;
  hipLaunchKernelGGL(k_probe_fallback, dim3(static_cast<uint32_t>((nq + kFallbackRows - 1) / kFallbackRows)), dim3(256),
                     static_cast<size_t>(M) * sizeof(uint64_t), stream, Q, qn, nq, C, cn, nlist,
                     dim, flags, S, P, M, out, stamp);
  return hipGetLastError();
}
