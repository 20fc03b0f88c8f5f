// scan.hip — fused code scan + shortlist select for IVF-PQ search on gfx950.
//
// Reference behaviour: for every probed list l of query q (in probe-rank order)
// the residual r = q - c_l gives the table T[m][j] = sum_u (r[m*dsub+u] -
// B[m][j][u])^2 (src/neighbors/indexes.cpp:764-785, always L2); each row's ADC
// score is sum_m T[m][code_m], left to right from +0 (src/prim/mixer.cpp:378-390);
// the shortlist is the first krefine rows under the total order on (score,
// dense ordinal) where the ordinal runs over the query's accepted rows in probe
// order (indexes.cpp:683-712,1019-1066; the reference's own GPU design for this
// step is src/prim/gpu/backend_gpu.cpp:791-1010).
//
// Design (one 256-lane workgroup per query; its four wave64s work independently,
// wave w on the probed lists of rank w, w+4, ..., and share only the K-th best
// keys they publish in LDS):
//   * The device mirror stores each list as segments of up to 128 rows with
//     nearby PQ reconstructions, each with the per-dimension range (box) of its
//     rows' reconstructions. For the residual r, the entry of subspace m of any
//     row of the segment is at least the sum over m's dimensions of the squared
//     distance from r to the box, so the box bounds every row's score from below
//     (and the part after block 0). fp32 rounding is monotone, so the bounds hold
//     for the rounded scores up to a small relative allowance.
//   * A segment whose bound exceeds the K-th best score found so far cannot
//     contribute: it is skipped without reading its codes. Consecutive segments
//     (subtrees of the segmentation, at most four segments) form groups with the
//     union of their boxes, and so does each list: a list or group whose bound
//     exceeds the K-th best is skipped whole. Group and segment bounds are
//     evaluated 4-64 lanes per box, up to 16 boxes per pass.
//   * Rows of the other segments are read in 64-row code tiles (one coalesced
//     512-byte access per wave and block) and scored through block 0 (the first 8
//     subspaces). A row whose partial sum plus the segment's tail bound still
//     exceeds the K-th best is dropped; the rest are queued and, 64 at a time,
//     completed block by block. Table entries are computed where they are used,
//     from the codebook, with the reference's operation order: with the bounds in
//     place a query scores a few hundred rows, so building whole tables would cost
//     more than the entries it reads. Every row that can enter the shortlist is
//     scored completely, so the shortlist is exactly the reference's.
//   * Each wave keeps its own running top-K as a sorted register list (64 keys
//     per register row, KPL rows), a 128-slot LDS candidate buffer and a
//     threshold it publishes in LDS: rows are appended with ballot/popcount (no
//     atomics), buffers are merged by a cross-lane bitonic sort plus a bitonic
//     merge, and at the end the four lists are merged once.
//   * Data without cluster structure defeats the bounds: a query whose rows scored
//     after the first phase exceed a budget stops and is handed off to a full
//     scan (k_scan_wave: the codebook in LDS, one query per wave; k_scan_table:
//     each list's whole table in LDS), which rewrites all of its outputs.
// Keys are (order-preserving score bits << 32 | raw ordinal); a row's raw ordinal
// is the number of rows of earlier probed lists plus its index within its list,
// which orders accepted rows exactly as the dense ordinal does, whatever order the
// scan visits them in.
#include <hip/hip_fp16.h>

#include "device_common.hpp"
#include "kernels.hpp"

using namespace ovvs_dev;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kBufCap = 128;
constexpr int kBlock = OVVS_CODE_BLOCK;      // subspaces per block (8)
constexpr int kTile = OVVS_CODE_TILE_ROWS;   // rows per code tile (64)

__host__ __device__ constexpr size_t round16(size_t b) { return (b + 15) & ~static_cast<size_t>(15); }

template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, 0xf, 0xf, false));
}

// v of lane (this lane ^ s), all in VALU: within 16-lane rows by DPP (quad_perm for
// s = 1, 2; row rotations, where lane i reads lane i - n, for s = 4, 8), across rows
// by the gfx950 row swaps (v_permlane16_swap / v_permlane32_swap with both operands
// v: the first result holds the even rows (lower half) twice, the second the odd rows
// (upper half)). s is a constant after unrolling; all lanes active.
__device__ __forceinline__ uint32_t xor_lane(uint32_t v, int s) {
  switch (s) {
    case 1: return dpp_u<0xB1>(v);
    case 2: return dpp_u<0x4E>(v);
    case 4: {
      // Both rotations run on all lanes and are blended by a lane mask (a select the
      // compiler may turn into a branch would run each rotation with its source
      // lanes off).
      const uint32_t down = dpp_u<0x124>(v), up = dpp_u<0x12C>(v);
      const uint32_t m = 0u - ((static_cast<uint32_t>(lane_id()) >> 2) & 1u);
      return (down & m) | (up & ~m);
    }
    case 8: return dpp_u<0x128>(v);
    case 16: {
      const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
      return (lane_id() & 16) ? r[0] : r[1];
    }
    case 32: {
      const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
      return (lane_id() & 32) ? r[0] : r[1];
    }
    default: return static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), s, 64));
  }
}

// v of the previous lane (lane 0: lane 63's), DPP wave_ror:1. All lanes active.
__device__ __forceinline__ uint32_t wave_ror1(uint32_t v) { return dpp_u<0x13C>(v); }

// v of lane 63 - this lane (row_mirror reverses each 16-lane row, then the rows swap).
__device__ __forceinline__ uint32_t rev_lane(uint32_t v) {
  return xor_lane(xor_lane(dpp_u<0x140>(v), 16), 32);
}

// Compare-exchange of (k, p) with the lane `s` away; this lane keeps the
// smaller key when keep_min.
__device__ __forceinline__ void cx_lane(uint64_t& k, int32_t& p, int s, bool keep_min) {
  const uint64_t ok = (static_cast<uint64_t>(xor_lane(static_cast<uint32_t>(k >> 32), s)) << 32) |
                      xor_lane(static_cast<uint32_t>(k), s);
  const int32_t op = static_cast<int32_t>(xor_lane(static_cast<uint32_t>(p), s));
  const bool take = keep_min ? (ok < k) : (ok > k);
  if (take) {
    k = ok;
    p = op;
  }
}

// Sorts one key per lane ascending across the wave.
__device__ __forceinline__ void sort64(uint64_t& k, int32_t& p) {
  const int lane = lane_id();
#pragma unroll
  for (int sz = 2; sz <= 64; sz <<= 1) {
#pragma unroll
    for (int s = sz >> 1; s > 0; s >>= 1) {
      const bool asc = (lane & sz) == 0;
      const bool lower = (lane & s) == 0;
      cx_lane(k, p, s, lower == asc);
    }
  }
}

// Sorts a bitonic sequence of 64*KPL elements (element e = j*64 + lane)
// ascending.
template <int KPL>
__device__ __forceinline__ void bitonic_merge_asc(uint64_t (&lk)[KPL], int32_t (&lp)[KPL]) {
  const int lane = lane_id();
#pragma unroll
  for (int s = KPL / 2; s >= 1; s >>= 1) {
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      if ((j & s) == 0) {
        const int o = j | s;
        if (lk[o] < lk[j]) {
          const uint64_t tk = lk[j];
          lk[j] = lk[o];
          lk[o] = tk;
          const int32_t tp = lp[j];
          lp[j] = lp[o];
          lp[o] = tp;
        }
      }
    }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
#pragma unroll
    for (int j = 0; j < KPL; ++j) cx_lane(lk[j], lp[j], s, (lane & s) == 0);
  }
}

// Merges 64 keys (one per lane, sorted ascending) into the sorted list, keeping
// the 64*KPL smallest.
template <int KPL>
__device__ __forceinline__ void merge64(uint64_t (&lk)[KPL], int32_t (&lp)[KPL], uint64_t bk,
                                        int32_t bp) {
  const uint64_t rk = (static_cast<uint64_t>(rev_lane(static_cast<uint32_t>(bk >> 32))) << 32) |
                      rev_lane(static_cast<uint32_t>(bk));
  const int32_t rp = static_cast<int32_t>(rev_lane(static_cast<uint32_t>(bp)));
  if (rk < lk[KPL - 1]) {
    lk[KPL - 1] = rk;
    lp[KPL - 1] = rp;
  }
  bitonic_merge_asc<KPL>(lk, lp);
}

// Key at element e = K-1 of the sorted list (wave-uniform result).
template <int KPL>
__device__ __forceinline__ uint64_t kth_key(const uint64_t (&lk)[KPL], int K) {
  const int j = (K - 1) >> 6;
  uint64_t v = lk[0];
#pragma unroll
  for (int r = 1; r < KPL; ++r) v = (r == j) ? lk[r] : v;
  const int l = __builtin_amdgcn_readfirstlane((K - 1) & 63);
  return (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), l))) << 32) |
         static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), l));
}

// Inserts one key (wave-uniform) into the sorted list, dropping the largest.
template <int KPL>
__device__ __forceinline__ void insert_one(uint64_t (&lk)[KPL], int32_t (&lp)[KPL], uint64_t key,
                                           int32_t pos) {
  const int lane = lane_id();
  int at = 0;  // number of list elements smaller than key
#pragma unroll
  for (int j = 0; j < KPL; ++j) at += __popcll(__ballot(lk[j] < key));
  uint64_t prev_tail = 0;
  int32_t prev_tail_p = 0;
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    // Element e = j*64 + lane takes element e-1 when e > at: the previous lane's
    // element by a wave rotation (DPP wave_ror:1), lane 63's by readlane.
    uint64_t up = (static_cast<uint64_t>(wave_ror1(static_cast<uint32_t>(lk[j] >> 32))) << 32) |
                  wave_ror1(static_cast<uint32_t>(lk[j]));
    int32_t upp = static_cast<int32_t>(wave_ror1(static_cast<uint32_t>(lp[j])));
    const uint64_t tail =
        (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lk[j] >> 32), 63))) << 32) |
        static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lk[j]), 63));
    const int32_t tailp = __builtin_amdgcn_readlane(lp[j], 63);
    if (lane == 0) {
      up = prev_tail;
      upp = prev_tail_p;
    }
    const int e = j * 64 + lane;
    if (e == at) {
      lk[j] = key;
      lp[j] = pos;
    } else if (e > at) {
      lk[j] = up;
      lp[j] = upp;
    }
    prev_tail = tail;
    prev_tail_p = tailp;
  }
}

// Score whose keys are above `key`'s score word: the float the order-preserving
// transform maps to key >> 32 (+inf for an empty slot, NaN stays NaN).
__device__ __forceinline__ float key_score(uint64_t key) {
  const uint32_t k = static_cast<uint32_t>(key >> 32);
  if (k == 0xffffffffu) return __builtin_inff();
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// The DSUB floats of one codebook entry, loaded in one piece (entries are
// DSUB * 4-byte aligned).
template <int DSUB>
struct Codeword {
  float v[DSUB];
  __device__ __forceinline__ void load(const float* __restrict__ p) {
    if constexpr (DSUB == 1) {
      v[0] = p[0];
    } else if constexpr (DSUB == 2) {
      const float2 x = *reinterpret_cast<const float2*>(p);
      v[0] = x.x;
      v[1] = x.y;
    } else {
#pragma unroll
      for (int h = 0; h < DSUB / 4; ++h) {
        const float4 x = reinterpret_cast<const float4*>(p)[h];
        v[4 * h + 0] = x.x;
        v[4 * h + 1] = x.y;
        v[4 * h + 2] = x.z;
        v[4 * h + 3] = x.w;
      }
    }
  }
};

// Table slice builders for the first phase (whole lists, all four waves): entry
// (m - m0) * ks + j of the slice is sum_u (r[m*dsub+u] - B[m][j][u])^2, left to
// right from +0. For ks = 256 thread j computes
// entry j of every subspace of the slice, its codebook loads (coalesced across
// threads) issued a group of subspaces ahead of the arithmetic.
template <int DSUB>
__device__ __forceinline__ void build_slice_256(const float* resid,
                                                const float* __restrict__ codebooks, int m0,
                                                float* lut32) {
  constexpr int kGroup = DSUB <= 2 ? kBlock : 16 / DSUB;
  const int j = static_cast<int>(threadIdx.x);
  const float* __restrict__ cb = codebooks + (static_cast<int64_t>(m0) * 256 + j) * DSUB;
#pragma unroll
  for (int g0 = 0; g0 < kBlock; g0 += kGroup) {
    Codeword<DSUB> cw[kGroup];
#pragma unroll
    for (int i = 0; i < kGroup; ++i) cw[i].load(cb + (g0 + i) * 256 * DSUB);
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      const float* r = resid + (m0 + g0 + i) * DSUB;
      float acc = 0.f;
#pragma unroll
      for (int u = 0; u < DSUB; ++u) {
        const float t = r[u] - cw[i].v[u];
        acc = acc + t * t;
      }
      lut32[(g0 + i) * 256 + j] = acc;
    }
  }
}

// Any shape: mb subspaces of ks entries, dsub dimensions each.
__device__ __forceinline__ void build_slice_any(const float* resid, const float* __restrict__ codebooks,
                                                int m0, int mb, int ks, int ks_log2, int dsub,
                                                float* lut32) {
  const int slice = mb << ks_log2;
  for (int e = static_cast<int>(threadIdx.x); e < slice; e += kThreads) {
    const int m = m0 + (e >> ks_log2);
    const float* r = resid + m * dsub;
    const float* __restrict__ cw = codebooks + (static_cast<int64_t>(m) * ks + (e & (ks - 1))) * dsub;
    float acc = 0.f;
    for (int u = 0; u < dsub; ++u) {
      const float t = r[u] - cw[u];
      acc = acc + t * t;
    }
    lut32[e] = acc;
  }
}

// One table entry computed directly from the codebook, with the operation order
// of the reference's table build: sum_u (r[m*dsub+u] - B[m][code][u])^2 left to
// right from +0.
template <int FD>
__device__ __forceinline__ float direct_entry(const float* resid, const float* __restrict__ codebooks,
                                              int m, int code, int ks, int dsub) {
  const int d = FD > 0 ? FD : dsub;
  const float* __restrict__ cw = codebooks + (static_cast<int64_t>(m) * ks + code) * d;
  const float* r = resid + m * d;
  float acc = 0.f;
  if constexpr (FD > 0) {
    Codeword<FD> c;
    c.load(cw);
#pragma unroll
    for (int u = 0; u < FD; ++u) {
      const float t = r[u] - c.v[u];
      acc = acc + t * t;
    }
  } else {
    for (int u = 0; u < d; ++u) {
      const float t = r[u] - cw[u];
      acc = acc + t * t;
    }
  }
  return acc;
}

// Squared distance from r to the range [lo, hi] packed as binary16 lo | hi << 16
// (the nearest point of the range is med3(r, lo, hi); both halves widen exactly).
__device__ __forceinline__ float box_e2(float r, uint32_t b) {
  const float lo = __half2float(__ushort_as_half(static_cast<uint16_t>(b & 0xffffu)));
  const float hi = __half2float(__ushort_as_half(static_cast<uint16_t>(b >> 16)));
  const float e = r - __builtin_amdgcn_fmed3f(r, lo, hi);
  return e * e;
}

// acc + d^2 for the distance d from r to the range packed in b (one rounding).
__device__ __forceinline__ float box_acc(float r, uint32_t b, float acc) {
  const float lo = __half2float(__ushort_as_half(static_cast<uint16_t>(b & 0xffffu)));
  const float hi = __half2float(__ushort_as_half(static_cast<uint16_t>(b >> 16)));
  const float e = r - __builtin_amdgcn_fmed3f(r, lo, hi);
  return __builtin_fmaf(e, e, acc);
}

// v from another lane of the same row, by a DPP control (quad_perm, row mirrors).
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}

// Inclusive prefix sum across the 64 lanes (row shifts within 16 lanes, then row
// broadcasts; all lanes active). Lanes a shift moves past a row's edge add 0.
__device__ __forceinline__ int32_t wave_incl_scan(int32_t v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31 into rows 2, 3
  return v;
}

// Sum over aligned groups of 2^gl lanes; every lane of a group gets the same value
// (each step adds two equal partial sums in either order). All lanes active.
__device__ __forceinline__ float group_sum(float e, int gl) {
  if (gl >= 1) e = e + dpp_f<0xB1>(e);   // quad_perm(1, 0, 3, 2): lane ^ 1
  if (gl >= 2) e = e + dpp_f<0x4E>(e);   // quad_perm(2, 3, 0, 1): lane ^ 2
  if (gl >= 3) e = e + dpp_f<0x141>(e);  // row_half_mirror: the other quad of 8 lanes
  if (gl >= 4) e = e + dpp_f<0x140>(e);  // row_mirror: the other half of 16 lanes
  if (gl >= 5) e = e + __uint_as_float(xor_lane(__float_as_uint(e), 16));
  if (gl >= 6) e = e + __uint_as_float(xor_lane(__float_as_uint(e), 32));
  return e;
}

// Boxes are stored in absolute coordinates (the list centroid added), so the
// distance is measured from q rather than from the residual fl(q - c) the table
// entries use. Rounding moves each residual coordinate by at most s (2^-21 times
// max|q| + max|c|), so over D dimensions the squared residual distance is at
// least e - 2 s sqrt(D e) (Cauchy-Schwarz); the 2^-20 and the 2.02 also cover the
// rounding of e itself. Returns that lower bound (NaN, which prunes nothing, when
// e or s is not finite).
__device__ __forceinline__ float box_bound(float e, float s, float D) {
  return e * (1.f - 0x1p-20f) - 2.02f * s * __builtin_sqrtf(D * e);
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Position in the query order of workgroup b of n. Workgroups go to the eight XCDs in
// turn (b to XCD b % 8). The order is cut into 8 * kXcdParts parts of B = n / (8 *
// kXcdParts) queries; XCD x takes parts x, x + 8, x + 16, ... one after another, so the
// queries resident on an XCD at a time lie in one region of the order (its L2 serves
// lists near each other) while every XCD gets kXcdParts regions. With one part per XCD
// the XCDs holding slow regions finished last (C5's scan 3.16 ms against 2.73 ms with
// four); with no parts (the order taken in turn) C4's scan took 1.40 ms against 1.33.
// Positions from 8 * kXcdParts * B on are taken in turn.
constexpr int64_t kXcdParts = 4;
__device__ __forceinline__ int64_t xcd_slot(int64_t b, int64_t n) {
  const int64_t B = n / (8 * kXcdParts);
  if (b >= 8 * kXcdParts * B) return b;
  const int64_t x = b & 7, k = b >> 3;
  return ((k / B) * 8 + x) * B + k % B;
}

constexpr int kQueueCap = 128;
// At most this many segments share one bound pass (at least 4 lanes each).
constexpr int kSegPerPass = 16;
// Segment slots of one group pass (every group holds at most OVVS_GROUP_SEGMENTS).
constexpr int kSegSlots = OVVS_GROUP_SEGMENTS * kSegPerPass;
// Groups the independent phase holds in LDS at a time.
constexpr int kItemCap = 256;
// Phase 0: candidate groups per rank (of the first kWaves ranks) and rounds.
constexpr int kP0Cand = 64;
// Shortlists of more than 64 keys (K up to 128) take up to kP0RoundsLong rounds: the
// union's K-th key needs more rows (C3, k 100: scan 1.25 -> 0.95 ms with 8 rounds instead
// of 4, while C2 and C4 measured 3% slower with 8).
constexpr int kP0Rounds = 4;
constexpr int kP0RoundsLong = 8;
// misc words after the phase-0 groups misc[4, 4 + kP0RoundsLong): tiles scored after
// phase 0, rows of the lists whose bound passed.
constexpr int kMiscTiles = 4 + kP0RoundsLong;
constexpr int kMiscRows = 5 + kP0RoundsLong;
static_assert(kMiscRows < 16, "the misc words hold 16 int32");
// Tiles a query may score after phase 0 before it is handed off to the full-table scan
// (at least; more when its live lists are large).
constexpr int kPuntTiles = 32;
static_assert(kWaves * kP0Cand * 8 <= kWaves * 2 * kSegSlots * 4, "phase-0 candidates must fit the slot area");
// Rounding allowances of the lower bounds (valid for up to OVVS_MAX_BOX_DIMS box
// dimensions and as many subspaces): a threshold raised by 2^-10 relative and a
// tail bound lowered by 2^-10 relative cover every rounding of the bound sums and
// of the scores they bound.
constexpr float kBoundUp = 1.0f + 0x1p-10f;
constexpr float kBoundDown = 1.0f - 0x1p-10f;

struct ScanLayout {
  size_t bufk_off;   // per wave: candidate keys [kBufCap]
  size_t bufp_off;   //           candidate positions [kBufCap]
  size_t qpos_off;   //           survivor queue positions [kQueueCap]
  size_t qsc_off;    //           survivor queue partial scores [kQueueCap]
  size_t work_bytes; // the above, or the final cross-wave merge (aliased)
  size_t query_off;  // the query row [dim_pad]
  size_t resid_off;  // per wave: residual of its current list [dim_pad]
  size_t thr_off;    // [kWaves + 1] published K-th keys (the last: the union's, after phase 0)
  size_t misc_off;   // [16] int32: end of phase 0, bad probe flag, rows, lists, groups
                     //      scored in phase 0 (up to kP0RoundsLong), tiles scored after phase 0,
                     //      rows of the lists whose bound passed after phase 0
  size_t slot_off;   // per wave: [2][kSegSlots] int32, the segments of a bound pass and
                     //           their list ranks; before: phase 0's candidate groups
                     //           [kWaves * kP0Cand] u64
  size_t item_off;   // [kItemCap] int32 group ids, then [kItemCap] int16 list ranks
  size_t table_off;  // [8][P] per probe rank: list, rows, ordinal base, first group,
                     //        groups, list bound, items (groups of the list if its bound
                     //        passed), first item within its 64-rank chunk; then one
                     //        unused word and the first item of every chunk
  size_t total;
};

__host__ __device__ inline ScanLayout scan_layout(int dim, int kpl, int P) {
  ScanLayout L;
  const size_t dim_pad = static_cast<size_t>((dim + 3) & ~3);
  L.bufk_off = 0;
  L.bufp_off = L.bufk_off + static_cast<size_t>(kWaves) * kBufCap * 8;
  L.qpos_off = L.bufp_off + static_cast<size_t>(kWaves) * kBufCap * 4;
  L.qsc_off = L.qpos_off + static_cast<size_t>(kWaves) * kQueueCap * 4;
  const size_t cand = L.qsc_off + static_cast<size_t>(kWaves) * kQueueCap * 4;
  const size_t merge = static_cast<size_t>(kWaves) * 64 * kpl * (8 + 4);
  L.work_bytes = round16(cand > merge ? cand : merge);
  L.query_off = L.work_bytes;
  L.resid_off = L.query_off + dim_pad * 4;
  L.thr_off = L.resid_off + static_cast<size_t>(kWaves) * dim_pad * 4;
  L.misc_off = L.thr_off + (kWaves + 1) * 8;
  L.slot_off = L.misc_off + 64;
  L.item_off = L.slot_off + static_cast<size_t>(kWaves) * 2 * kSegSlots * 4;
  L.table_off = L.item_off + static_cast<size_t>(kItemCap) * 6;
  L.total = L.table_off + (8 * static_cast<size_t>(P) + 1 + (P + 63) / 64) * 4;
  return L;
}

// FD > 0: the shape-specialised body for ks = 256, pq_m % 8 == 0 and dsub = FD;
// FD = 0: any shape.
template <int KPL, int FD>
__device__ __forceinline__ void scan_query(const OvvsScanArgs& a, unsigned char* smem) {
  const ScanLayout L = scan_layout(a.dim, KPL, a.P);
  const int dim_pad = (a.dim + 3) & ~3;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = lane_id();
  float* qs = reinterpret_cast<float*>(smem + L.query_off);
  float* resid = reinterpret_cast<float*>(smem + L.resid_off) + wave * dim_pad;
  uint64_t* wave_thr = reinterpret_cast<uint64_t*>(smem + L.thr_off);
  uint64_t* bufk = reinterpret_cast<uint64_t*>(smem + L.bufk_off) + wave * kBufCap;
  int32_t* bufp = reinterpret_cast<int32_t*>(smem + L.bufp_off) + wave * kBufCap;
  int32_t* qpos = reinterpret_cast<int32_t*>(smem + L.qpos_off) + wave * kQueueCap;
  float* qsc = reinterpret_cast<float*>(smem + L.qsc_off) + wave * kQueueCap;

  const int64_t q = a.order ? a.order[xcd_slot(blockIdx.x, a.nq)] : static_cast<int64_t>(blockIdx.x);
  const int ks = a.ks;
  const int K = a.K;
  const int pq_m = a.pq_m;
  const int dsub = FD > 0 ? FD : a.dsub;
  const int nblocks = (pq_m + kBlock - 1) / kBlock;
  const int mb0 = pq_m < kBlock ? pq_m : kBlock;
  const int box_dims = pq_m * dsub;
  const uint32_t* __restrict__ boxes = a.seg_box;
  const uint32_t* __restrict__ lboxes = a.list_box;
  int32_t* misc = reinterpret_cast<int32_t*>(smem + L.misc_off);
  int32_t* t_list = reinterpret_cast<int32_t*>(smem + L.table_off);
  int32_t* t_rows = t_list + a.P;
  uint32_t* t_ord = reinterpret_cast<uint32_t*>(t_rows + a.P);
  int32_t* t_g0 = reinterpret_cast<int32_t*>(t_ord + a.P);
  int32_t* t_ngrp = t_g0 + a.P;
  float* t_lbound = reinterpret_cast<float*>(t_ngrp + a.P);
  int32_t* t_icnt = reinterpret_cast<int32_t*>(t_lbound + a.P);
  int32_t* t_item = t_icnt + a.P;
  // Bytes of one 64-row code tile.
  const uint32_t tile_bytes = static_cast<uint32_t>(nblocks) * kTile * kBlock;

  for (int t = static_cast<int>(threadIdx.x); t < a.dim; t += kThreads) qs[t] = a.queries[q * a.dim + t];
  if (lane == 0) wave_thr[wave] = kNoKey;
  if (threadIdx.x == 0) wave_thr[kWaves] = kNoKey;
  // Probe table: list, rows and group range per rank (an
  // invalid probe id is marked -1 with no rows: the search then fails).
  for (int t = static_cast<int>(threadIdx.x); t < a.P; t += kThreads) {
    const int l = a.probes[q * a.P + t];
    const bool ok = static_cast<uint32_t>(l) < static_cast<uint32_t>(a.nlist);
    const int lv = ok ? l : 0;
    t_list[t] = ok ? l : -1;
    t_rows[t] = ok ? static_cast<int32_t>(a.list_offsets[lv + 1] - a.list_offsets[lv]) : 0;
    const int32_t g0 = a.list_grp[lv];
    t_g0[t] = g0;
    t_ngrp[t] = ok ? a.list_grp[lv + 1] - g0 : 0;
  }
  __syncthreads();
  // Largest query coordinate magnitude, for the residual rounding allowance.
  float qmax = 0.f;
  for (int t = lane; t < a.dim; t += 64) {
    const float v = __builtin_fabsf(qs[t]);
    qmax = (v <= qmax) ? qmax : v;  // NaN propagates
  }
  // Lane exchanges as DPP and row swaps (no lane-address registers to keep live).
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float v = __uint_as_float(xor_lane(__float_as_uint(qmax), o));
    qmax = (v <= qmax) ? qmax : v;
  }
  const float slack = 0x1p-21f * (qmax + a.box_cmax);
  const float dims_all = static_cast<float>(box_dims);
  const float dims_tail = static_cast<float>(box_dims - mb0 * dsub);
  // Squared distance from the query to each of n <= 16 boxes (box ids[j] of base,
  // or box id0 + j when ids is null; a negative id reads box 0), before
  // box_bound's allowance. S boxes share the pass (n rounded up to a power of
  // two), G = 64 / S = 2^gl lanes each; every lane of a box returns its sum.
  auto box_total = [&](const uint32_t* __restrict__ base, const int32_t* ids, int id0, int n, int& gl,
                       bool& valid, int& id) -> float {
    gl = 2;
    while (gl < 6 && (32 >> gl) >= n) ++gl;
    const int G = 1 << gl;
    const int jl = lane >> gl;
    const int g = lane & (G - 1);
    valid = jl < n;
    id = !valid ? 0 : ids ? ids[jl] : id0 + jl;
    id = id < 0 ? 0 : id;
    float e = 0.f;
    if (valid && base) {
      const uint32_t* __restrict__ box = base + static_cast<size_t>(id) * static_cast<size_t>(box_dims);
      if constexpr (FD > 0) {
        // box_dims is a multiple of 8 here: 16-byte chunks of four dimensions,
        // lane g of a box takes chunks g, g + G, ..., three requested at a time
        // (chunks past the end read the lane's first one and add +0).
        const int nch = box_dims >> 2;
        const uint4* __restrict__ b4 = reinterpret_cast<const uint4*>(box);
        const float4* q4 = reinterpret_cast<const float4*>(qs);
        for (int k = g; k < nch; k += 3 * G) {
          uint4 bx[3];
#pragma unroll
          for (int i = 0; i < 3; ++i) bx[i] = b4[k + i * G < nch ? k + i * G : k];
#pragma unroll
          for (int i = 0; i < 3; ++i) {
            const float4 qv = q4[k + i * G < nch ? k + i * G : k];
            float t = box_acc(qv.x, bx[i].x, 0.f);
            t = box_acc(qv.y, bx[i].y, t);
            t = box_acc(qv.z, bx[i].z, t);
            t = box_acc(qv.w, bx[i].w, t);
            e = e + (k + i * G < nch ? t : 0.f);
          }
        }
      } else {
        const int cd = (box_dims + G - 1) >> gl;
        const int d_end = (g + 1) * cd < box_dims ? (g + 1) * cd : box_dims;
        for (int d = g * cd; d < d_end; ++d) e = box_acc(qs[d], box[d], e);
      }
    }
    return group_sum(e, gl);
  };
  // Lower bound of every probed list's scores from its box (16 lists per wave
  // pass): the sum over the subspace dimensions of the squared distance from the
  // residual q - c to the box. A list whose bound exceeds the K-th best score
  // when its turn comes is skipped without touching memory.
  if (lboxes) {
    for (int pb = wave * kSegPerPass; pb < a.P; pb += kWaves * kSegPerPass) {
      const int n = a.P - pb < kSegPerPass ? a.P - pb : kSegPerPass;
      int gl, id;
      bool valid;
      const float e = box_total(lboxes, t_list + pb, 0, n, gl, valid, id);
      if (valid && (lane & ((1 << gl) - 1)) == 0) t_lbound[pb + (lane >> gl)] = box_bound(e, slack, dims_all);
    }
  }
  // Ordinal bases (exclusive prefix sums of the rows) and the end of phase 0:
  // the first ranks holding 2K rows.
  if (wave == 0) {
    uint32_t base = 0;
    int bad = 0, p0 = -1, tasks_q = 0;
    for (int c = 0; c < a.P; c += 64) {
      const int t = c + lane;
      const uint32_t r = t < a.P ? static_cast<uint32_t>(t_rows[t]) : 0u;
      bad |= (t < a.P && t_list[t] < 0) ? 1 : 0;
      tasks_q += __popcll(__ballot(t < a.P && r > 0));
      const uint32_t incl = static_cast<uint32_t>(wave_incl_scan(static_cast<int32_t>(r)));
      if (t < a.P) t_ord[t] = base + incl - r;
      const uint64_t reach = __ballot(t < a.P && static_cast<uint64_t>(base) + incl >= 2u * static_cast<uint64_t>(K));
      if (p0 < 0 && reach) p0 = c + __builtin_ctzll(reach) + 1;
      base += __shfl(incl, 63, 64);
    }
    const uint64_t anybad = __ballot(bad != 0);
    if (lane == 0) {
      misc[0] = p0 < 0 ? a.P : p0;
      misc[1] = anybad ? 1 : 0;
      misc[2] = static_cast<int32_t>(base);
      misc[3] = tasks_q;
    }
  }
  __syncthreads();

  uint64_t lk[KPL];
  int32_t lp[KPL];
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    lk[j] = kNoKey;
    lp[j] = -1;
  }
  uint64_t thr = kNoKey;  // the wave's own K-th key
  // Score of the smallest K-th key any wave has published, and that score
  // raised by the bound allowance.
  float thr_f = __builtin_inff(), thr_hi = __builtin_inff();
  int cnt = 0, qcnt = 0;
  uint32_t ord_base = 0;

  auto refresh = [&]() {
    uint64_t t = wave_thr[0];
#pragma unroll
    for (int w = 1; w <= kWaves; ++w) t = wave_thr[w] < t ? wave_thr[w] : t;
    thr_f = key_score(t);
    thr_hi = thr_f * kBoundUp;
  };
  auto publish = [&]() {
    thr = kth_key<KPL>(lk, K);
    if (lane == 0) wave_thr[wave] = thr;
    refresh();
  };
  // Merges the first min(cnt, 64) buffered candidates into the wave's list.
  auto flush = [&]() {
    const int take = cnt < 64 ? cnt : 64;
    uint64_t bk = lane < take ? bufk[lane] : kNoKey;
    int32_t bp = lane < take ? bufp[lane] : -1;
    const int rest = cnt - take;
    if (lane < rest) {
      const uint64_t mk = bufk[64 + lane];
      const int32_t mp = bufp[64 + lane];
      bufk[lane] = mk;
      bufp[lane] = mp;
    }
    cnt = rest;
    sort64(bk, bp);
    merge64<KPL>(lk, lp, bk, bp);
    publish();
  };
  // Rows with their complete score (lanes with ok) are offered to the wave's list.
  auto offer = [&](bool ok, float score, int32_t pos) {
    uint64_t key = kNoKey;
    if (ok) key = make_key(score, ord_base + static_cast<uint32_t>(a.rord[pos]));
    const bool pass = key < thr;
    const uint64_t bal = __ballot(pass);
    if (bal) {
      const int before = __popcll(bal & ((1ull << lane) - 1ull));
      if (pass) {
        bufk[cnt + before] = key;
        bufp[cnt + before] = pos;
      }
      cnt += __popcll(bal);
      if (cnt >= 64) flush();
    }
  };
  // Completes up to 64 queued rows (scored through block 0) with the entries of
  // their remaining blocks, in subspace order; a row whose partial sum exceeds
  // the K-th best score already is dropped (entries are >= +0, so partial sums
  // never decrease).
  auto finish_queue = [&]() {
    const int take = qcnt < 64 ? qcnt : 64;
    const int32_t pos = lane < take ? qpos[lane] : 0;
    float sc = lane < take ? qsc[lane] : 0.f;
    const int rest = qcnt - take;
    if (lane < rest) {
      const int32_t p2 = qpos[64 + lane];
      const float s2 = qsc[64 + lane];
      qpos[lane] = p2;
      qsc[lane] = s2;
    }
    qcnt = rest;
    bool alive = lane < take;
    auto code_word = [&](int b) {
      return *reinterpret_cast<const uint2*>(a.codes + static_cast<size_t>(pos >> 6) * tile_bytes +
                                             b * (kTile * kBlock) + (pos & (kTile - 1)) * kBlock);
    };
    uint2 wnext = make_uint2(0u, 0u);
    if (alive && nblocks > 1) wnext = code_word(1);
    for (int b = 1; b < nblocks; ++b) {
      if (__ballot(alive) == 0) break;
      const int m0 = b * kBlock;
      const int mb = pq_m - m0 < kBlock ? pq_m - m0 : kBlock;
      const uint2 w = wnext;
      // The next block's code word is requested before this block's entries.
      if (alive && b + 1 < nblocks) wnext = code_word(b + 1);
      if (alive) {
        const uint32_t wv[2] = {w.x, w.y};
        if (FD > 0) {
          float v[kBlock];
#pragma unroll
          for (int j = 0; j < kBlock; ++j) {
            const int code = static_cast<int>((wv[j >> 2] >> (8 * (j & 3))) & 0xffu);
            v[j] = direct_entry<FD>(resid, a.codebooks, m0 + j, code, ks, dsub);
          }
#pragma unroll
          for (int j = 0; j < kBlock; ++j) sc = sc + v[j];
        } else {
          for (int j = 0; j < mb; ++j) {
            const int code = static_cast<int>((wv[j >> 2] >> (8 * (j & 3))) & 0xffu);
            sc = sc + direct_entry<FD>(resid, a.codebooks, m0 + j, code, ks, dsub);
          }
        }
      }
      alive = alive && !(sc > thr_f);
    }
    offer(alive, sc, pos);
  };

  // Completes the queued rows and folds the buffered candidates into the wave's
  // list, so that the published threshold is current: a few keys are inserted one
  // by one, more go through the sort-and-merge.
  auto settle = [&]() {
    while (qcnt > 0) finish_queue();
    if (cnt > 0 && cnt <= 8) {
      for (int t = 0; t < cnt; ++t) insert_one<KPL>(lk, lp, bufk[t], bufp[t]);
      cnt = 0;
      publish();
    } else {
      while (cnt > 0) flush();
    }
  };

  // Lower bound of every row's ADC score in each of n <= 16 segment boxes (box
  // ids[j] of base, list rank ps[j]): per dimension the squared distance from the query to
  // the box; the entry of subspace m is a sum of its dimensions' squared residual
  // differences, each at least that (up to box_bound's rounding allowance). S
  // boxes share the pass (n rounded up to a power of two), G = 64 / S lanes each;
  // lane g of a box takes the subspaces [g * c, (g + 1) * c), c = ceil(pq_m / G).
  // e0: block 0's subspaces, et: the others (partial sums of the lane).
  auto box_pass = [&](const uint32_t* __restrict__ base, const int32_t* ids, const int32_t* ps, int n, int& gl,
                      bool& valid, int& id, int& pp, float& e0, float& et) {
    gl = 2;  // log2(G)
    while (gl < 6 && (32 >> gl) >= n) ++gl;
    const int G = 1 << gl;
    const int jl = lane >> gl;
    const int g = lane & (G - 1);
    valid = jl < n;
    id = valid ? ids[jl] : 0;
    pp = valid ? ps[jl] : 0;
    e0 = 0.f;
    et = 0.f;
    if (valid && base) {
      const uint32_t* __restrict__ box = base + static_cast<size_t>(id) * static_cast<size_t>(box_dims);
      const int c = (pq_m + G - 1) >> gl;
      const int m_end = (g + 1) * c < pq_m ? (g + 1) * c : pq_m;
      if constexpr (FD > 0) {
        // Sixteen dimensions of box requested at a time, then reduced.
        constexpr int kBatch = FD >= 16 ? 1 : 16 / FD;
        for (int mb = g * c; mb < m_end; mb += kBatch) {
          // Subspaces past the chunk are clamped to its last one (the loads stay
          // unconditional) and their terms replaced by +0.
          uint32_t bx[kBatch][FD];
#pragma unroll
          for (int i = 0; i < kBatch; ++i) {
            const int m = mb + i < m_end ? mb + i : m_end - 1;
#pragma unroll
            for (int u = 0; u < FD; ++u) bx[i][u] = box[m * FD + u];
          }
#pragma unroll
          for (int i = 0; i < kBatch; ++i) {
            const int m = mb + i < m_end ? mb + i : m_end - 1;
            float part = 0.f;
#pragma unroll
            for (int u = 0; u < FD; ++u) part = part + box_e2(qs[m * FD + u], bx[i][u]);
            part = mb + i < m_end ? part : 0.f;
            e0 = e0 + (mb + i < kBlock ? part : 0.f);
            et = et + (mb + i < kBlock ? 0.f : part);
          }
        }
      } else {
        for (int m = g * c; m < m_end; ++m) {
          float part = 0.f;
          for (int u = 0; u < dsub; ++u) part = part + box_e2(qs[m * dsub + u], box[m * dsub + u]);
          if (m < kBlock) {
            e0 = e0 + part;
          } else {
            et = et + part;
          }
        }
      }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      if (o < G) {
        e0 = e0 + __uint_as_float(xor_lane(__float_as_uint(e0), o));
        et = et + __uint_as_float(xor_lane(__float_as_uint(et), o));
      }
    }
  };

  // Phase 0: in the nearest lists, until they hold 2K rows (or all of them), the
  // group with the smallest bound is scored completely by all four waves
  // together (64-row tiles in turn, table slices of 8 subspaces built in LDS from
  // coalesced codebook reads), so that every wave starts the rest with a
  // threshold; at the end of the phase the K-th best key of the union of the four
  // lists is published to every wave. The lists' other groups are left to the
  // independent phase. The slices live in the candidate-buffer and queue area,
  // unused until a chunk's rows are offered.
  constexpr int kP0Tiles = 2;  // tiles per wave per chunk (a group holds at most 8 tiles)
  static_assert(static_cast<size_t>(kBlock) * 256 * 4 <=
                    static_cast<size_t>(kWaves) * (kBufCap * 12 + kQueueCap * 8),
                "table slice must fit the candidate buffers and survivor queues");
  float* lut32 = reinterpret_cast<float*>(smem + L.bufk_off);
  const int ks_log2 = __ffs(ks) - 1;
  // Candidates: the first kP0Cand groups of ranks 0 .. kWaves-1 (wave w evaluates
  // rank w's) with their bounds, as keys (bound key << 32 | w * kP0Cand + j).
  uint64_t* p0c = reinterpret_cast<uint64_t*>(smem + L.slot_off);
  {
    for (int j = lane; j < kP0Cand; j += 64) p0c[wave * kP0Cand + j] = kNoKey;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int r = wave;
    const int ngc = r < a.P && t_rows[r] > 0 ? (t_ngrp[r] < kP0Cand ? t_ngrp[r] : kP0Cand) : 0;
    for (int j0 = 0; j0 < ngc; j0 += kSegPerPass) {
      const int n = ngc - j0 < kSegPerPass ? ngc - j0 : kSegPerPass;
      int gl, grp;
      bool valid;
      const float etot = box_bound(box_total(a.grp_box, nullptr, t_g0[r] + j0, n, gl, valid, grp), slack, dims_all);
      if (valid && (lane & ((1 << gl) - 1)) == 0) {
        const int c = wave * kP0Cand + j0 + (lane >> gl);
        p0c[c] = (static_cast<uint64_t>(score_key(etot)) << 32) | static_cast<uint32_t>(c);
      }
    }
  }
  constexpr int kRounds = KPL >= 2 ? kP0RoundsLong : kP0Rounds;
  if (threadIdx.x < kRounds) misc[4 + threadIdx.x] = -1;
  if (threadIdx.x == kRounds) misc[kMiscTiles] = 0;  // tiles scored after phase 0
  if (threadIdx.x == kRounds + 1) misc[kMiscRows] = 0;  // rows of the lists whose bound passed
  __syncthreads();
  // Rounds: the candidate with the smallest bound (ties: the first) is scored; a
  // further round runs while the best remaining candidate's bound does not exceed
  // the union's K-th best score (a group the rest of the search would score anyway).
  for (int round = 0; round < kRounds; ++round) {
    uint64_t best = kNoKey;
    for (int k = lane; k < kWaves * kP0Cand; k += 64) best = p0c[k] < best ? p0c[k] : best;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const uint64_t v = shfl_xor_u64(best, o);
      best = v < best ? v : best;
    }
    if (best == kNoKey || (round > 0 && key_score(best) > thr_hi)) break;
    const int ck = static_cast<int>(best & 0xffffffffu);
    const int p = ck / kP0Cand;
    const int bg = t_g0[p] + ck % kP0Cand;
    const int l = t_list[p];
    ord_base = t_ord[p];
    const float* __restrict__ cv = a.centroids + static_cast<int64_t>(l) * a.dim;
    for (int t = lane; t < a.dim; t += 64) resid[t] = qs[t] - cv[t];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // The group's segments are consecutive in scan order; padding rows have no
    // in-list index.
    const int sgf = a.grp_seg[bg];
    const int sgl = a.grp_seg[bg + 1] - 1;
    const int32_t first = a.seg_start[sgf];
    const int ntiles = (a.seg_start[sgl] + ((a.seg_len[sgl] + kTile - 1) & ~(kTile - 1)) - first) / kTile;
    for (int c = 0; c < ntiles; c += kWaves * kP0Tiles) {
      float sc[kP0Tiles];
      bool ok[kP0Tiles];
#pragma unroll
      for (int i = 0; i < kP0Tiles; ++i) {
        const int tile = c + wave + kWaves * i;
        const int32_t pos = first + tile * kTile + lane;
        sc[i] = 0.f;
        ok[i] = tile < ntiles && a.rord[tile < ntiles ? pos : first] >= 0;
        if (ok[i] && a.bitset) {
          const int64_t id = a.ids[pos];
          ok[i] = ((a.bitset[id >> 3] >> (id & 7)) & 1u) != 0;
        }
      }
      for (int b = 0; b < nblocks; ++b) {
        const int m0 = b * kBlock;
        const int mb = pq_m - m0 < kBlock ? pq_m - m0 : kBlock;
        // This block's code words, requested before the slice is built.
        uint2 wq[kP0Tiles];
#pragma unroll
        for (int i = 0; i < kP0Tiles; ++i) {
          const int tile = c + wave + kWaves * i;
          wq[i] = make_uint2(0u, 0u);
          if (ok[i]) {
            wq[i] = *reinterpret_cast<const uint2*>(a.codes +
                                                    static_cast<size_t>((first >> 6) + tile) * tile_bytes +
                                                    b * (kTile * kBlock) + lane * kBlock);
          }
        }
        __syncthreads();  // every wave is done with the previous slice (or buffers)
        if (FD > 0) {
          build_slice_256<(FD > 0 ? FD : 1)>(resid, a.codebooks, m0, lut32);
        } else {
          build_slice_any(resid, a.codebooks, m0, mb, ks, ks_log2, dsub, lut32);
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kP0Tiles; ++i) {
          const int tile = c + wave + kWaves * i;
          if (tile >= ntiles) continue;
          const uint32_t wv[2] = {wq[i].x, wq[i].y};
          float acc = sc[i];
          if (FD > 0) {
            float v[kBlock];
#pragma unroll
            for (int jj = 0; jj < kBlock; ++jj) {
              const int code = static_cast<int>((wv[jj >> 2] >> (8 * (jj & 3))) & 0xffu);
              v[jj] = lut32[jj * 256 + code];
            }
#pragma unroll
            for (int jj = 0; jj < kBlock; ++jj) acc = acc + v[jj];
          } else {
            for (int jj = 0; jj < mb; ++jj) {
              const int code = static_cast<int>((wv[jj >> 2] >> (8 * (jj & 3))) & 0xffu);
              const int idx = (jj << ks_log2) + code;
              acc = acc + lut32[idx];
            }
          }
          sc[i] = acc;
        }
      }
      __syncthreads();  // the slice area serves as candidate buffers again
#pragma unroll
      for (int i = 0; i < kP0Tiles; ++i) {
        const int tile = c + wave + kWaves * i;
        offer(ok[i], sc[i], first + tile * kTile + lane);
      }
      settle();
    }
    // Every wave has folded this round's candidates; wave 0 merges copies of the
    // four lists and publishes the K-th key of the union.
    constexpr int M = 64 * KPL;
    __syncthreads();
    if (threadIdx.x == 0) {
      p0c[ck] = kNoKey;
      misc[4 + round] = bg;
    }
    uint64_t* mk = reinterpret_cast<uint64_t*>(smem);
#pragma unroll
    for (int j = 0; j < KPL; ++j) mk[wave * M + j * 64 + lane] = lk[j];
    __syncthreads();
    if (wave == 0) {
      uint64_t tk[KPL];
      int32_t tp[KPL];
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        tk[j] = lk[j];
        tp[j] = 0;
      }
      for (int w = 1; w < kWaves; ++w) {
#pragma unroll
        for (int j = 0; j < KPL; ++j) {
          const uint64_t rk = mk[w * M + (KPL - 1 - j) * 64 + (63 - lane)];
          if (rk < tk[j]) tk[j] = rk;
        }
        bitonic_merge_asc<KPL>(tk, tp);
      }
      const uint64_t u = kth_key<KPL>(tk, K);
      if (lane == 0) wave_thr[kWaves] = u;
    }
    __syncthreads();
    refresh();
  }

  // The rest: the items are the groups of every probed list whose list bound does
  // not exceed the K-th best score, in rank order (the groups phase 0 scored are
  // passed over). They are dealt to the waves 16 at a time (pass j of wave w takes items
  // 64 j + 16 w onwards), up to kItemCap per round; the segments of the groups
  // whose bound does not exceed the K-th best are evaluated the same way, 16 at a
  // time, and the segments kept are scored grouped by list, best bound first within
  // a list.
  int32_t p0done[kRounds];  // groups phase 0 scored (-1: none), in scalar registers
#pragma unroll
  for (int r = 0; r < kRounds; ++r) p0done[r] = __builtin_amdgcn_readfirstlane(misc[4 + r]);
  int32_t* sslot = reinterpret_cast<int32_t*>(smem + L.slot_off) + wave * 2 * kSegSlots;
  int32_t* sslot_p = sslot + kSegSlots;
  int32_t* it_grp = reinterpret_cast<int32_t*>(smem + L.item_off);
  int16_t* it_rank = reinterpret_cast<int16_t*>(it_grp + kItemCap);
  // Item counts per rank and their prefix sums: wave w takes the 64-rank chunks
  // w, w + 4, ... (one rank per lane), chunk totals meet in LDS.
  int32_t* chunk_tot = t_item + a.P + 1;
  const int nchunk = (a.P + 63) >> 6;
  for (int c = wave; c < nchunk; c += kWaves) {
    const int t = 64 * c + lane;
    int32_t n = 0;
    if (t < a.P && t_rows[t] > 0 && !(lboxes && t_lbound[t] > thr_hi)) n = t_ngrp[t];
    int32_t live = n > 0 ? t_rows[t] : 0;  // rows of the lists whose bound passed
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) live += static_cast<int32_t>(xor_lane(static_cast<uint32_t>(live), o));
    if (lane == 0) atomicAdd(&misc[kMiscRows], live);
    const int32_t incl = wave_incl_scan(n);
    if (t < a.P) {
      t_item[t] = incl - n;  // within the chunk
      t_icnt[t] = n;         // the rounds below use these counts, whatever the threshold is then
    }
    if (lane == 63) chunk_tot[c] = incl;
  }
  __syncthreads();
  // First item of every chunk (at most 64 chunks: lane c holds chunk c's), in every wave.
  const int32_t ctot = lane < nchunk ? chunk_tot[lane] : 0;
  const int32_t cincl = wave_incl_scan(ctot);
  const int32_t cexcl = cincl - ctot;
  const int32_t n_items = __builtin_amdgcn_readlane(cincl, 63);
  // Handoff to the full-table scan, for data whose lower bounds do not prune (no
  // cluster structure, or no boxes): once the segments scored after phase 0 hold
  // more than `budget` tiles (kPuntTiles, or an eighth of the tiles of the lists
  // whose bound passed if that is more), the waves stop scoring, and the query is
  // handed off at the end (its outputs are then written by the full-table scan).
  const int32_t budget = a.punt ? max(kPuntTiles, misc[kMiscRows] / (8 * kTile)) : 0x7fffffff;
  auto over_budget = [&]() {
    return __hip_atomic_load(&misc[kMiscTiles], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) > budget;
  };
  int cur_p = -1;  // list whose residual is in resid
  for (int ib = 0; ib < n_items; ib += kItemCap) {
    const int nb = n_items - ib < kItemCap ? n_items - ib : kItemCap;
    // Items [ib, ib + nb) into LDS, each rank's by one lane.
    for (int t = static_cast<int>(threadIdx.x); t < a.P; t += kThreads) {
      const int o0 = __builtin_amdgcn_readlane(cexcl, __builtin_amdgcn_readfirstlane(t >> 6)) + t_item[t];
      const int cnt = t_icnt[t];
      const int g0 = t_g0[t];
      const int j0 = ib - o0 > 0 ? ib - o0 : 0;
      const int j1 = ib + nb - o0 < cnt ? ib + nb - o0 : cnt;
      for (int j = j0; j < j1; ++j) {
        it_grp[o0 + j - ib] = g0 + j;
        it_rank[o0 + j - ib] = static_cast<int16_t>(t);
      }
    }
    __syncthreads();
    for (int s0 = wave * kSegPerPass; s0 < nb; s0 += kWaves * kSegPerPass) {
    if (over_budget()) break;
    const int filled = nb - s0 < kSegPerPass ? nb - s0 : kSegPerPass;
    refresh();
    // Group bounds; the segments of the groups kept (in item order, so lists stay
    // in rank order) go to the segment slots.
    int ns = 0;
    {
      int gl, grp;
      bool valid;
      const float etot = box_bound(box_total(a.grp_box, it_grp + s0, 0, filled, gl, valid, grp), slack, dims_all);
      const int pp = valid ? static_cast<int>(it_rank[s0 + (lane >> gl)]) : 0;
      const int32_t gs0 = a.grp_seg[grp];
      const int32_t gs1 = a.grp_seg[grp + 1];
      refresh();
      bool done = false;
#pragma unroll
      for (int r = 0; r < kRounds; ++r) done |= grp == p0done[r];
      const bool lead = valid && (lane & ((1 << gl) - 1)) == 0 && !done && !(etot > thr_hi);
      for (uint64_t m = __builtin_amdgcn_ballot_w64(lead); m; m &= m - 1) {
        const int b = __builtin_ctzll(m);
        const int sg = __builtin_amdgcn_readlane(gs0, b);
        const int n1 = __builtin_amdgcn_readlane(gs1, b) - sg;
        const int n = n1 < OVVS_GROUP_SEGMENTS ? n1 : OVVS_GROUP_SEGMENTS;
        const int p = __builtin_amdgcn_readlane(pp, b);
        if (lane < n) {
          sslot[ns + lane] = sg + lane;
          sslot_p[ns + lane] = p;
        }
        ns += n;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int c0 = 0; c0 < ns; c0 += kSegPerPass) {
      const int remaining = ns - c0 < kSegPerPass ? ns - c0 : kSegPerPass;
      int gl, seg, pp;
      bool valid;
      float e0, et;
      box_pass(boxes, sslot + c0, sslot_p + c0, remaining, gl, valid, seg, pp, e0, et);
      const int g = lane & ((1 << gl) - 1);
      const float etot = box_bound(e0 + et, slack, dims_all);
      const float tb = box_bound(et, slack, dims_tail);
      const float tl = (tb > 0.f ? tb : 0.f) * kBoundDown;
      refresh();
      // Kept segments in (list, bound, slot) order: rank = number of kept segments
      // before this one.
      const bool lead = valid && g == 0 && !(etot > thr_hi);
      const uint64_t kept = __builtin_amdgcn_ballot_w64(lead);
      const uint32_t my_key = score_key(etot);
      int rank = 0;
      for (uint64_t m = kept; m;) {
        const int b = __builtin_ctzll(m);
        m &= m - 1;
        const int pb = __builtin_amdgcn_readlane(pp, b);
        const uint32_t kb = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(my_key), b));
        rank += (pb < pp || (pb == pp && (kb < my_key || (kb == my_key && b < lane)))) ? 1 : 0;
      }
      const int nkept = __popcll(kept);
      for (int r = 0; r < nkept; ++r) {
        const int b = __builtin_ctzll(__builtin_amdgcn_ballot_w64(lead && rank == r));
        // The threshold may have dropped since the pass (this wave's or another's).
        refresh();
        if (readlane_f(etot, b) > thr_hi || over_budget()) continue;
        const float tl_j = readlane_f(tl, b);
        const int gs = __builtin_amdgcn_readlane(seg, b);
        const int p = __builtin_amdgcn_readlane(pp, b);
        if (p != cur_p) {
          // A new list: complete the rows queued for the previous one (its residual
          // and ordinal base), then form this list's residual.
          settle();
          const int l = t_list[p];
          ord_base = t_ord[p];
          const float* __restrict__ cv = a.centroids + static_cast<int64_t>(l) * a.dim;
          for (int t = lane; t < a.dim; t += 64) resid[t] = qs[t] - cv[t];
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
          cur_p = p;
        }
        const int32_t st = a.seg_start[gs];
        const int32_t len = a.seg_len[gs];
        if (lane == 0) atomicAdd(&misc[kMiscTiles], (len + kTile - 1) / kTile);
        for (int32_t t0 = 0; t0 < len; t0 += kTile) {
          const int32_t pos0 = st + t0;
          const int32_t pos = pos0 + lane;
          bool ok = lane < len - t0;
          if (ok && a.bitset) {
            const int64_t id = a.ids[pos];
            ok = ((a.bitset[id >> 3] >> (id & 7)) & 1u) != 0;
          }
          uint2 w = make_uint2(0u, 0u);
          if (ok) {
            w = *reinterpret_cast<const uint2*>(a.codes + static_cast<size_t>(pos0 >> 6) * tile_bytes +
                                                lane * kBlock);
          }
          const uint32_t wv[2] = {w.x, w.y};
          // Block 0: the first min(8, pq_m) entries, added left to right from +0.
          float sc = 0.f;
          if (FD > 0) {
            float v[kBlock];
#pragma unroll
            for (int jj = 0; jj < kBlock; ++jj) {
              const int code = static_cast<int>((wv[jj >> 2] >> (8 * (jj & 3))) & 0xffu);
              v[jj] = direct_entry<FD>(resid, a.codebooks, jj, code, ks, dsub);
            }
#pragma unroll
            for (int jj = 0; jj < kBlock; ++jj) sc = sc + v[jj];
          } else {
            for (int jj = 0; jj < mb0; ++jj) {
              const int code = static_cast<int>((wv[jj >> 2] >> (8 * (jj & 3))) & 0xffu);
              sc = sc + direct_entry<FD>(resid, a.codebooks, jj, code, ks, dsub);
            }
          }
          if (nblocks == 1) {
            offer(ok, sc, pos);
          } else {
            // The rest of the row's score is at least the segment's tail bound.
            const bool surv = ok && !((sc + tl_j) > thr_hi);
            const uint64_t bal = __ballot(surv);
            if (bal) {
              const int before = __popcll(bal & ((1ull << lane) - 1ull));
              if (surv) {
                qpos[qcnt + before] = pos;
                qsc[qcnt + before] = sc;
              }
              qcnt += __popcll(bal);
              if (qcnt >= 64) finish_queue();
            }
          }
        }
        // Complete and publish at once, so that every wave prunes with the rows
        // scored so far.
        settle();
      }
    }
    }
    __syncthreads();  // every wave is done with this round's items
  }
  settle();

  // Cross-wave merge: each wave publishes its sorted list, wave 0 folds in the rest.
  constexpr int M = 64 * KPL;
  __syncthreads();
  uint64_t* mk = reinterpret_cast<uint64_t*>(smem);
  int32_t* mp = reinterpret_cast<int32_t*>(smem + static_cast<size_t>(kWaves) * M * 8);
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    mk[wave * M + j * 64 + lane] = lk[j];
    mp[wave * M + j * 64 + lane] = lp[j];
  }
  __syncthreads();
  if (wave == 0) {
    for (int w = 1; w < kWaves; ++w) {
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        const int src = w * M + (KPL - 1 - j) * 64 + (63 - lane);
        const uint64_t rk = mk[src];
        if (rk < lk[j]) {
          lk[j] = rk;
          lp[j] = mp[src];
        }
      }
      bitonic_merge_asc<KPL>(lk, lp);
    }
    int valid = 0;
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      const int e = j * 64 + lane;
      if (e < K) {
        a.out_keys[q * K + e] = lk[j];
        a.out_pos[q * K + e] = lp[j];
        valid += lk[j] != kNoKey;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) valid += static_cast<int>(xor_lane(static_cast<uint32_t>(valid), o));
    if (lane == 0 && misc[kMiscTiles] > budget) a.punt[atomicAdd(a.punt_count, 1u)] = static_cast<int32_t>(q);
    if (lane == 0) {
      a.out_count[q] = valid;
      // Per-query statistics, summed by the statistics workgroups of the refine
      // launch (no atomics here: tens of thousands of workgroups adding into one
      // address serialize).
      a.out_stats[q * 4 + 0] = misc[2];
      a.out_stats[q * 4 + 1] = misc[3];
      a.out_stats[q * 4 + 2] = valid;
      a.out_stats[q * 4 + 3] = misc[1];
    }
  }
}

// Shortlists of up to 64 keys run at 6 waves per SIMD (80 VGPRs, no spills), those of
// up to 128 at 7 (72 VGPRs): the scan is latency-bound, and measured on C2 (64 keys)
// 6 waves were within 1% of 7 without 7's spill traffic, and on C3 (128 keys) 7
// waves took 1.24-1.25 ms against 1.31 at 6. Longer register lists keep the
// compiler's own allocation.
template <int KPL, int FD>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(KPL == 1 ? 6 : 7))) void k_scan(
    const OvvsScanArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  if (a.stamp && blockIdx.x == 0 && threadIdx.x == 0) *a.stamp = wall_clock64();
  scan_query<KPL, FD>(a, smem);
}

template <int KPL>
__global__ __launch_bounds__(kThreads) void k_scan_long(const OvvsScanArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  if (a.stamp && blockIdx.x == 0 && threadIdx.x == 0) *a.stamp = wall_clock64();
  scan_query<KPL, 0>(a, smem);
}

template <int KPL>
hipError_t launch_scan(const OvvsScanArgs& a, size_t lds, hipStream_t stream) {
  void (*fn)(OvvsScanArgs);
  if constexpr (KPL <= 2) {
    const bool shaped = a.ks == 256 && a.pq_m % kBlock == 0;
    switch (shaped ? a.dsub : 0) {
      case 1: fn = k_scan<KPL, 1>; break;
      case 2: fn = k_scan<KPL, 2>; break;
      case 4: fn = k_scan<KPL, 4>; break;
      case 8: fn = k_scan<KPL, 8>; break;
      default: fn = k_scan<KPL, 0>;
    }
  } else {
    fn = k_scan_long<KPL>;
  }
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(a.nq)), dim3(kThreads), lds, stream, a);
  return hipGetLastError();
}

// ---- full-table scan (queries the bounded scan hands off) ----
//
// One workgroup per query (the grid's workgroups take the handed-off queries in
// turn). For every non-empty probed list in rank order: the whole table T[m][j] of
// the list in LDS (all 256 threads, entry by entry in the reference's operation
// order), then every row of the list scored from it, the rows offered to the wave's
// running top-K under the same (score, raw ordinal) keys as the bounded scan. No
// bound is evaluated: this serves data whose bounds rule nothing out, where building
// each list's table once costs less than computing entries row by row.
//
// Latency is what limits this loop (two barriers per list, few waves per CU), so
// every global load is issued ahead of its use: the codebook entries of the table
// stay in registers for the kernel's whole run when they fit (pq_m * ks * dsub <=
// 256 * kCbRegs; dim <= 96 at 256 centres per subspace), the next list's centroid is
// loaded while the current list is scored, and each wave loads the codes and
// ordinals of its next 64-row slot while it scores the current one. A list's rows
// are dealt in slots: slot 2s + h is rows [64h, 64h + 64) of the list's segment s
// (segments hold at most 128 rows), slot j to wave j % 4.
struct TableLayout {
  size_t lut_off;    // [pq_m][ks] f32; at the end, the cross-wave merge (aliased)
  size_t bufk_off;   // per wave: candidate keys [kBufCap]
  size_t bufp_off;   // per wave: candidate positions [kBufCap]
  size_t query_off;  // [dim_pad] f32
  size_t resid_off;  // [dim_pad] f32, the current list's residual
  size_t thr_off;    // [kWaves] u64 published K-th keys
  size_t meta_off;   // [4][P] int32: first segment, end segment, ordinal base, rows
  size_t total;
};

// Probes a handed-off query may have, and dimensions the full-table scan supports.
constexpr int kTableMaxProbes = 1024;
constexpr int kTableMaxDim = 1024;
// Floats of codebook entries each thread keeps in registers.
constexpr int kCbRegs = 96;
// Code blocks (8 subspaces each) whose words are loaded one slot ahead.
constexpr int kPfBlocks = 6;
// Table entries a thread computes together when the codebook is read from memory
// (their loads in flight at once).
constexpr int kTableBatch = 8;

__host__ __device__ inline TableLayout table_layout(int pq_m, int ks, int dim, int kpl, int P) {
  TableLayout L;
  const size_t dim_pad = static_cast<size_t>((dim + 3) & ~3);
  const size_t lut = static_cast<size_t>(pq_m) * ks * 4;
  const size_t merge = static_cast<size_t>(kWaves) * 64 * kpl * (8 + 4);
  L.lut_off = 0;
  L.bufk_off = round16(lut > merge ? lut : merge);
  L.bufp_off = L.bufk_off + static_cast<size_t>(kWaves) * kBufCap * 8;
  L.query_off = L.bufp_off + static_cast<size_t>(kWaves) * kBufCap * 4;
  L.resid_off = L.query_off + dim_pad * 4;
  L.thr_off = L.resid_off + dim_pad * 4;
  L.meta_off = L.thr_off + kWaves * 8;
  L.total = L.meta_off + static_cast<size_t>(P) * 16;
  return L;
}

// Subspaces whose codebook entries a thread can hold in kCbRegs registers (a multiple
// of 8, so that subspaces go in whole code blocks).
__host__ __device__ constexpr int cb_reg_subspaces(int ds) { return ds > 0 ? (kCbRegs / ds) & ~7 : 0; }

// True when thread-held codebook registers cover the whole table: 256 centres per
// subspace (thread t holds centre t of every subspace), dsub 1, 2, 4 or 8, and whole
// code blocks of subspaces (pq_m a multiple of 8) within the register budget.
__host__ __device__ inline bool table_cb_in_regs(int pq_m, int ks, int dsub) {
  return ks == kThreads && (dsub == 1 || dsub == 2 || dsub == 4 || dsub == 8) && pq_m % kBlock == 0 &&
         pq_m <= cb_reg_subspaces(dsub);
}

// Register copy of the codebook for table_cb_in_regs shapes: c[m] holds the DS
// coordinates of centre threadIdx.x of subspace m, loaded once per workgroup.
template <int DS>
struct CbRegs {
  float c[DS > 0 ? cb_reg_subspaces(DS) : 1][DS > 0 ? DS : 1];
};

template <int DS>
__device__ __forceinline__ void load_cb_regs(CbRegs<DS>& r, const float* __restrict__ codebooks, int pq_m) {
  if constexpr (DS > 0) {
#pragma unroll
    for (int m = 0; m < cb_reg_subspaces(DS); ++m) {
      const float* __restrict__ cw =
          codebooks + (static_cast<int64_t>(m < pq_m ? m : 0) * kThreads + threadIdx.x) * DS;
#pragma unroll
      for (int u = 0; u < DS; ++u) r.c[m][u] = m < pq_m ? cw[u] : 0.f;
    }
  }
}

// The table of one list: entry e = (m, j) is the sum over the subspace's coordinates
// u of (r[m * dsub + u] - codebook[e][u])^2, in order from +0 (the reference's table,
// src/neighbors/indexes.cpp:764-785). From the register copy when DS > 0 (thread t
// computes centre t of every subspace, eight subspaces per step under one uniform
// test), else from memory kTableBatch entries at a time.
template <int DS>
__device__ __forceinline__ void build_table(float* lut, const float* resid, const CbRegs<DS>& cr,
                                            const float* __restrict__ codebooks, int n_e,
                                            int ks_log2, int dsub, int pq_m) {
  if constexpr (DS > 0) {
#pragma unroll
    for (int g = 0; g < cb_reg_subspaces(DS); g += kBlock) {
      if (g < pq_m) {
        float acc[kBlock];
#pragma unroll
        for (int j = 0; j < kBlock; ++j) {
          const float* r = resid + (g + j) * DS;
          float t = 0.f;
#pragma unroll
          for (int u = 0; u < DS; ++u) {
            const float d = r[u] - cr.c[g + j][u];
            t = t + d * d;
          }
          acc[j] = t;
        }
#pragma unroll
        for (int j = 0; j < kBlock; ++j) lut[(g + j) * kThreads + threadIdx.x] = acc[j];
      }
    }
  } else {
    for (int e0 = static_cast<int>(threadIdx.x); e0 < n_e; e0 += kThreads * kTableBatch) {
      float c[kTableBatch][8];
      if (dsub <= 8) {
#pragma unroll
        for (int i = 0; i < kTableBatch; ++i) {
          const int e = e0 + i * kThreads;
          const float* __restrict__ cw = codebooks + static_cast<int64_t>(e < n_e ? e : 0) * dsub;
#pragma unroll
          for (int u = 0; u < 8; ++u) c[i][u] = u < dsub ? cw[u] : 0.f;
        }
      }
#pragma unroll
      for (int i = 0; i < kTableBatch; ++i) {
        const int e = e0 + i * kThreads;
        if (e < n_e) {
          const float* r = resid + (e >> ks_log2) * dsub;
          float acc = 0.f;
          if (dsub <= 8) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              if (u < dsub) {
                const float d = r[u] - c[i][u];
                acc = acc + d * d;
              }
            }
          } else {
            const float* __restrict__ cw = codebooks + static_cast<int64_t>(e) * dsub;
            for (int u = 0; u < dsub; ++u) {
              const float d = r[u] - cw[u];
              acc = acc + d * d;
            }
          }
          lut[e] = acc;
        }
      }
    }
  }
}

// One 64-row slot of a list, as loaded ahead of its scoring.
struct TableSlot {
  uint2 w[kPfBlocks];  // code words of the first kPfBlocks blocks
  int32_t pos;         // this lane's row position
  int32_t ord;         // its ordinal within the list (rord)
  bool ok;             // the lane holds a row that passes the filter
};

template <int KPL, int DS>
__device__ __forceinline__ void table_query(const OvvsScanArgs& a, int64_t q, unsigned char* smem,
                                            const CbRegs<DS>& cr) {
  const TableLayout L = table_layout(a.pq_m, a.ks, a.dim, KPL, a.P);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = lane_id();
  float* lut = reinterpret_cast<float*>(smem + L.lut_off);
  uint64_t* bufk = reinterpret_cast<uint64_t*>(smem + L.bufk_off) + wave * kBufCap;
  int32_t* bufp = reinterpret_cast<int32_t*>(smem + L.bufp_off) + wave * kBufCap;
  float* qs = reinterpret_cast<float*>(smem + L.query_off);
  float* resid = reinterpret_cast<float*>(smem + L.resid_off);
  uint64_t* wave_thr = reinterpret_cast<uint64_t*>(smem + L.thr_off);
  int32_t* m_seg0 = reinterpret_cast<int32_t*>(smem + L.meta_off);
  int32_t* m_seg1 = m_seg0 + a.P;
  int32_t* m_ord = m_seg1 + a.P;
  int32_t* m_rows = m_ord + a.P;
  const int K = a.K, P = a.P, pq_m = a.pq_m, dim = a.dim;
  const int ks_log2 = __ffs(a.ks) - 1;
  const int n_e = pq_m << ks_log2;
  const int nblocks = (pq_m + kBlock - 1) / kBlock;
  const uint32_t tile_bytes = static_cast<uint32_t>(nblocks) * kTile * kBlock;
  const int tid = static_cast<int>(threadIdx.x);

  // Per-rank metadata: segment range (empty for an empty or out-of-range list), rows,
  // and the ordinal base (rows of the lists before it), by contiguous chunks of ranks
  // per thread and a prefix sum of the chunk totals.
  const int chunk = (P + kThreads - 1) / kThreads;
  int32_t my_rows = 0, my_lists = 0, my_bad = 0;
  for (int p = tid * chunk; p < P && p < (tid + 1) * chunk; ++p) {
    const int l = a.probes[q * P + p];
    int32_t s0 = 0, s1 = 0, rows = 0;
    if (static_cast<uint32_t>(l) >= static_cast<uint32_t>(a.nlist)) {
      my_bad = 1;
    } else {
      rows = static_cast<int32_t>(a.list_offsets[l + 1] - a.list_offsets[l]);
      if (rows > 0) {
        s0 = a.list_seg[l];
        s1 = a.list_seg[l + 1];
        ++my_lists;
      }
    }
    m_seg0[p] = s0;
    m_seg1[p] = s1;
    m_rows[p] = rows;
    my_rows += rows;
  }
  for (int t = tid; t < dim; t += kThreads) qs[t] = a.queries[q * dim + t];
  if (lane == 0) wave_thr[wave] = kNoKey;
  // Block prefix of the chunk totals: the waves' sums (and list counts and bad-probe
  // flags) meet in their candidate areas, unused until the metadata is complete.
  const int32_t incl = wave_incl_scan(my_rows);
  int32_t* wsum = reinterpret_cast<int32_t*>(bufp);  // this wave's candidate area is unused yet
  const int32_t wave_total = __builtin_amdgcn_readlane(incl, 63);
  if (lane == 0) wsum[0] = wave_total;
  int32_t rows_total = 0, lists = 0, bad = 0;
  {
    int32_t l = my_lists, b = my_bad;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      l += __shfl_xor(l, o, 64);
      b |= __shfl_xor(b, o, 64);
    }
    lists = l;
    bad = b;
  }
  if (lane == 0) {
    wsum[1] = lists;
    wsum[2] = bad;
  }
  __syncthreads();
  int32_t before = 0;
  for (int w = 0; w < kWaves; ++w) {
    const int32_t* ws = reinterpret_cast<const int32_t*>(smem + L.bufp_off) + w * kBufCap;
    if (w < wave) before += ws[0];
    rows_total += ws[0];
    if (w != wave) {
      lists += ws[1];
      bad |= ws[2];
    }
  }
  {
    int32_t o = before + incl - my_rows;
    for (int p = tid * chunk; p < P && p < (tid + 1) * chunk; ++p) {
      m_ord[p] = o;
      o += m_rows[p];
    }
  }
  __syncthreads();  // metadata complete; the candidate areas are free again

  uint64_t lk[KPL];
  int32_t lp[KPL];
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    lk[j] = kNoKey;
    lp[j] = -1;
  }
  uint64_t thr = kNoKey;  // the smallest K-th key any wave has published
  int cnt = 0;
  uint32_t ord_base = 0;
  auto publish = [&]() {
    const uint64_t own = kth_key<KPL>(lk, K);
    if (lane == 0) wave_thr[wave] = own;
    uint64_t t = own;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) t = wave_thr[w] < t ? wave_thr[w] : t;
    thr = t;
  };
  auto flush = [&]() {
    const int take = cnt < 64 ? cnt : 64;
    uint64_t bk = lane < take ? bufk[lane] : kNoKey;
    int32_t bp = lane < take ? bufp[lane] : -1;
    const int rest = cnt - take;
    if (lane < rest) {
      const uint64_t mk = bufk[64 + lane];
      const int32_t mp = bufp[64 + lane];
      bufk[lane] = mk;
      bufp[lane] = mp;
    }
    cnt = rest;
    sort64(bk, bp);
    merge64<KPL>(lk, lp, bk, bp);
    publish();
  };
  auto offer = [&](bool ok, float score, int32_t pos, int32_t ord) {
    uint64_t key = kNoKey;
    if (ok) key = make_key(score, ord_base + static_cast<uint32_t>(ord));
    const bool pass = key < thr;
    const uint64_t bal = __ballot(pass);
    if (bal) {
      const int before_l = __popcll(bal & ((1ull << lane) - 1ull));
      if (pass) {
        bufk[cnt + before_l] = key;
        bufp[cnt + before_l] = pos;
      }
      cnt += __popcll(bal);
      if (cnt >= 64) flush();
    }
  };
  auto settle = [&]() {
    if (cnt > 0 && cnt <= 8) {
      for (int t = 0; t < cnt; ++t) insert_one<KPL>(lk, lp, bufk[t], bufp[t]);
      cnt = 0;
      publish();
    } else {
      while (cnt > 0) flush();
    }
  };
  // First rank at or after p whose list has rows (P when none).
  auto next_list = [&](int p) {
    while (p < P && m_seg1[p] == m_seg0[p]) ++p;
    return p;
  };
  // Slot k of list p for this wave: slot j = wave + 4k, rows [64 (j & 1), + 64) of the
  // list's segment j >> 1. Every load is issued whatever the slot holds (lanes without a
  // row read the segment's first row, blocks past the last re-read it), so that the
  // compiler can count the loads in flight exactly and wait only for the ones it uses.
  auto load_slot = [&](TableSlot& s, int pl, int k) {
    const int nslot = 2 * (m_seg1[pl] - m_seg0[pl]);
    const int j = wave + kWaves * k;
    const bool has = j < nslot;
    const int sg = __builtin_amdgcn_readfirstlane(m_seg0[pl] + (has ? (j >> 1) : 0));
    const int h = has ? (j & 1) : 0;
    const int32_t st = a.seg_start[sg];
    const int32_t len = a.seg_len[sg];
    s.pos = st + kTile * h + lane;
    s.ok = has && lane < len - kTile * h;
    const int32_t at = s.ok ? s.pos : st;
    const unsigned char* __restrict__ cb =
        a.codes + static_cast<size_t>(at >> 6) * tile_bytes + (at & (kTile - 1)) * kBlock;
#pragma unroll
    for (int b = 0; b < kPfBlocks; ++b)
      s.w[b] = *reinterpret_cast<const uint2*>(cb + (b < nblocks ? b : nblocks - 1) * (kTile * kBlock));
    s.ord = a.rord[at];
  };
  auto score_slot = [&](TableSlot& s) {
    if (a.bitset && s.ok) {
      const int64_t id = a.ids[s.pos];
      s.ok = ((a.bitset[id >> 3] >> (id & 7)) & 1u) != 0;
    }
    float sc = 0.f;
    const unsigned char* __restrict__ cb =
        a.codes + static_cast<size_t>(s.pos >> 6) * tile_bytes + (s.pos & (kTile - 1)) * kBlock;
    if constexpr (DS > 0) {
      // 256 centres per subspace and whole blocks: a block's eight entries are read
      // (at fixed offsets from the block's table rows), then added in subspace order.
      for (int b0 = 0; b0 < nblocks; b0 += kPfBlocks) {
#pragma unroll
        for (int i = 0; i < kPfBlocks; ++i) {
          if (b0 + i < nblocks) {
            const uint2 w = b0 == 0 ? s.w[i]
                                    : (s.ok ? *reinterpret_cast<const uint2*>(cb + (b0 + i) * (kTile * kBlock))
                                            : make_uint2(0u, 0u));
            const uint32_t wv[2] = {w.x, w.y};
            const float* lrow = lut + (b0 + i) * kBlock * kThreads;
            float v[kBlock];
#pragma unroll
            for (int jj = 0; jj < kBlock; ++jj)
              v[jj] = lrow[jj * kThreads + static_cast<int>((wv[jj >> 2] >> (8 * (jj & 3))) & 0xffu)];
#pragma unroll
            for (int jj = 0; jj < kBlock; ++jj) sc = sc + v[jj];
          }
        }
      }
      offer(s.ok, sc, s.pos, s.ord);
      return;
    }
    for (int b0 = 0; b0 < nblocks; b0 += kPfBlocks) {
      uint2 w[kPfBlocks];
#pragma unroll
      for (int i = 0; i < kPfBlocks; ++i)
        w[i] = b0 == 0 ? s.w[i]
                       : (s.ok && b0 + i < nblocks
                              ? *reinterpret_cast<const uint2*>(cb + (b0 + i) * (kTile * kBlock))
                              : make_uint2(0u, 0u));
#pragma unroll
      for (int i = 0; i < kPfBlocks; ++i) {
        const int m0 = (b0 + i) * kBlock;
        if (m0 >= pq_m) break;
        const int mb = pq_m - m0 < kBlock ? pq_m - m0 : kBlock;
        const uint32_t wv[2] = {w[i].x, w[i].y};
        if (mb == kBlock) {
#pragma unroll
          for (int jj = 0; jj < kBlock; ++jj) {
            const int code = static_cast<int>((wv[jj >> 2] >> (8 * (jj & 3))) & 0xffu);
            sc = sc + lut[((m0 + jj) << ks_log2) + code];
          }
        } else {
          for (int jj = 0; jj < mb; ++jj) {
            const int code = static_cast<int>((wv[jj >> 2] >> (8 * (jj & 3))) & 0xffu);
            sc = sc + lut[((m0 + jj) << ks_log2) + code];
          }
        }
      }
    }
    offer(s.ok, sc, s.pos, s.ord);
  };

  // Prologue: the first list's residual, the next list's centroid, this wave's first
  // two slots of the first list.
  int p = next_list(0);
  if (p >= P) p = P;
  constexpr int kCv = kTableMaxDim / kThreads;
  float cvn[kCv];
  // Centroid coordinates of the list of rank pl (the last list when pl == P, whose
  // values are then unused), loaded by every lane.
  auto load_centroid = [&](int pl) {
    const int l = a.probes[q * P + (pl < P ? pl : P - 1)];
    const int lc = static_cast<uint32_t>(l) < static_cast<uint32_t>(a.nlist) ? l : 0;
    const float* __restrict__ cv = a.centroids + static_cast<int64_t>(lc) * dim;
#pragma unroll
    for (int i = 0; i < kCv; ++i) {
      const int t = tid + i * kThreads;
      cvn[i] = cv[t < dim ? t : dim - 1];
    }
  };
  if (p < P) {
    const float* __restrict__ cv = a.centroids + static_cast<int64_t>(a.probes[q * P + p]) * dim;
    for (int t = tid; t < dim; t += kThreads) resid[t] = qs[t] - cv[t];
  }
  int pn = p < P ? next_list(p + 1) : P;
  load_centroid(pn);
  TableSlot nx0, nx1;
  if (p < P) {
    load_slot(nx0, p, 0);
    load_slot(nx1, p, 1);
  }

  while (p < P) {
    __syncthreads();  // list p's residual is complete; every wave is done with the previous table
    // This list's first two slots (loaded a list ago), then the next list's.
    TableSlot c0 = nx0, c1 = nx1;
    if (pn < P) {
      load_slot(nx0, pn, 0);
      load_slot(nx1, pn, 1);
    }
    build_table<DS>(lut, resid, cr, a.codebooks, n_e, ks_log2, a.dsub, pq_m);
    __syncthreads();
    // The residual area is free: the next list's residual, then the centroid after it.
    const int pnn = pn < P ? next_list(pn + 1) : P;
    if (pn < P) {
#pragma unroll
      for (int i = 0; i < kCv; ++i)
        if (tid + i * kThreads < dim) resid[tid + i * kThreads] = qs[tid + i * kThreads] - cvn[i];
      load_centroid(pnn);
    }
    ord_base = static_cast<uint32_t>(m_ord[p]);
    const int nslot = 2 * (m_seg1[p] - m_seg0[p]);
    if (wave < nslot) score_slot(c0);
    if (wave + kWaves < nslot) score_slot(c1);
    for (int k = 2; wave + kWaves * k < nslot; ++k) {
      TableSlot t;
      load_slot(t, p, k);
      score_slot(t);
    }
    settle();
    p = pn;
    pn = pnn;
  }

  // Cross-wave merge (the table area is free), as in the bounded scan.
  constexpr int M = 64 * KPL;
  __syncthreads();
  uint64_t* mk = reinterpret_cast<uint64_t*>(smem + L.lut_off);
  int32_t* mp = reinterpret_cast<int32_t*>(smem + L.lut_off + static_cast<size_t>(kWaves) * M * 8);
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    mk[wave * M + j * 64 + lane] = lk[j];
    mp[wave * M + j * 64 + lane] = lp[j];
  }
  __syncthreads();
  if (wave == 0) {
    for (int w = 1; w < kWaves; ++w) {
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        const int src = w * M + (KPL - 1 - j) * 64 + (63 - lane);
        const uint64_t rk = mk[src];
        if (rk < lk[j]) {
          lk[j] = rk;
          lp[j] = mp[src];
        }
      }
      bitonic_merge_asc<KPL>(lk, lp);
    }
    int valid = 0;
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      const int e = j * 64 + lane;
      if (e < K) {
        a.out_keys[q * K + e] = lk[j];
        a.out_pos[q * K + e] = lp[j];
        valid += lk[j] != kNoKey;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) valid += __shfl_xor(valid, o, 64);
    if (lane == 0) {
      a.out_count[q] = valid;
      a.out_stats[q * 4 + 0] = rows_total;
      a.out_stats[q * 4 + 1] = lists;
      a.out_stats[q * 4 + 2] = valid;
      a.out_stats[q * 4 + 3] = bad;
    }
  }
}

// Two waves per SIMD: the table's LDS holds two workgroups per CU at C2's shape, and
// the register copy of the codebook takes 96 of the 256 registers that leaves a wave.
template <int KPL, int DS>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_scan_table(
    const OvvsScanArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const unsigned int n = *a.punt_count;
  if (blockIdx.x >= n) return;
  CbRegs<DS> cr;
  load_cb_regs<DS>(cr, a.codebooks, a.pq_m);
  for (unsigned int i = blockIdx.x; i < n; i += gridDim.x) {
    table_query<KPL, DS>(a, a.punt[i], smem, cr);
    __syncthreads();  // LDS is reused by the next query
  }
}

// Workgroups of the full-table launch (each takes handed-off queries in turn): two per
// CU, as many as the table's LDS lets run at once at C2's shape.
constexpr unsigned kTableGrid = 512;

template <int KPL, int DS>
hipError_t launch_scan_table(const OvvsScanArgs& a, size_t lds, hipStream_t stream) {
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_scan_table<KPL, DS>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(lds));
    if (e != hipSuccess) return e;
  }
  const unsigned grid = a.nq < static_cast<int64_t>(kTableGrid) ? static_cast<unsigned>(a.nq) : kTableGrid;
  hipLaunchKernelGGL((k_scan_table<KPL, DS>), dim3(grid), dim3(kThreads), lds, stream, a);
  return hipGetLastError();
}

// ---- per-wave full scan (handed-off queries whose codebook fits in LDS) ----
//
// The same outputs as table_query, for shapes whose whole codebook fits in LDS beside
// sixteen waves' working areas (C2: 98 KB): one workgroup of sixteen waves per CU
// copies the codebook into LDS once, then every wave takes handed-off queries in turn
// and scores every row of every probed list on its own, one row per lane, each entry
// computed from the LDS codebook where the row uses it (direct_entry: the reference's
// table arithmetic) and added in subspace order. There is no per-list table build and
// no barrier after the copy, so sixteen independent waves per CU hide each other's
// code-load latency.
constexpr int kWaveScanWaves = 16;
constexpr int kWaveScanThreads = 64 * kWaveScanWaves;
// Workgroups of the per-wave launch: one per CU of an MI355X (each holds the codebook).
constexpr unsigned kWaveScanGrid = 256;

struct WaveScanLayout {
  size_t cb_off;       // [pq_m][ks][dsub] f32
  size_t wave_off;     // per wave, wave_stride bytes:
  size_t wave_stride;  //   query [dim_pad] f32 | residual [dim_pad] f32 | keys [kBufCap] u64 |
                       //   positions [kBufCap] i32
  size_t dim_bytes;    // dim_pad * 4, rounded to 16
  size_t total;
};

__host__ __device__ inline WaveScanLayout wave_scan_layout(int pq_m, int ks, int dsub, int dim) {
  WaveScanLayout L;
  L.cb_off = 0;
  L.wave_off = round16(static_cast<size_t>(pq_m) * ks * dsub * 4);
  L.dim_bytes = round16(static_cast<size_t>((dim + 3) & ~3) * 4);
  L.wave_stride = 2 * L.dim_bytes + static_cast<size_t>(kBufCap) * 12;
  L.total = L.wave_off + kWaveScanWaves * L.wave_stride;
  return L;
}

// The per-wave scan serves shortlists of up to 128 keys, dsub 1, 2, 4 or 8 and dim up
// to 1024 when its LDS fits a workgroup.
__host__ __device__ inline bool wave_scan_ok(int pq_m, int ks, int dsub, int dim, int K) {
  return K <= 128 && (dsub == 1 || dsub == 2 || dsub == 4 || dsub == 8) && dim <= kTableMaxDim &&
         wave_scan_layout(pq_m, ks, dsub, dim).total <= 160u * 1024u;
}

// part / nparts: the wave scores the lists of probe ranks p with p % nparts == part
// (every wave still walks all of them for the ordinal bases and statistics). With
// nparts > 1, nparts consecutive waves of the workgroup take parts of the same query
// and `areas` / `area_stride` locate their areas: each publishes its shortlist in its
// buffers, the part-0 wave merges them and writes the query's outputs. Every wave of
// the workgroup then passes two barriers (lists published, merge done); k_scan_wave
// has the waves without a query in that round pass two barriers of their own.
template <int KPL, int DS>
__device__ __forceinline__ void wave_query(const OvvsScanArgs& a, int64_t q, const float* cb,
                                           unsigned char* area, size_t dim_bytes, int part,
                                           int nparts, unsigned char* areas, size_t area_stride) {
  const int lane = lane_id();
  float* qs = reinterpret_cast<float*>(area);
  float* resid = reinterpret_cast<float*>(area + dim_bytes);
  uint64_t* bufk = reinterpret_cast<uint64_t*>(area + 2 * dim_bytes);
  int32_t* bufp = reinterpret_cast<int32_t*>(area + 2 * dim_bytes + static_cast<size_t>(kBufCap) * 8);
  const int K = a.K, P = a.P, pq_m = a.pq_m, dim = a.dim, ks = a.ks;
  const int nblocks = (pq_m + kBlock - 1) / kBlock;
  const uint32_t tile_bytes = static_cast<uint32_t>(nblocks) * kTile * kBlock;

  for (int t = lane; t < dim; t += 64) qs[t] = a.queries[q * dim + t];
  uint64_t lk[KPL];
  int32_t lp[KPL];
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    lk[j] = kNoKey;
    lp[j] = -1;
  }
  uint64_t thr = kNoKey;  // the wave's K-th key
  int cnt = 0;
  uint32_t ord_base = 0;
  auto flush = [&]() {
    const int take = cnt < 64 ? cnt : 64;
    uint64_t bk = lane < take ? bufk[lane] : kNoKey;
    int32_t bp = lane < take ? bufp[lane] : -1;
    const int rest = cnt - take;
    if (lane < rest) {
      const uint64_t mk = bufk[64 + lane];
      const int32_t mp = bufp[64 + lane];
      bufk[lane] = mk;
      bufp[lane] = mp;
    }
    cnt = rest;
    sort64(bk, bp);
    merge64<KPL>(lk, lp, bk, bp);
    thr = kth_key<KPL>(lk, K);
  };
  auto offer = [&](bool ok, float score, int32_t pos, int32_t ord) {
    uint64_t key = kNoKey;
    if (ok) key = make_key(score, ord_base + static_cast<uint32_t>(ord));
    const bool pass = key < thr;
    const uint64_t bal = __ballot(pass);
    if (bal) {
      const int before = __popcll(bal & ((1ull << lane) - 1ull));
      if (pass) {
        bufk[cnt + before] = key;
        bufp[cnt + before] = pos;
      }
      cnt += __popcll(bal);
      if (cnt >= 64) flush();
    }
  };

  int32_t rows_total = 0, lists = 0, bad = 0;
  uint32_t ord = 0;
  for (int p = 0; p < P; ++p) {
    const int l = a.probes[q * P + p];
    if (static_cast<uint32_t>(l) >= static_cast<uint32_t>(a.nlist)) {
      bad = 1;
      continue;
    }
    const int32_t rows = static_cast<int32_t>(a.list_offsets[l + 1] - a.list_offsets[l]);
    if (rows == 0) continue;
    rows_total += rows;
    ++lists;
    ord_base = ord;
    ord += static_cast<uint32_t>(rows);
    if (p % nparts != part) continue;
    const float* __restrict__ cv = a.centroids + static_cast<int64_t>(l) * dim;
    for (int t = lane; t < dim; t += 64) resid[t] = qs[t] - cv[t];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int s1 = a.list_seg[l + 1];
    for (int sg = a.list_seg[l]; sg < s1; ++sg) {
      const int32_t st = a.seg_start[sg];
      const int32_t len = a.seg_len[sg];
      for (int32_t t0 = 0; t0 < len; t0 += kTile) {
        const int32_t pos = st + t0 + lane;
        bool ok = lane < len - t0;
        const int32_t at = ok ? pos : st;
        if (ok && a.bitset) {
          const int64_t id = a.ids[pos];
          ok = ((a.bitset[id >> 3] >> (id & 7)) & 1u) != 0;
        }
        const int32_t rord = a.rord[at];
        const unsigned char* __restrict__ cbp =
            a.codes + static_cast<size_t>(at >> 6) * tile_bytes + (at & (kTile - 1)) * kBlock;
        float sc = 0.f;
        for (int b0 = 0; b0 < nblocks; b0 += kPfBlocks) {
          uint2 w[kPfBlocks];
#pragma unroll
          for (int i = 0; i < kPfBlocks; ++i)
            w[i] = *reinterpret_cast<const uint2*>(cbp + (b0 + i < nblocks ? b0 + i : nblocks - 1) * (kTile * kBlock));
#pragma unroll
          for (int i = 0; i < kPfBlocks; ++i) {
            const int m0 = (b0 + i) * kBlock;
            if (m0 >= pq_m) break;
            const int mb = pq_m - m0 < kBlock ? pq_m - m0 : kBlock;
            const uint32_t wv[2] = {w[i].x, w[i].y};
            if (mb == kBlock) {
              float v[kBlock];
#pragma unroll
              for (int j = 0; j < kBlock; ++j) {
                const int code = static_cast<int>((wv[j >> 2] >> (8 * (j & 3))) & 0xffu);
                v[j] = direct_entry<DS>(resid, cb, m0 + j, code, ks, DS);
              }
#pragma unroll
              for (int j = 0; j < kBlock; ++j) sc = sc + v[j];
            } else {
              for (int j = 0; j < mb; ++j) {
                const int code = static_cast<int>((wv[j >> 2] >> (8 * (j & 3))) & 0xffu);
                sc = sc + direct_entry<DS>(resid, cb, m0 + j, code, ks, DS);
              }
            }
          }
        }
        offer(ok, sc, pos, rord);
      }
    }
  }
  if (cnt > 0 && cnt <= 8) {
    for (int t = 0; t < cnt; ++t) insert_one<KPL>(lk, lp, bufk[t], bufp[t]);
    cnt = 0;
  } else {
    while (cnt > 0) flush();
  }
  if (nparts > 1) {
    // Each wave's list (ascending) in its buffers; wave 0 takes, for every other wave,
    // the smaller of each of its keys and the other list's mirror (the lower half of a
    // bitonic merge) and sorts the result: the K smallest keys of the union.
    static_assert(64 * KPL <= kBufCap, "a wave's list must fit its buffers");
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      bufk[j * 64 + lane] = lk[j];
      bufp[j * 64 + lane] = lp[j];
    }
    __syncthreads();
    if (part == 0) {
      for (int w = 1; w < nparts; ++w) {
        const unsigned char* wa = areas + static_cast<size_t>(w) * area_stride;
        const uint64_t* wk = reinterpret_cast<const uint64_t*>(wa + 2 * dim_bytes);
        const int32_t* wp =
            reinterpret_cast<const int32_t*>(wa + 2 * dim_bytes + static_cast<size_t>(kBufCap) * 8);
#pragma unroll
        for (int j = 0; j < KPL; ++j) {
          const int e = (KPL - 1 - j) * 64 + (63 - lane);
          const uint64_t rk = wk[e];
          if (rk < lk[j]) {
            lk[j] = rk;
            lp[j] = wp[e];
          }
        }
        bitonic_merge_asc<KPL>(lk, lp);
      }
    }
    __syncthreads();  // the other parts' buffers are read
    if (part != 0) return;
  }
  int valid = 0;
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    const int e = j * 64 + lane;
    if (e < K) {
      a.out_keys[q * K + e] = lk[j];
      a.out_pos[q * K + e] = lp[j];
      valid += lk[j] != kNoKey;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) valid += __shfl_xor(valid, o, 64);
  if (lane == 0) {
    a.out_count[q] = valid;
    a.out_stats[q * 4 + 0] = rows_total;
    a.out_stats[q * 4 + 1] = lists;
    a.out_stats[q * 4 + 2] = valid;
    a.out_stats[q * 4 + 3] = bad;
  }
}

template <int KPL, int DS>
__global__ __launch_bounds__(kWaveScanThreads) void k_scan_wave(const OvvsScanArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const unsigned int n = *a.punt_count;
  // G queries per workgroup and round (the smallest power of two covering its share, at
  // most one per wave), each taken by kWaveScanWaves / G waves.
  const unsigned int share = (n + gridDim.x - 1) / gridDim.x;
  unsigned int G = 1;
  while (G < share && G < static_cast<unsigned int>(kWaveScanWaves)) G <<= 1;
  if (blockIdx.x * G >= n) return;  // no query for this workgroup in any round
  const WaveScanLayout L = wave_scan_layout(a.pq_m, a.ks, DS, a.dim);
  float* cb = reinterpret_cast<float*>(smem + L.cb_off);
  const int n4 = a.pq_m * a.ks * DS / 4;  // ks >= 16: a whole number of 16-byte vectors
  const float4* src = reinterpret_cast<const float4*>(a.codebooks);
  for (int i = static_cast<int>(threadIdx.x); i < n4; i += kWaveScanThreads)
    reinterpret_cast<float4*>(cb)[i] = src[i];
  __syncthreads();
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  unsigned char* area = smem + L.wave_off + static_cast<size_t>(wave) * L.wave_stride;
  const int nparts = kWaveScanWaves / static_cast<int>(G);
  if (nparts == 1) {
    for (unsigned int i = blockIdx.x * kWaveScanWaves + wave; i < n; i += gridDim.x * kWaveScanWaves)
      wave_query<KPL, DS>(a, a.punt[i], cb, area, L.dim_bytes, 0, 1, nullptr, 0);
    return;
  }
  const int g = wave / nparts, part = wave - g * nparts;
  unsigned char* group_areas = smem + L.wave_off + static_cast<size_t>(g * nparts) * L.wave_stride;
  const unsigned int rounds = (n + gridDim.x * G - 1) / (gridDim.x * G);
  for (unsigned int r = 0; r < rounds; ++r) {
    const unsigned int i = (r * gridDim.x + blockIdx.x) * G + static_cast<unsigned int>(g);
    if (i < n) {
      wave_query<KPL, DS>(a, a.punt[i], cb, area, L.dim_bytes, part, nparts, group_areas,
                          L.wave_stride);
    } else {
      __syncthreads();  // as a query's part does: lists published,
      __syncthreads();  // then merged
    }
  }
}

template <int KPL, int DS>
hipError_t launch_scan_wave(const OvvsScanArgs& a, hipStream_t stream) {
  const size_t lds = wave_scan_layout(a.pq_m, a.ks, DS, a.dim).total;
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_scan_wave<KPL, DS>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((k_scan_wave<KPL, DS>), dim3(kWaveScanGrid), dim3(kWaveScanThreads), lds, stream, a);
  return hipGetLastError();
}

int kpl_for(int K) { return K <= 64 ? 1 : K <= 128 ? 2 : K <= 256 ? 4 : K <= 512 ? 8 : 16; }

}  // namespace

extern "C" size_t ovvs_hip_scan_lds_bytes(int32_t pq_m, int32_t ks, int32_t dim, int32_t K,
                                          int32_t P) {
  if (pq_m <= 0 || ks <= 0 || dim <= 0 || K <= 0 || K > OVVS_HIP_MAX_REFINE || P <= 0 ||
      P > OVVS_HIP_MAX_PROBES)
    return 0;
  const size_t b = scan_layout(dim, kpl_for(K), P).total;
  return b <= 160u * 1024u ? b : 0;
}

extern "C" hipError_t ovvs_hip_scan(const OvvsScanArgs* args, hipStream_t stream) {
  if (!args) return hipErrorInvalidValue;
  const OvvsScanArgs& a = *args;
  if (a.nq <= 0) return hipSuccess;
  if (!a.queries || !a.probes || !a.centroids || !a.codebooks || !a.list_offsets || !a.codes ||
      !a.ids || !a.rord || !a.list_seg || !a.seg_start || !a.seg_len || !a.list_grp || !a.grp_seg ||
      (a.seg_box && !a.grp_box) || a.positions <= 0 ||
      a.positions > 0x7fffffff || !a.out_keys || !a.out_pos || !a.out_count || !a.out_stats ||
      a.nq > 0x7fffffff ||
      a.nlist <= 0 ||
      a.dim <= 0 || a.P <= 0 || a.pq_m <= 0 || a.dsub <= 0 || a.ks < 16 || a.ks > 256 ||
      (a.ks & (a.ks - 1)) != 0 || a.code_blocks != (a.pq_m + kBlock - 1) / kBlock ||
      static_cast<int64_t>(a.pq_m) * a.dsub > a.dim || a.K <= 0 || a.K > OVVS_HIP_MAX_REFINE ||
      (a.seg_box && static_cast<int64_t>(a.pq_m) * a.dsub > OVVS_MAX_BOX_DIMS))
    return hipErrorInvalidValue;
  const int kpl = kpl_for(a.K);
  if (a.P > OVVS_HIP_MAX_PROBES) return hipErrorInvalidValue;
  const size_t lds = scan_layout(a.dim, kpl, a.P).total;
  if (lds > 160u * 1024u) return hipErrorInvalidValue;
  switch (kpl) {
    case 1: return launch_scan<1>(a, lds, stream);
    case 2: return launch_scan<2>(a, lds, stream);
    case 4: return launch_scan<4>(a, lds, stream);
    case 8: return launch_scan<8>(a, lds, stream);
    default: return launch_scan<16>(a, lds, stream);
  }
}

extern "C" size_t ovvs_hip_scan_table_lds_bytes(int32_t pq_m, int32_t ks, int32_t dim, int32_t K,
                                                int32_t P) {
  if (pq_m <= 0 || ks <= 0 || dim <= 0 || dim > kTableMaxDim || K <= 0 || K > OVVS_HIP_MAX_REFINE ||
      P <= 0 || P > kTableMaxProbes)
    return 0;
  const size_t b = table_layout(pq_m, ks, dim, kpl_for(K), P).total;
  return b <= 160u * 1024u ? b : 0;
}

extern "C" hipError_t ovvs_hip_scan_table(const OvvsScanArgs* args, hipStream_t stream) {
  if (!args) return hipErrorInvalidValue;
  const OvvsScanArgs& a = *args;
  if (a.nq <= 0 || !a.punt) return hipSuccess;
  if (!a.punt_count || !a.queries || !a.probes || !a.centroids || !a.codebooks || !a.list_offsets ||
      !a.codes || !a.ids || !a.rord || !a.list_seg || !a.seg_start || !a.seg_len || !a.out_keys ||
      !a.out_pos || !a.out_count || !a.out_stats || a.nq > 0x7fffffff || a.nlist <= 0 || a.dim <= 0 ||
      a.P <= 0 || a.pq_m <= 0 || a.dsub <= 0 || a.ks < 16 || a.ks > 256 || (a.ks & (a.ks - 1)) != 0 ||
      a.code_blocks != (a.pq_m + kBlock - 1) / kBlock || static_cast<int64_t>(a.pq_m) * a.dsub > a.dim ||
      a.K <= 0 || a.K > OVVS_HIP_MAX_REFINE)
    return hipErrorInvalidValue;
  const size_t lds = ovvs_hip_scan_table_lds_bytes(a.pq_m, a.ks, a.dim, a.K, a.P);
  if (lds == 0) return hipErrorInvalidValue;
  const int kpl = kpl_for(a.K);
  if (wave_scan_ok(a.pq_m, a.ks, a.dsub, a.dim, a.K)) {
    switch (a.dsub * 4 + kpl) {
      case 1 * 4 + 1: return launch_scan_wave<1, 1>(a, stream);
      case 2 * 4 + 1: return launch_scan_wave<1, 2>(a, stream);
      case 4 * 4 + 1: return launch_scan_wave<1, 4>(a, stream);
      case 8 * 4 + 1: return launch_scan_wave<1, 8>(a, stream);
      case 1 * 4 + 2: return launch_scan_wave<2, 1>(a, stream);
      case 2 * 4 + 2: return launch_scan_wave<2, 2>(a, stream);
      case 4 * 4 + 2: return launch_scan_wave<2, 4>(a, stream);
      default: return launch_scan_wave<2, 8>(a, stream);
    }
  }
  if (kpl <= 2 && table_cb_in_regs(a.pq_m, a.ks, a.dsub)) {
    switch (a.dsub * 4 + kpl) {
      case 1 * 4 + 1: return launch_scan_table<1, 1>(a, lds, stream);
      case 2 * 4 + 1: return launch_scan_table<1, 2>(a, lds, stream);
      case 4 * 4 + 1: return launch_scan_table<1, 4>(a, lds, stream);
      case 8 * 4 + 1: return launch_scan_table<1, 8>(a, lds, stream);
      case 1 * 4 + 2: return launch_scan_table<2, 1>(a, lds, stream);
      case 2 * 4 + 2: return launch_scan_table<2, 2>(a, lds, stream);
      case 4 * 4 + 2: return launch_scan_table<2, 4>(a, lds, stream);
      default: return launch_scan_table<2, 8>(a, lds, stream);
    }
  }
  switch (kpl) {
    case 1: return launch_scan_table<1, 0>(a, lds, stream);
    case 2: return launch_scan_table<2, 0>(a, lds, stream);
    case 4: return launch_scan_table<4, 0>(a, lds, stream);
    case 8: return launch_scan_table<8, 0>(a, lds, stream);
    default: return launch_scan_table<16, 0>(a, lds, stream);
  }
}

// Bucket of every query: the spatial rank of its nearest probed list, shifted to at
// most 4096 buckets (bucket 0 for an invalid probe id).
__global__ __launch_bounds__(256) void k_query_keys(const int32_t* __restrict__ probes, int64_t nq, int P,
                                                    const int32_t* __restrict__ list_rank, int nlist, int shift,
                                                    int32_t* __restrict__ keys) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (q >= nq) return;
  const int l = probes[q * P];
  const bool in = static_cast<uint32_t>(l) < static_cast<uint32_t>(nlist);
  keys[q] = in ? (list_rank[l] >> shift) : 0;
}

// Counting sort of the queries by bucket; one workgroup, LDS counters.
constexpr int kOrderThreads = 1024;
constexpr int kOrderKeys = 16;  // keys per thread held in registers
__global__ __launch_bounds__(kOrderThreads) void k_query_order(const int32_t* __restrict__ keys, int64_t nq,
                                                               int32_t* __restrict__ order) {
  __shared__ int32_t hist[4096];
  __shared__ int32_t wsum[kOrderThreads / 64];
  const int t = static_cast<int>(threadIdx.x);
  const int lane = lane_id(), wave = t >> 6;
  // Batches of kOrderKeys keys stay in registers between the count and the
  // placement when the batch holds them all (nq <= kOrderKeys * kOrderThreads).
  const bool held = nq <= static_cast<int64_t>(kOrderKeys) * kOrderThreads;
  int32_t kv[kOrderKeys];
#pragma unroll
  for (int j = 0; j < kOrderKeys; ++j) {
    const int64_t q = t + static_cast<int64_t>(j) * kOrderThreads;
    kv[j] = held && q < nq ? keys[q] : -1;
  }
  for (int i = t; i < 4096; i += kOrderThreads) hist[i] = 0;
  __syncthreads();
  if (held) {
#pragma unroll
    for (int j = 0; j < kOrderKeys; ++j)
      if (kv[j] >= 0) atomicAdd(&hist[kv[j]], 1);
  } else {
    for (int64_t q = t; q < nq; q += kOrderThreads) atomicAdd(&hist[keys[q]], 1);
  }
  __syncthreads();
  // Exclusive prefix sums of the 4096 counters: four per thread, then across the
  // lanes of each wave and across the 16 waves.
  int32_t c[4];
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c[i] = hist[4 * t + i];
    s += c[i];
  }
  const int32_t incl = wave_incl_scan(s);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int32_t base = 0;
  for (int w = 0; w < wave; ++w) base += wsum[w];
  base += incl - s;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hist[4 * t + i] = base;
    base += c[i];
  }
  __syncthreads();
  if (held) {
#pragma unroll
    for (int j = 0; j < kOrderKeys; ++j)
      if (kv[j] >= 0) order[atomicAdd(&hist[kv[j]], 1)] = t + j * kOrderThreads;
  } else {
    for (int64_t q = t; q < nq; q += kOrderThreads) order[atomicAdd(&hist[keys[q]], 1)] = static_cast<int32_t>(q);
  }
}

extern "C" int32_t ovvs_hip_query_key_shift(int32_t nlist) {
  int32_t shift = 0;
  while (nlist > 0 && ((nlist - 1) >> shift) >= 4096) ++shift;
  return shift;
}

extern "C" hipError_t ovvs_hip_query_order(const int32_t* probes, int64_t nq, int32_t P, const int32_t* list_rank,
                                           int32_t nlist, int32_t* keys, int32_t keys_ready, int32_t* order,
                                           hipStream_t stream) {
  if (nq <= 0) return hipSuccess;
  if (!probes || !list_rank || !keys || !order || P <= 0 || nlist <= 0 || nq > 0x7fffffff)
    return hipErrorInvalidValue;
  const int shift = ovvs_hip_query_key_shift(nlist);
  if (!keys_ready) {
    hipLaunchKernelGGL(k_query_keys, dim3(static_cast<uint32_t>((nq + 255) / 256)), dim3(256), 0, stream, probes,
                       nq, static_cast<int>(P), list_rank, static_cast<int>(nlist), shift, keys);
  }
  hipLaunchKernelGGL(k_query_order, dim3(1), dim3(kOrderThreads), 0, stream, keys, nq, order);
  return hipGetLastError();
}

