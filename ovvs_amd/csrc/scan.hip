// scan.hip — fused residual-LUT build + PQ code scan + shortlist select for
// IVF-PQ search on gfx950.
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
// Design (one 256-lane workgroup per query, four wave64s):
//   * Rows are processed in chunks of up to 2048 (8 per lane, partial sums in
//     registers) and subspaces in blocks of 8. For each block the workgroup
//     builds only that block's 8 x ks table slice into LDS (each entry with the
//     reference's operation order), then every live row adds its 8 entries in
//     order m = 8b..8b+7.
//   * Table entries are squared distances (>= +0, or NaN), so fp32 partial sums
//     never decrease. A row whose partial sum already exceeds the K-th best key
//     of any wave (each such key has K better rows behind it) cannot enter the
//     shortlist and is dropped; when a block has no live row left the remaining
//     blocks (their table slices and their code bytes) are skipped. Surviving
//     rows are scored completely, so the shortlist is exactly the reference's.
//   * Codes are stored tiled: 64-row tiles, inside a tile 8-byte slabs of one
//     block for 64 consecutive rows, so a wave's block load is one coalesced
//     512-byte access and skipped blocks are never fetched.
//   * Each wave keeps its own running top-K as a sorted register list (64 keys
//     per register row, KPL rows), a 128-slot LDS candidate buffer and a
//     threshold it publishes in LDS: rows are appended with ballot/popcount (no
//     atomics), buffers are merged by a cross-lane bitonic sort plus a bitonic
//     merge, and at the end the four lists are merged once.
// Keys are (order-preserving score bits << 32 | raw ordinal); raw ordinals count
// every row of earlier probed lists, which orders accepted rows exactly as the
// dense ordinal does.
#include <hip/hip_fp16.h>

#include "device_common.hpp"
#include "kernels.hpp"

using namespace ovvs_dev;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kBufCap = 128;
constexpr int kRowsPerLane = 8;
constexpr int kChunkRows = kThreads * kRowsPerLane;
constexpr int kBlock = OVVS_CODE_BLOCK;      // subspaces per block (8)
constexpr int kTile = OVVS_CODE_TILE_ROWS;   // rows per code tile (64)

__host__ __device__ constexpr size_t round16(size_t b) { return (b + 15) & ~static_cast<size_t>(15); }

// Compare-exchange of (k, p) with the lane `s` away; this lane keeps the
// smaller key when keep_min.
__device__ __forceinline__ void cx_lane(uint64_t& k, int32_t& p, int s, bool keep_min) {
  const uint64_t ok = shfl_xor_u64(k, s);
  const int32_t op = __shfl_xor(p, s, 64);
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
  const int lane = lane_id();
  const uint64_t rk = shfl_u64(bk, 63 - lane);
  const int32_t rp = __shfl(bp, 63 - lane, 64);
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
  return shfl_u64(v, (K - 1) & 63);
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
    // Element e = j*64 + lane takes element e-1 when e > at.
    uint64_t up = shfl_u64(lk[j], (lane + 63) & 63);
    int32_t upp = __shfl(lp[j], (lane + 63) & 63, 64);
    const uint64_t tail = shfl_u64(lk[j], 63);
    const int32_t tailp = __shfl(lp[j], 63, 64);
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

// build_slice for ks == 256: thread j computes entry (i, j) of every subspace i of
// the slice; codebook loads are issued a group of subspaces (16 floats) at a time
// ahead of the arithmetic.
template <int DSUB, bool F16>
__device__ __forceinline__ void build_slice_256(const float* resid,
                                                const float* __restrict__ codebooks, int m0,
                                                int mb, float* lut32, uint16_t* lut16) {
  constexpr int kGroup = DSUB <= 2 ? kBlock : 16 / DSUB;
  const int j = static_cast<int>(threadIdx.x);
  const float* __restrict__ cb = codebooks + (static_cast<int64_t>(m0) * 256 + j) * DSUB;
#pragma unroll
  for (int g0 = 0; g0 < kBlock; g0 += kGroup) {
    Codeword<DSUB> cw[kGroup];
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      if (g0 + i < mb) cw[i].load(cb + (g0 + i) * 256 * DSUB);
    }
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      if (g0 + i < mb) {
        const float* r = resid + (m0 + g0 + i) * DSUB;
        float acc = 0.f;
#pragma unroll
        for (int u = 0; u < DSUB; ++u) {
          const float t = r[u] - cw[i].v[u];
          acc = acc + t * t;
        }
        if (F16) {
          lut16[(g0 + i) * 256 + j] = __half_as_ushort(__float2half_rn(acc));
        } else {
          lut32[(g0 + i) * 256 + j] = acc;
        }
      }
    }
  }
}

// Builds the table slice of subspaces [m0, m0 + mb) into LDS: entry
// (m - m0) * ks + j = sum_u (r[m*dsub+u] - B[m][j][u])^2, left to right from +0.
template <int DSUB, bool F16>
__device__ __forceinline__ void build_slice(const float* resid, const float* __restrict__ codebooks,
                                            int m0, int mb, int ks, int ks_log2, int dsub,
                                            float* lut32, uint16_t* lut16) {
  if constexpr (DSUB == 1 || DSUB == 2 || DSUB == 4 || DSUB == 8) {
    if (ks == 256) {
      build_slice_256<DSUB, F16>(resid, codebooks, m0, mb, lut32, lut16);
      return;
    }
  }
  const int d = DSUB > 0 ? DSUB : dsub;
  const int slice = mb << ks_log2;
  for (int e = threadIdx.x; e < slice; e += 256) {
    const int m = m0 + (e >> ks_log2);
    const float* r = resid + m * d;
    const float* __restrict__ cw = codebooks + (static_cast<int64_t>(m) * ks + (e & (ks - 1))) * d;
    float acc = 0.f;
    if (DSUB > 0) {
#pragma unroll
      for (int u = 0; u < DSUB; ++u) {
        const float t = r[u] - cw[u];
        acc = acc + t * t;
      }
    } else {
      for (int u = 0; u < d; ++u) {
        const float t = r[u] - cw[u];
        acc = acc + t * t;
      }
    }
    if (F16) {
      lut16[e] = __half_as_ushort(__float2half_rn(acc));
    } else {
      lut32[e] = acc;
    }
  }
}

// Byte offset of (packed row pos, block b) in the tiled code layout.
__device__ __forceinline__ int64_t code_offset(int64_t pos, int b, int nblocks) {
  return (pos / kTile) * (static_cast<int64_t>(nblocks) * kTile * kBlock) +
         static_cast<int64_t>(b) * (kTile * kBlock) + (pos % kTile) * kBlock;
}

// One block's table slice lives in static LDS (its address is then a link-time
// constant, folded into the table reads' immediate offsets); the rest is dynamic.
constexpr size_t kLutBytes = static_cast<size_t>(kBlock) * 256 * 4;

struct ScanLayout {
  size_t merge_bytes;  // the final cross-wave merge of the wave lists
  size_t resid_off;
  size_t thr_off;
  size_t any_off;
  size_t bufk_off;
  size_t bufp_off;
  size_t total;
};

__host__ __device__ inline ScanLayout scan_layout(int dim, int kpl) {
  ScanLayout L;
  L.merge_bytes = round16(static_cast<size_t>(kWaves) * 64 * kpl * (8 + 4));
  L.resid_off = L.merge_bytes;
  L.thr_off = L.resid_off + round16(static_cast<size_t>(dim) * 4);
  L.any_off = L.thr_off + kWaves * 8;
  L.bufk_off = L.any_off + round16(2 * kWaves * 4);
  L.bufp_off = L.bufk_off + static_cast<size_t>(kWaves) * kBufCap * 8;
  L.total = L.bufp_off + static_cast<size_t>(kWaves) * kBufCap * 4;
  return L;
}

// FD > 0: the shape-specialised body for ks = 256, pq_m % 8 == 0 and dsub = FD
// (every block full, table rows 1 KiB apart); FD = 0: any shape.
template <int KPL, bool F16, int FD>
__device__ __forceinline__ void scan_query(const OvvsScanArgs& a, unsigned char* smem) {
  const ScanLayout L = scan_layout(a.dim, KPL);
  __shared__ __attribute__((aligned(16))) float s_lut[kLutBytes / 4];
  float* lut32 = s_lut;
  uint16_t* lut16 = reinterpret_cast<uint16_t*>(s_lut);
  float* resid = reinterpret_cast<float*>(smem + L.resid_off);
  uint64_t* wave_thr = reinterpret_cast<uint64_t*>(smem + L.thr_off);
  // Per wave: 1 while any of its rows of the current chunk is alive, in two
  // slots used by alternate reads (any_rd is the slot the next read uses; every
  // wave performs the same sequence of reads). A wave that leaves the block loop
  // can start the next chunk and write its flag before a slower wave has read
  // the flags that ended the loop: the write goes to the other slot, and it can
  // be two reads ahead only after a barrier that the slower wave must reach.
  int32_t* wave_any = reinterpret_cast<int32_t*>(smem + L.any_off);
  int any_rd = 0;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = lane_id(), tid = static_cast<int>(threadIdx.x);
  uint64_t* bufk = reinterpret_cast<uint64_t*>(smem + L.bufk_off) + wave * kBufCap;
  int32_t* bufp = reinterpret_cast<int32_t*>(smem + L.bufp_off) + wave * kBufCap;

  const int64_t q = blockIdx.x;
  const float* __restrict__ qv = a.queries + q * a.dim;
  const int ks = a.ks;
  const int ks_log2 = __ffs(ks) - 1;
  const int K = a.K;
  const int nblocks = (a.pq_m + kBlock - 1) / kBlock;
  // Bytes of one 64-row code tile, and the distance between a lane's rows i, i+1.
  const uint32_t tile_bytes = static_cast<uint32_t>(nblocks) * kTile * kBlock;
  const uint32_t row_step = (kThreads / kTile) * tile_bytes;

  uint64_t lk[KPL];
  int32_t lp[KPL];
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    lk[j] = kNoKey;
    lp[j] = -1;
  }
  uint64_t thr = kNoKey;
  int cnt = 0;
  uint32_t ord_base = 0;
  unsigned long long rows_total = 0, tasks = 0;
  int bad_probe = 0;
  if (lane == 0) wave_thr[wave] = kNoKey;

  // Merges the first min(cnt, 64) buffered candidates into the wave's list and
  // republishes the wave's threshold.
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
    if (lane == 0) wave_thr[wave] = thr;
  };

  for (int p = 0; p < a.P; ++p) {
    int l = a.probes[q * a.P + p];
    if (static_cast<uint32_t>(l) >= static_cast<uint32_t>(a.nlist)) {
      bad_probe = 1;  // reported at the end (the search then fails), never dereferenced
      l = 0;
    }
    const int64_t begin = a.list_offsets[l];
    const int64_t rows = a.list_offsets[l + 1] - begin;
    if (rows <= 0) continue;
    ++tasks;
    rows_total += static_cast<unsigned long long>(rows);

    __syncthreads();  // the previous list no longer reads resid
    const float* __restrict__ cv = a.centroids + static_cast<int64_t>(l) * a.dim;
    for (int t = threadIdx.x; t < a.dim; t += kThreads) resid[t] = qv[t] - cv[t];

    for (int64_t c0 = 0; c0 < rows; c0 += kChunkRows) {
      const int chunk = static_cast<int>(rows - c0 < kChunkRows ? rows - c0 : kChunkRows);
      // Chunk rows are packed positions cpos + r, r = tid + i * kThreads. Their
      // codes are addressed from a uniform base (the chunk's first tile) plus a
      // 32-bit per-lane offset; rows i and i+1 of a lane are 4 tiles apart.
      const int64_t cpos = begin + c0;
      const uint8_t* __restrict__ cbase = a.codes + (cpos >> 6) * tile_bytes;
      const uint32_t lrow = static_cast<uint32_t>(cpos & (kTile - 1)) + static_cast<uint32_t>(tid);
      const uint32_t loff = (lrow >> 6) * tile_bytes + (lrow & (kTile - 1)) * kBlock;
      float s[kRowsPerLane];
      // live[i]: the wave's lanes whose row i is still a shortlist candidate
      // (a wave-uniform lane mask, used directly as the execution mask).
      uint64_t live[kRowsPerLane];
#pragma unroll
      for (int i = 0; i < kRowsPerLane; ++i) {
        s[i] = 0.f;
        const int r = tid + i * kThreads;
        bool ok = r < chunk;
        if (ok && a.bitset) {
          const int64_t id = a.ids[cpos + r];
          ok = ((a.bitset[id >> 3] >> (id & 7)) & 1u) != 0;
        }
        live[i] = __builtin_amdgcn_ballot_w64(ok);
      }
      {
        uint64_t any = 0;
#pragma unroll
        for (int i = 0; i < kRowsPerLane; ++i) any |= live[i];
        if (lane == 0) wave_any[any_rd * kWaves + wave] = any != 0 ? 1 : 0;
      }

      for (int b = 0; b < nblocks; ++b) {
        // Retires the previous block's table slice, publishes the waves' live
        // flags (and resid, for the first block).
        __syncthreads();
        int any = wave_any[any_rd * kWaves];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) any |= wave_any[any_rd * kWaves + w];
        any_rd ^= 1;
        if (!any) break;
        const int mb = FD > 0 ? kBlock : (a.pq_m - b * kBlock < kBlock ? a.pq_m - b * kBlock : kBlock);
        if constexpr (FD > 0) {
          build_slice_256<FD, F16>(resid, a.codebooks, b * kBlock, kBlock, lut32, lut16);
        } else {
        switch (a.dsub) {
          case 1:
            build_slice<1, F16>(resid, a.codebooks, b * kBlock, mb, ks, ks_log2, 1, lut32, lut16);
            break;
          case 2:
            build_slice<2, F16>(resid, a.codebooks, b * kBlock, mb, ks, ks_log2, 2, lut32, lut16);
            break;
          case 4:
            build_slice<4, F16>(resid, a.codebooks, b * kBlock, mb, ks, ks_log2, 4, lut32, lut16);
            break;
          case 8:
            build_slice<8, F16>(resid, a.codebooks, b * kBlock, mb, ks, ks_log2, 8, lut32, lut16);
            break;
          default:
            build_slice<0, F16>(resid, a.codebooks, b * kBlock, mb, ks, ks_log2, a.dsub, lut32,
                                lut16);
        }
        }
        __syncthreads();
        // Prune bound: the smallest K-th key any wave has published. Partial
        // sums are >= +0 (or NaN, never pruned), so comparing floats against the
        // decoded score is the same as comparing order-preserving keys.
        uint64_t tmin = wave_thr[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) tmin = wave_thr[w] < tmin ? wave_thr[w] : tmin;
        const float thr_f = key_score(tmin);
        const uint8_t* __restrict__ bbase = cbase + b * (kTile * kBlock);
        // Recompute the per-row offsets in every block (one 32-bit add each)
        // rather than let them be hoisted out of the block loop as 64-bit
        // addresses held in registers across it.
        uint32_t loff_b = loff;
        asm volatile("" : "+v"(loff_b));
        // Every live row's code word of this block is requested up front (codes
        // that are not L2-resident cost an HBM round trip each).
        constexpr int kD = kRowsPerLane;
        uint2 wq[kD];
#pragma unroll
        for (int d = 0; d < kD; ++d) {
          wq[d] = make_uint2(0u, 0u);
          if (d < kRowsPerLane && __builtin_amdgcn_inverse_ballot_w64(live[d]))
            wq[d] = *reinterpret_cast<const uint2*>(bbase + (loff_b + d * row_step));
        }
#pragma unroll
        for (int i = 0; i < kRowsPerLane; ++i) {
          const uint2 w = wq[i % kD];
          if (i + kD < kRowsPerLane && __builtin_amdgcn_inverse_ballot_w64(live[i + kD]))
            wq[i % kD] = *reinterpret_cast<const uint2*>(bbase + (loff_b + (i + kD) * row_step));
          // Uniform skip; within a live row every lane scores its code word (a
          // dead lane's word is an earlier row's or zero, so its table reads stay
          // in the slice) and only live lanes keep the result.
          if (live[i] == 0) continue;
          const uint32_t wv[2] = {w.x, w.y};
          float acc = s[i];
          if (FD > 0 || (mb == kBlock && ks_log2 == 8)) {
            // All eight table reads are independent: issue them before the
            // left-to-right additions.
            float v[kBlock];
#pragma unroll
            for (int j = 0; j < kBlock; ++j) {
              const int code = static_cast<int>((wv[j >> 2] >> (8 * (j & 3))) & 0xffu);
              v[j] = F16 ? __half2float(__ushort_as_half(lut16[j * 256 + code]))
                         : lut32[j * 256 + code];
            }
#pragma unroll
            for (int j = 0; j < kBlock; ++j) acc = acc + v[j];
          } else if constexpr (FD > 0) {
          } else if (mb == kBlock) {
#pragma unroll
            for (int j = 0; j < kBlock; ++j) {
              const int code = static_cast<int>((wv[j >> 2] >> (8 * (j & 3))) & 0xffu);
              const int idx = (j << ks_log2) + code;
              acc = acc + (F16 ? __half2float(__ushort_as_half(lut16[idx])) : lut32[idx]);
            }
          } else {
            for (int j = 0; j < mb; ++j) {
              const int code = static_cast<int>((wv[j >> 2] >> (8 * (j & 3))) & 0xffu);
              const int idx = (j << ks_log2) + code;
              acc = acc + (F16 ? __half2float(__ushort_as_half(lut16[idx])) : lut32[idx]);
            }
          }
          s[i] = acc;
          live[i] &= __builtin_amdgcn_ballot_w64(!(acc > thr_f));
        }
        // For the next block's read.
        uint64_t any_left = 0;
#pragma unroll
        for (int i = 0; i < kRowsPerLane; ++i) any_left |= live[i];
        if (lane == 0) wave_any[any_rd * kWaves + wave] = any_left != 0 ? 1 : 0;
      }

      // Rows still alive carry their complete score: offer them to the wave's list.
#pragma unroll
      for (int i = 0; i < kRowsPerLane; ++i) {
        if (i * kThreads >= chunk) break;
        if (live[i] == 0) continue;
        const int r = tid + i * kThreads;
        const bool ok = __builtin_amdgcn_inverse_ballot_w64(live[i]);
        const uint64_t key =
            ok ? make_key(s[i], ord_base + static_cast<uint32_t>(c0) + static_cast<uint32_t>(r))
               : kNoKey;
        const bool pass = key < thr;
        const uint64_t bal = __ballot(pass);
        if (bal) {
          const int before = __popcll(bal & ((1ull << lane) - 1ull));
          if (pass) {
            bufk[cnt + before] = key;
            bufp[cnt + before] = static_cast<int32_t>(cpos) + r;
          }
          cnt += __popcll(bal);
          if (cnt >= 64) flush();
        }
      }
      // Fold what is left so the threshold used for pruning stays current: a few
      // keys are inserted one by one, more go through the sort-and-merge.
      if (cnt > 0 && cnt <= 8) {
        for (int t = 0; t < cnt; ++t) insert_one<KPL>(lk, lp, bufk[t], bufp[t]);
        cnt = 0;
        thr = kth_key<KPL>(lk, K);
        if (lane == 0) wave_thr[wave] = thr;
      } else if (cnt > 0) {
        flush();
      }
    }
    ord_base += static_cast<uint32_t>(rows);
  }

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
    for (int o = 32; o >= 1; o >>= 1) valid += __shfl_xor(valid, o, 64);
    if (lane == 0) {
      a.out_count[q] = valid;
      atomicAdd(&a.counters[0], rows_total);
      atomicAdd(&a.counters[1], tasks);
      atomicAdd(&a.counters[2], static_cast<unsigned long long>(valid));
      if (bad_probe) atomicAdd(&a.counters[3], 1ull);
    }
  }
}

// The scan is latency-bound, so shortlists of up to 128 keys run at 8 waves per
// SIMD (64 VGPRs): the row loop fits without spilling and only the rarely taken
// shortlist merge keeps a few values in scratch. Longer register lists keep the
// compiler's own allocation.
template <int KPL, bool F16, int FD>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8))) void k_scan(
    const OvvsScanArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  scan_query<KPL, F16, FD>(a, smem);
}

template <int KPL, bool F16>
__global__ __launch_bounds__(kThreads) void k_scan_long(const OvvsScanArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  scan_query<KPL, F16, 0>(a, smem);
}

template <int KPL, bool F16>
hipError_t launch_scan(const OvvsScanArgs& a, size_t lds, hipStream_t stream) {
  void (*fn)(OvvsScanArgs);
  if constexpr (KPL <= 2) {
    const bool shaped = a.ks == 256 && a.pq_m % kBlock == 0;
    switch (shaped ? a.dsub : 0) {
      case 1: fn = k_scan<KPL, F16, 1>; break;
      case 2: fn = k_scan<KPL, F16, 2>; break;
      case 4: fn = k_scan<KPL, F16, 4>; break;
      case 8: fn = k_scan<KPL, F16, 8>; break;
      default: fn = k_scan<KPL, F16, 0>;
    }
  } else {
    fn = k_scan_long<KPL, F16>;
  }
  if (lds + kLutBytes > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(a.nq)), dim3(kThreads), lds, stream, a);
  return hipGetLastError();
}

int kpl_for(int K) { return K <= 64 ? 1 : K <= 128 ? 2 : K <= 256 ? 4 : K <= 512 ? 8 : 16; }

}  // namespace

extern "C" size_t ovvs_hip_scan_lds_bytes(int32_t pq_m, int32_t ks, int32_t dim,
                                          int32_t lut_f16, int32_t K) {
  if (pq_m <= 0 || ks <= 0 || dim <= 0 || K <= 0 || K > OVVS_HIP_MAX_REFINE) return 0;
  (void)lut_f16;
  const size_t b = scan_layout(dim, kpl_for(K)).total + kLutBytes;
  return b <= 160u * 1024u ? b : 0;
}

extern "C" hipError_t ovvs_hip_scan(const OvvsScanArgs* args, hipStream_t stream) {
  if (!args) return hipErrorInvalidValue;
  const OvvsScanArgs& a = *args;
  if (a.nq <= 0) return hipSuccess;
  if (!a.queries || !a.probes || !a.centroids || !a.codebooks || !a.list_offsets || !a.codes ||
      !a.ids || !a.out_keys || !a.out_pos || !a.out_count || !a.counters || a.nq > 0x7fffffff ||
      a.nlist <= 0 ||
      a.dim <= 0 || a.P <= 0 || a.pq_m <= 0 || a.dsub <= 0 || a.ks < 16 || a.ks > 256 ||
      (a.ks & (a.ks - 1)) != 0 || a.code_blocks != (a.pq_m + kBlock - 1) / kBlock ||
      static_cast<int64_t>(a.pq_m) * a.dsub > a.dim || a.K <= 0 || a.K > OVVS_HIP_MAX_REFINE)
    return hipErrorInvalidValue;
  const int kpl = kpl_for(a.K);
  const size_t lds = scan_layout(a.dim, kpl).total;
  if (lds + kLutBytes > 160u * 1024u) return hipErrorInvalidValue;
  if (a.lut_f16) {
    switch (kpl) {
      case 1: return launch_scan<1, true>(a, lds, stream);
      case 2: return launch_scan<2, true>(a, lds, stream);
      case 4: return launch_scan<4, true>(a, lds, stream);
      case 8: return launch_scan<8, true>(a, lds, stream);
      default: return launch_scan<16, true>(a, lds, stream);
    }
  }
  switch (kpl) {
    case 1: return launch_scan<1, false>(a, lds, stream);
    case 2: return launch_scan<2, false>(a, lds, stream);
    case 4: return launch_scan<4, false>(a, lds, stream);
    case 8: return launch_scan<8, false>(a, lds, stream);
    default: return launch_scan<16, false>(a, lds, stream);
  }
}
