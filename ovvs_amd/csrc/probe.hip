// probe.hip — coarse probe on the matrix cores with fused candidate selection,
// exact re-score and an exact fallback, for IVF-PQ search on gfx950.
//
// The probe set of query q is the first P centroids under the total order on
// (s(q,c), c) with the exact fp32 score s = (|q|^2 + |c|^2) - 2*(q.c), each term a
// left-to-right sum (reference src/neighbors/indexes.cpp:597-606,
// src/prim/mixer.cpp:174-199, src/prim/cpu/cpu_prims.cpp:24-106).
//
// k_probe_mfma, one workgroup of NW wave64s per 16 queries (8; 16 when the batch
// gives fewer workgroups than CUs):
//   operands  mu = the mean of the centroids (per dimension). The queries' and the
//            centroids' centred coordinates fl(x - mu) are rounded to bf16 (round
//            to nearest even); the centroid operands are stored in MFMA fragment
//            order with their centred norms |c'|^2 (left-to-right fp32 sums).
//            Centring makes the bf16 error relative to |q - mu| |c - mu| instead
//            of |q| |c| (data far from the origin, such as [0, 255] coordinates,
//            would otherwise carry a large absolute error).
//   pass 1   v_mfma_f32_16x16x32_bf16 tiles of 16 queries x 16 centroids give the
//            approximate score a'(q,c) = |c'|^2 - 2 (q^ . c^), one bf16 product per
//            element accumulated in fp32; a' approximates s(q,c) minus a constant of
//            the query (|q - mu|^2), which no comparison below needs. The tiles are
//            cut into nch chunks of gt consecutive tiles; group (chunk, column j)
//            holds the centroids 16t + j of the chunk's tiles and each lane keeps the
//            running minimum of a' over its groups; t_q = the P-th smallest of the
//            16 * nch group minima: at least P distinct centroids have a' <= t_q.
//            The minimum over each chunk per query is kept as well.
//   bound    E_q >= |a'(q,c) + |q - mu|^2 - s(q,c)| for every centroid c
//            (candidate_bound): the reference's own rounding of s (sequential sums
//            of n = dim terms, within gamma_n of the real |q - c|^2 terms), the
//            rounding of the centred coordinates and of |c'|^2, the bf16 rounding of
//            both operands (at most (2^-7 + 2^-16) |q'_i c'_i| per product), the
//            matrix core's fp32 accumulation (2^-20 per addition, whatever order or
//            rounding it uses) and flushed subnormals. T_q = t_q + 2 E_q, rounded up.
//   pass 2   every centroid with !(a' > T_q) is a candidate (chunks whose minimum
//            exceeds T_q for all 16 queries are passed over). A centroid outside
//            has s > t_q + |q - mu|^2 + E_q >= s of at least P candidates, so P
//            entries precede it in the exact order: the exact first P are all
//            candidates.
//   pass 3   each candidate is re-scored with the reference's sequential fp32 sums;
//            its rank is the number of candidates with a smaller (s, c) key, and the
//            P of rank < P are the probes in order, bit for bit.
// A query with more candidates than the re-score capacity, or fewer than P (only NaN
// or infinite inputs can cause that), is flagged in `fallback`; k_probe_fallback
// (coarse.hip) then ranks it from exact scores of every centroid.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "device_common.hpp"
#include "kernels.hpp"

using namespace ovvs_dev;

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kRows = 16;                     // queries per workgroup (MFMA M dimension)
constexpr int kMaxChunks = OVVS_PROBE_MAX_GROUPS / 16;

constexpr size_t align16(size_t b) { return (b + 15) & ~static_cast<size_t>(15); }

// Launch shape and LDS carve of one probe launch.
struct ProbeShape {
  int ntile;        // 16-centroid tiles (nlist padded to 16)
  int ks;           // 32-dimension k-steps (dim padded to 32)
  int gt;           // tiles per chunk
  int nch;          // chunks; 16 * nch group slots
  int cap;          // re-score capacity per query
  int dq;           // LDS row stride of the staged queries (dim rounded up to 4)
  int real_groups;  // groups holding at least one real centroid
  size_t mu_off;    // [dq] f32: the centring vector
  size_t a_off;     // [ks][64] uint4: the queries' bf16 operand fragments
  size_t misc_off;  // count [16] | thr [16] | qn [16] | qcn [16] | flag [4]
  size_t chmin_off; // [16][nch] u32: per query, the minimum key of each chunk
  size_t area_off;  // gmin [16][16*nch] u32 during passes 1-2, then slot [16][cap] u64
  size_t lds;       // dynamic LDS bytes
};

struct Carve {
  float* qs;
  float* mu;
  const uint4* aop;
  int32_t* count;
  float* thr;
  float* qn;
  float* qcn;
  int32_t* flag;
  uint32_t* chmin;
  uint32_t* gmin;
  uint64_t* slot;
};

__device__ __forceinline__ Carve carve(unsigned char* base, const ProbeShape& sh) {
  Carve c;
  c.qs = reinterpret_cast<float*>(base);
  c.mu = reinterpret_cast<float*>(base + sh.mu_off);
  c.aop = reinterpret_cast<const uint4*>(base + sh.a_off);
  unsigned char* m = base + sh.misc_off;
  c.count = reinterpret_cast<int32_t*>(m);
  c.thr = reinterpret_cast<float*>(m + kRows * 4);
  c.qn = reinterpret_cast<float*>(m + 2 * kRows * 4);
  c.qcn = reinterpret_cast<float*>(m + 3 * kRows * 4);
  c.flag = reinterpret_cast<int32_t*>(m + 4 * kRows * 4);
  c.chmin = reinterpret_cast<uint32_t*>(base + sh.chmin_off);
  c.gmin = reinterpret_cast<uint32_t*>(base + sh.area_off);
  c.slot = reinterpret_cast<uint64_t*>(base + sh.area_off);
  return c;
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Sum of v over the 64 lanes, in every lane (row shifts within 16 lanes, then row
// broadcasts; all lanes active).
__device__ __forceinline__ int wave_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return __builtin_amdgcn_readlane(v, 63);
}

// bf16 bits of x, rounded to nearest even (NaN stays NaN).
__host__ __device__ __forceinline__ uint16_t bf16_bits(uint32_t u) {
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 w) {
  bf16x8 v;
  __builtin_memcpy(&v, &w, sizeof(v));
  return v;
}

// Score of a 32-bit order key (the inverse of score_key); the NaN key gives +inf.
__device__ __forceinline__ float key_to_score(uint32_t k) {
  if (k == 0xffffffffu) return __builtin_inff();
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// The next float above a finite f.
__device__ __forceinline__ float next_up(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) == 0) return __uint_as_float(1u);
  return __uint_as_float((u & 0x80000000u) ? u - 1u : u + 1u);
}

// Left-to-right fp32 sum from +0 of x[t]^2 (kCentred: of (x[t] - m[t])^2), t < d, for
// rows in LDS that start 16-byte aligned: eight 16-byte reads issued before their
// terms are added (the sum's order is unchanged).
template <bool kCentred>
__device__ __forceinline__ float lds_seq_sumsq(const float* x, const float* m, int d) {
  const float4* x4 = reinterpret_cast<const float4*>(x);
  const float4* m4 = reinterpret_cast<const float4*>(m);
  const int n4 = d >> 2;
  float s = 0.f;
  auto add4 = [&](float4 v, float4 w) {
    const float e0 = kCentred ? v.x - w.x : v.x, e1 = kCentred ? v.y - w.y : v.y;
    const float e2 = kCentred ? v.z - w.z : v.z, e3 = kCentred ? v.w - w.w : v.w;
    s = s + e0 * e0;
    s = s + e1 * e1;
    s = s + e2 * e2;
    s = s + e3 * e3;
  };
  int i = 0;
  for (; i + 8 <= n4; i += 8) {
    float4 v[8], w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[j] = x4[i + j];
      w[j] = kCentred ? m4[i + j] : v[j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) add4(v[j], w[j]);
  }
  for (; i < n4; ++i) add4(x4[i], kCentred ? m4[i] : x4[i]);
  for (int t = 4 * n4; t < d; ++t) {
    const float e = kCentred ? x[t] - m[t] : x[t];
    s = s + e * e;
  }
  return s;
}

// Candidate bound T = t + 2E for one query, rounded up (see the file comment).
// qn: the query's exact squared norm (sequential fp32 sum), qcn: the sequential
// fp32 sum of its squared centred coordinates, cn_max / ccn_max: the largest of the
// centroids' exact and centred squared norms. u = 2^-23 covers any rounding mode.
__device__ float candidate_bound(float t, float qn, float qcn, float cn_max, float ccn_max, int dim,
                                 int ksteps) {
  if (!(t < __builtin_inff()) || !(qn < __builtin_inff()) || !(qcn < __builtin_inff()) ||
      !(cn_max < __builtin_inff()) || !(ccn_max < __builtin_inff()))
    return __builtin_inff();
  const double u = 1.1920928955078125e-7;   // 2^-23
  const double um = 9.5367431640625e-7;     // 2^-20, per matrix-core addition
  const double n = static_cast<double>(dim) + 4.0;
  const double g = n * u / (1.0 - n * u);
  // The reference's score s against the real |q - c|^2: qd, cd bound |q|^2, |c|^2.
  const double qd = static_cast<double>(qn) * (1.0 + 4.0 * n * u);
  const double cd = static_cast<double>(cn_max) * (1.0 + 4.0 * n * u);
  const double S = sqrt(qd * cd) * (1.0 + 1e-6);
  const double e2 = (g + 3.0 * u) * (qd + cd) + 2.0 * (g + u) * S + u * (qd + cd + 2.0 * S);
  // a' against the real |c'|^2 - 2 q'.c': qc, cc bound |q - mu|^2, |c - mu|^2.
  const double qc = static_cast<double>(qcn) * (1.0 + 4.0 * n * u);
  const double cc = static_cast<double>(ccn_max) * (1.0 + 4.0 * n * u);
  const double Sc = sqrt(qc * cc) * (1.0 + 1e-6);
  const double m = 33.0 * ksteps + 8.0;
  const double gm = m * um / (1.0 - m * um);
  const double ep = 0.0078125 + 1.52587890625e-5 + 3.0 * u;  // 2^-7 + 2^-16 per product
  const double e1 = (g + 5.0 * u) * cc + 2.0 * (ep + 1.02 * gm + 1.02 * u) * Sc +
                    m * 1e-30 * (1.0 + sqrt(qc) + sqrt(cc) + sqrt(qd) + sqrt(cd));
  const double E = 1.01 * (e1 + e2);
  const double T = static_cast<double>(t) + 2.0 * E;
  float f = static_cast<float>(T);
  if (static_cast<double>(f) < T && f < __builtin_inff()) f = next_up(f);
  return f;
}

// Tiles per operand batch (every batch requests the B fragments of its tiles and
// their centred norms before its matrix-core products), and 16-byte vectors per round
// trip of the exact re-score. The wide instance (shapes whose LDS admits one
// workgroup per CU: sixteen waves, four per SIMD, up to 128 registers each) keeps
// twice the vectors in flight, and with operands in registers twice the tiles (the
// LDS-operand shapes already request a k-step ahead).
template <int KS, bool WIDE>
constexpr int batch_tiles() {
  return WIDE && KS > 0 ? 8 : 4;
}
template <bool WIDE>
constexpr int rescore_chunk() {
  return WIDE ? 24 : 12;
}

// KS in 1..4: the queries' operand fragments are held in registers (dim <= 128);
// KS = 0: any number of k-steps, fragments read from LDS per k-step, the next
// k-step's B fragments requested before the current products.
// Six waves per SIMD (at most 80 VGPRs) for the register-operand shapes: with three
// workgroups of eight waves per CU (their LDS allows it up to dim 128 and 256
// candidates), a 10k-query batch's 625 workgroups run in one round on 256 CUs instead
// of 1.2. The LDS-operand shapes keep the compiler's allocation (their LDS allows one
// workgroup per CU); the wide instance (sixteen waves) allows four waves per SIMD.
template <int KS, int NW, bool WIDE>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WIDE ? 4 : KS > 0 ? 6 : 1))) void k_probe_mfma(
    const OvvsProbeArgs p, const ProbeShape shape) {
  constexpr int kWaves = NW;
  constexpr int kThreads = 64 * NW;
  constexpr int kRowsPerWave = kRows / kWaves;  // rows each wave selects and ranks
  constexpr int kG = batch_tiles<KS, WIDE>();
  extern __shared__ __align__(16) unsigned char smem[];
  const Carve L = carve(smem, shape);
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t q0 = static_cast<int64_t>(blockIdx.x) * kRows;
  const int dim = p.dim, dq = shape.dq, ks = shape.ks, nch = shape.nch;
  if (p.stamp && blockIdx.x == 0 && threadIdx.x == 0) *p.stamp = wall_clock64();

  // Stage the 16 query rows (zero past dim and past nq).
  for (int i = static_cast<int>(threadIdx.x); i < kRows * dq; i += kThreads) {
    const int r = i / dq, t = i - r * dq;
    const int64_t q = q0 + r;
    L.qs[i] = (q < p.nq && t < dim) ? p.queries[q * dim + t] : 0.f;
  }
  for (int t = static_cast<int>(threadIdx.x); t < dim; t += kThreads) L.mu[t] = p.cmu[t];
  if (threadIdx.x < kRows) L.count[threadIdx.x] = 0;
  if (threadIdx.x == 0) L.flag[0] = 0;
  if (p.zero && blockIdx.x == 0 && threadIdx.x < 8) p.zero[threadIdx.x] = 0;
  __syncthreads();
  // Query norms (given, or the sequential sums of squares of the staged rows), the
  // centred sums, and the bf16 operand fragments of fl(q - mu): lane l of k-step s
  // holds A[l % 16][32 s + 8 (l / 16) + j], j = 0..7.
  if (threadIdx.x < kRows) {
    const int64_t q = q0 + threadIdx.x;
    const float* r = L.qs + threadIdx.x * dq;
    float s = 0.f;
    if (p.qnorm) {
      s = q < p.nq ? p.qnorm[q] : 0.f;
    } else {
      s = lds_seq_sumsq<false>(r, r, dim);
      if (q < p.nq) p.qnorm_out[q] = s;
    }
    const float sc = lds_seq_sumsq<true>(r, L.mu, dim);
    L.qn[threadIdx.x] = q < p.nq ? s : 0.f;
    L.qcn[threadIdx.x] = q < p.nq ? sc : 0.f;
  }
  {
    uint4* aop = reinterpret_cast<uint4*>(smem + shape.a_off);
    for (int i = static_cast<int>(threadIdx.x); i < ks * 64; i += kThreads) {
      const int s = i >> 6, l = i & 63, row = l & 15;
      const bool live = q0 + row < p.nq;
      uint16_t h[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = 32 * s + 8 * (l >> 4) + j;
        const float x = (live && k < dim) ? L.qs[row * dq + k] - L.mu[k] : 0.f;
        h[j] = bf16_bits(__float_as_uint(x));
      }
      uint4 w;
      __builtin_memcpy(&w, h, sizeof(w));
      aop[i] = w;
    }
  }
  __syncthreads();

  bf16x8 ah[KS > 0 ? KS : 1];
  if constexpr (KS > 0) {
#pragma unroll
    for (int s = 0; s < KS; ++s) ah[s] = as_bf16x8(L.aop[s * 64 + lane]);
  }
  const int col = lane & 15;
  const uint4* __restrict__ bops = reinterpret_cast<const uint4*>(p.cmfma) + lane;
  // Dot products of the kG tiles t0 + g (tiles at or past tend repeat tile t0 and
  // are ignored by the caller), and the centred norm of each lane's centroid.
  auto batch = [&](int t0, int tend, f32x4 (&acc)[kG], float (&cn)[kG]) {
    int tt[kG];
#pragma unroll
    for (int g = 0; g < kG; ++g) {
      tt[g] = t0 + g < tend ? t0 + g : t0;
      acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int c = 16 * tt[g] + col;
      cn[g] = c < p.nlist ? p.cnc[c] : 0.f;
    }
    if constexpr (KS > 0) {
      uint4 b[kG][KS];
#pragma unroll
      for (int g = 0; g < kG; ++g)
#pragma unroll
        for (int s = 0; s < KS; ++s) b[g][s] = bops[(static_cast<int64_t>(tt[g]) * KS + s) * 64];
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int g = 0; g < kG; ++g)
          acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[s], as_bf16x8(b[g][s]), acc[g], 0, 0, 0);
    } else {
      uint4 cur[kG], nxt[kG];
#pragma unroll
      for (int g = 0; g < kG; ++g) cur[g] = bops[static_cast<int64_t>(tt[g]) * ks * 64];
      for (int s = 0; s < ks; ++s) {
        if (s + 1 < ks) {
#pragma unroll
          for (int g = 0; g < kG; ++g) nxt[g] = bops[(static_cast<int64_t>(tt[g]) * ks + s + 1) * 64];
        }
        const bf16x8 a = as_bf16x8(L.aop[s * 64 + lane]);
#pragma unroll
        for (int g = 0; g < kG; ++g)
          acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, as_bf16x8(cur[g]), acc[g], 0, 0, 0);
#pragma unroll
        for (int g = 0; g < kG; ++g) cur[g] = nxt[g];
      }
    }
  };

  // A wave takes the chunks wave, wave + kWaves, ..., starting at a rotation that
  // differs between neighbouring workgroups of an XCD (blockIdx.x / 8), so that they
  // do not all miss in L2 on the same tiles at the same time. Operand copies larger
  // than 8 MB (1 KB per tile and k-step) do not fit an XCD's L2: there the
  // workgroups keep one order and share what the L2 holds of their current chunks
  // (C5's 12 MB probe measured 3% faster so, C2's and C3's 4-5% slower).
  const int nmine = (nch - wave + kWaves - 1) / kWaves;
  const bool rotate = static_cast<int64_t>(shape.ntile) * ks <= 8192;
  const int rot = rotate && nmine > 0 ? static_cast<int>((blockIdx.x >> 3) % static_cast<uint32_t>(nmine)) : 0;
  auto chunk_of = [&](int i) {
    const int j = i + rot;
    return wave + kWaves * (j >= nmine ? j - nmine : j);
  };

  // Pass 1: running minimum of a' over each (chunk, column) group, and of each
  // query row over the chunk. A NaN score (only non-finite inputs make one) turns
  // chunk skipping off for the workgroup.
  const int ng = 16 * nch;
  bool bad = false;
  for (int i = 0; i < nmine; ++i) {
    const int ch = chunk_of(i);
    const int t0 = ch * shape.gt;
    const int t1 = min(t0 + shape.gt, shape.ntile);
    float m[4] = {__builtin_inff(), __builtin_inff(), __builtin_inff(), __builtin_inff()};
    for (int t = t0; t < t1; t += kG) {
      f32x4 acc[kG];
      float cn[kG];
      batch(t, t1, acc, cn);
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        if (t + g < t1 && 16 * (t + g) + col < p.nlist) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float a = cn[g] - 2.f * acc[g][r];
          bad |= a != a;
          m[r] = __builtin_fminf(m[r], a);
        }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * (lane >> 4) + r;
      L.gmin[row * ng + ch * 16 + col] = score_key(m[r]);
      float v = m[r];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) v = __builtin_fminf(v, __shfl_xor(v, o, 64));
      if (col == 0) L.chmin[row * nch + ch] = score_key(v);
    }
  }
  if (__builtin_amdgcn_ballot_w64(bad) != 0 && lane == 0) atomicOr(&L.flag[0], 1);
  __syncthreads();

  // The P-th smallest group minimum of each row, bit by bit from the top: v is the
  // smallest key with at least P group minima <= v. Each lane holds its slots; the
  // wave's rows are searched together (independent compare/count chains).
  {
    uint32_t g[kRowsPerWave][kMaxChunks / 4];
    uint32_t v[kRowsPerWave];
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr) {
      const int row = kRowsPerWave * wave + rr;
#pragma unroll
      for (int i = 0; i < kMaxChunks / 4; ++i) {
        const int s = lane + 64 * i;
        g[rr][i] = s < ng ? L.gmin[row * ng + s] : 0xffffffffu;
      }
      v[rr] = 0;
    }
    // Counts in the VALU (per-lane sums, then a DPP sum): every wave of the CU runs
    // this loop at once, and ballot/popcount counting would queue on the scalar unit.
    for (int b = 31; b >= 0; --b) {
      int cnt[kRowsPerWave];
#pragma unroll
      for (int rr = 0; rr < kRowsPerWave; ++rr) {
        const uint32_t probe = v[rr] | ((1u << b) - 1u);
        int c = 0;
#pragma unroll
        for (int i = 0; i < kMaxChunks / 4; ++i) c += g[rr][i] <= probe ? 1 : 0;
        cnt[rr] = wave_sum(c);
      }
#pragma unroll
      for (int rr = 0; rr < kRowsPerWave; ++rr)
        if (cnt[rr] < p.P) v[rr] |= 1u << b;
    }
    if (lane == 0) {
#pragma unroll
      for (int rr = 0; rr < kRowsPerWave; ++rr) {
        const int row = kRowsPerWave * wave + rr;
        const int64_t q = q0 + row;
        const bool live = q < p.nq;
        L.thr[row] = candidate_bound(key_to_score(v[rr]), live ? L.qn[row] : 0.f,
                                     live ? L.qcn[row] : 0.f, p.cnorm_max, p.cnc_max, dim, ks);
      }
    }
  }
  __syncthreads();

  // Pass 2: every centroid whose approximate score is not above the bound; a chunk
  // whose minimum exceeds the bound for all 16 rows holds none.
  float T[4];
  uint32_t kT[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    T[r] = L.thr[4 * (lane >> 4) + r];
    kT[r] = score_key(T[r]);
  }
  const bool may_skip = L.flag[0] == 0;
  const int cap = shape.cap;
  for (int i = 0; i < nmine; ++i) {
    const int ch = chunk_of(i);
    if (may_skip) {
      bool hit = false;
#pragma unroll
      for (int r = 0; r < 4; ++r) hit |= L.chmin[(4 * (lane >> 4) + r) * nch + ch] <= kT[r];
      if (__builtin_amdgcn_ballot_w64(hit) == 0) continue;
    }
    const int t0 = ch * shape.gt;
    const int t1 = min(t0 + shape.gt, shape.ntile);
    for (int t = t0; t < t1; t += kG) {
      f32x4 acc[kG];
      float cn[kG];
      batch(t, t1, acc, cn);
      // Per tile, bit r: the lane's centroid is a candidate of its row r; the
      // candidates are appended one per lane and step.
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        const int c = 16 * (t + g) + col;
        uint32_t hits = 0;
        if (t + g < t1 && c < p.nlist) {
#pragma unroll
          for (int r = 0; r < 4; ++r) hits |= !(cn[g] - 2.f * acc[g][r] > T[r]) ? 1u << r : 0u;
        }
        while (hits) {
          const int row = 4 * (lane >> 4) + __builtin_ctz(hits);
          hits &= hits - 1u;
          const int at = atomicAdd(&L.count[row], 1);
          if (at < cap) L.slot[row * cap + at] = static_cast<uint64_t>(c);
        }
      }
    }
  }
  __syncthreads();

  // Pass 3: exact keys of the candidates of this wave's rows, then ranks by counting.
  int cnt[kRowsPerWave], pre[kRowsPerWave + 1];
  pre[0] = 0;
#pragma unroll
  for (int rr = 0; rr < kRowsPerWave; ++rr) {
    const int row = kRowsPerWave * wave + rr;
    const int64_t q = q0 + row;
    const int c = L.count[row];
    const bool ok = q < p.nq && c >= p.P && c <= cap;
    cnt[rr] = ok ? c : 0;
    pre[rr + 1] = pre[rr] + cnt[rr];
    if (q < p.nq && lane == 0) {
      p.fallback[q] = ok ? 0 : 1;
      if (!ok && p.order_keys) p.order_keys[q] = 0;
    }
  }
  const int total = pre[kRowsPerWave];
  for (int f = lane; f < total; f += 64) {
    int rr = 0;
#pragma unroll
    for (int j = 1; j < kRowsPerWave; ++j) rr += f >= pre[j] ? 1 : 0;
    const int row = kRowsPerWave * wave + rr;
    uint64_t* s = L.slot + row * cap + (f - pre[rr]);
    const uint32_t c = static_cast<uint32_t>(*s);
    const float* crow = p.centroids + static_cast<int64_t>(c) * dim;
    const float* qrow = L.qs + row * dq;
    const float dot =
        (dim & 3) == 0 ? seq_dot_v4_chunked<rescore_chunk<WIDE>()>(qrow, crow, dim) : seq_dot(qrow, crow, dim);
    *s = make_key((L.qn[row] + p.cnorm[c]) - 2.f * dot, c);
  }
  wave_sync();
  // Ranks. A row of at most kCountRank candidates: each candidate's rank is the number
  // of smaller keys. A longer row: its keys in registers, the P-th smallest key by a
  // bit search (keys are distinct: exactly P keys are at most it), those P keys moved
  // to the front of the row in position order, then ranked among themselves.
  constexpr int kCountRank = 256;
  constexpr int kKeysPerLane = OVVS_PROBE_CAP / 64;
#pragma unroll
  for (int rr = 0; rr < kRowsPerWave; ++rr) {
    const int row = kRowsPerWave * wave + rr;
    uint64_t* keys = L.slot + row * cap;
    int n = cnt[rr];
    if (n > kCountRank) {
      uint64_t k[kKeysPerLane];
#pragma unroll
      for (int i = 0; i < kKeysPerLane; ++i) {
        const int f = lane + 64 * i;
        k[i] = f < n ? keys[f] : ~0ull;
      }
      uint64_t v = 0;
      for (int b = 63; b >= 0; --b) {
        const uint64_t probe = v | ((1ull << b) - 1ull);
        int c = 0;
#pragma unroll
        for (int i = 0; i < kKeysPerLane; ++i) c += __popcll(__ballot(k[i] <= probe));
        if (c < p.P) v |= 1ull << b;
      }
      wave_sync();
      int base = 0;
#pragma unroll
      for (int i = 0; i < kKeysPerLane; ++i) {
        const bool keep = k[i] <= v;
        const uint64_t bal = __ballot(keep);
        if (keep) keys[base + __popcll(bal & ((1ull << lane) - 1ull))] = k[i];
        base += __popcll(bal);
      }
      wave_sync();
      n = p.P;
    }
    for (int f = lane; f < n; f += 64) {
      const uint64_t key = keys[f];
      int rank = 0;
      int j = 0;
      // Eight keys per step, read 16 bytes at a time (the row starts 16-byte aligned).
      for (; j + 8 <= n; j += 8) {
        uint64_t kk[8];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint4 w = reinterpret_cast<const uint4*>(keys + j)[u];
          kk[2 * u] = (static_cast<uint64_t>(w.y) << 32) | w.x;
          kk[2 * u + 1] = (static_cast<uint64_t>(w.w) << 32) | w.z;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) rank += kk[u] < key ? 1 : 0;
      }
      for (; j < n; ++j) rank += keys[j] < key ? 1 : 0;
      if (rank < p.P) p.probes[(q0 + row) * p.P + rank] = static_cast<int32_t>(key & 0xffffffffu);
      if (rank == 0 && p.order_keys) p.order_keys[q0 + row] = p.list_rank[key & 0xffffffffu] >> p.key_shift;
    }
  }
}

// Shape of a launch, or false when the fused probe does not serve these sizes.
bool probe_shape(int32_t dim, int32_t nlist, int32_t P, ProbeShape* sh) {
  if (dim <= 0 || dim > 32 * OVVS_PROBE_MAX_KSTEPS || nlist <= 0 || nlist > (1 << 24) || P <= 0 ||
      P > OVVS_PROBE_MAX_P)
    return false;
  sh->ntile = (nlist + 15) / 16;
  sh->ks = (dim + 31) / 32;
  sh->gt = (sh->ntile + kMaxChunks - 1) / kMaxChunks;
  sh->nch = (sh->ntile + sh->gt - 1) / sh->gt;
  int real = 0;
  for (int ch = 0; ch < sh->nch; ++ch) real += min(16, nlist - 16 * ch * sh->gt);
  sh->real_groups = real;
  if (2 * P > real) return false;
  // Re-score capacity: about four times P (the candidates are the P-th group
  // minimum's centroids plus the bound's window), 512 when 1024 would not fit.
  sh->cap = P <= 64 ? 256 : P <= 128 ? 512 : OVVS_PROBE_CAP;
  sh->dq = (dim + 3) & ~3;
  sh->mu_off = align16(static_cast<size_t>(kRows) * sh->dq * 4);
  sh->a_off = sh->mu_off + align16(static_cast<size_t>(sh->dq) * 4);
  sh->misc_off = sh->a_off + static_cast<size_t>(sh->ks) * 64 * 16;
  sh->chmin_off = sh->misc_off + align16(4 * kRows * 4 + 16);
  sh->area_off = sh->chmin_off + align16(static_cast<size_t>(kRows) * sh->nch * 4);
  const size_t gmin = static_cast<size_t>(kRows) * 16 * sh->nch * 4;
  for (;;) {
    const size_t slot = static_cast<size_t>(kRows) * sh->cap * 8;
    sh->lds = sh->area_off + (gmin > slot ? gmin : slot);
    if (sh->lds <= 160 * 1024 || sh->cap <= 512) break;
    sh->cap = 512;
  }
  // 2P + 32 slots (at least 256) when that lets three workgroups share a CU and the
  // capacity above does not: a 10k batch's 625 workgroups then run in one round on
  // 256 CUs instead of two (C3, P 128: 218 candidates per query at the median, 272 at
  // most; the probe took 0.73 ms with 512 slots). A query with more candidates takes
  // the exact fallback.
  {
    const int cap3 = std::max(256, (2 * P + 32 + 31) & ~31);
    const size_t slot3 = static_cast<size_t>(kRows) * cap3 * 8;
    const size_t lds3 = sh->area_off + (gmin > slot3 ? gmin : slot3);
    if (cap3 < sh->cap && 3 * sh->lds > 160 * 1024 && 3 * lds3 <= 160 * 1024) {
      sh->cap = cap3;
      sh->lds = lds3;
    }
  }
  return sh->lds <= 160 * 1024;
}

template <int KS, int NW, bool WIDE>
hipError_t launch_probe_nw(const OvvsProbeArgs& p, const ProbeShape& sh, hipStream_t stream) {
  if (sh.lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_probe_mfma<KS, NW, WIDE>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(sh.lds));
    if (e != hipSuccess) return e;
  }
  const int64_t blocks = (p.nq + kRows - 1) / kRows;
  hipLaunchKernelGGL((k_probe_mfma<KS, NW, WIDE>), dim3(static_cast<uint32_t>(blocks)), dim3(64 * NW),
                     sh.lds, stream, p, sh);
  return hipGetLastError();
}

// 16 waves per workgroup when the batch gives fewer workgroups than the 256 CUs
// (small batches: the latency of one workgroup is the launch) or when the LDS of two
// workgroups does not fit a CU (the wide instance where its batches fit the chunks:
// C5's probe took 2.04 ms with eight waves of up to 256 registers, 1.54 with sixteen
// of 80 and 1.35 with sixteen of 128; C4's 0.61, 0.59 and 0.58), else 8.
template <int KS>
hipError_t launch_probe(const OvvsProbeArgs& p, const ProbeShape& sh, hipStream_t stream) {
  if ((p.nq + kRows - 1) / kRows < 256) return launch_probe_nw<KS, 16, false>(p, sh, stream);
  if (2 * sh.lds > 160 * 1024) {
    if (sh.gt >= batch_tiles<KS, true>()) return launch_probe_nw<KS, 16, true>(p, sh, stream);
    return launch_probe_nw<KS, 16, false>(p, sh, stream);
  }
  return launch_probe_nw<KS, 8, false>(p, sh, stream);
}

}  // namespace

extern "C" int ovvs_hip_probe_mfma_supported(int32_t dim, int32_t nlist, int32_t P) {
  ProbeShape sh;
  return probe_shape(dim, nlist, P, &sh) ? 1 : 0;
}

extern "C" size_t ovvs_hip_probe_cmfma_words(int32_t dim, int32_t nlist) {
  if (dim <= 0 || dim > 32 * OVVS_PROBE_MAX_KSTEPS || nlist <= 0) return 0;
  const size_t ks = static_cast<size_t>((dim + 31) / 32);
  return static_cast<size_t>((nlist + 15) / 16) * ks * 64 * 4;
}

extern "C" void ovvs_probe_prepare(const float* C, int32_t nlist, int32_t dim, uint32_t* ops,
                                   float* mu, float* cnc, float* cnc_max) {
  const int ks = (dim + 31) / 32, ntile = (nlist + 15) / 16;
  for (int t = 0; t < dim; ++t) {
    double s = 0.0;
    for (int c = 0; c < nlist; ++c) s += static_cast<double>(C[static_cast<size_t>(c) * dim + t]);
    mu[t] = static_cast<float>(s / static_cast<double>(nlist));
  }
  float mx = 0.f;
  for (int c = 0; c < nlist; ++c) {
    float s = 0.f;
    for (int t = 0; t < dim; ++t) {
      const float d = C[static_cast<size_t>(c) * dim + t] - mu[t];
      s = s + d * d;
    }
    cnc[c] = s;
    if (!(s <= mx)) mx = std::isfinite(s) ? s : INFINITY;
    if (std::isinf(mx)) {
      for (int r = c + 1; r < nlist; ++r) cnc[r] = INFINITY;
      break;
    }
  }
  *cnc_max = mx;
  for (int t = 0; t < ntile; ++t)
    for (int s = 0; s < ks; ++s)
      for (int lane = 0; lane < 64; ++lane) {
        uint16_t h[8];
        for (int j = 0; j < 8; ++j) {
          const int k = 32 * s + 8 * (lane / 16) + j, c = 16 * t + lane % 16;
          const float x = (c < nlist && k < dim) ? C[static_cast<size_t>(c) * dim + k] - mu[k] : 0.f;
          uint32_t u;
          std::memcpy(&u, &x, 4);
          h[j] = bf16_bits(u);
        }
        uint32_t* d = ops + ((static_cast<size_t>(t) * ks + s) * 64 + lane) * 4;
        for (int w = 0; w < 4; ++w)
          d[w] = static_cast<uint32_t>(h[2 * w]) | (static_cast<uint32_t>(h[2 * w + 1]) << 16);
      }
}

extern "C" hipError_t ovvs_hip_probe_mfma(const OvvsProbeArgs* args, hipStream_t stream) {
  if (!args) return hipErrorInvalidValue;
  const OvvsProbeArgs& p = *args;
  if (p.nq <= 0) return hipSuccess;
  ProbeShape sh;
  if (!p.queries || (!p.qnorm && !p.qnorm_out) || !p.centroids || !p.cmfma || !p.cnorm || !p.cmu ||
      !p.cnc || !p.probes || !p.fallback || p.nq > 0x7fffffff || !probe_shape(p.dim, p.nlist, p.P, &sh))
    return hipErrorInvalidValue;
  switch (sh.ks) {
    case 1: return launch_probe<1>(p, sh, stream);
    case 2: return launch_probe<2>(p, sh, stream);
    case 3: return launch_probe<3>(p, sh, stream);
    case 4: return launch_probe<4>(p, sh, stream);
    default: return launch_probe<0>(p, sh, stream);
  }
}
