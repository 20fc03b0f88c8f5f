// probe.hip — coarse probe on the fp32 matrix cores with fused candidate selection,
// exact re-score and an exact fallback, for IVF-PQ search on gfx950.
//
// The probe set of query q is the first P centroids under the total order on
// (s(q,c), c) with the exact fp32 score s = (|q|^2 + |c|^2) - 2*(q.c), each term a
// left-to-right sum (reference src/neighbors/indexes.cpp:597-606,
// src/prim/mixer.cpp:174-199, src/prim/cpu/cpu_prims.cpp:24-106).
//
// k_probe_mfma, one workgroup of NW wave64s per 16 queries (8; 16 when the batch
// gives fewer workgroups than CUs, so that each wave's tile chain is half as long):
//   pass 1   v_mfma_f32_16x16x32_bf16 tiles of 16 queries x 16 centroids give
//            approximate scores a(q,c) from split operands: every fp32 value x is
//            x_hi + x_lo with x_hi = bf16(x), x_lo = bf16(x - x_hi) (round to nearest
//            even; x - x_hi is exact), and q.c ~ q_hi.c_hi + q_hi.c_lo + q_lo.c_hi,
//            three bf16 products per element accumulated in fp32. The tiles are cut
//            into nch chunks of gt consecutive tiles;
//            group (chunk, column j) holds the centroids 16t + j of the chunk's tiles,
//            and each lane keeps the running minimum of a over its group in registers.
//            v_q is the P-th smallest of the 16 * nch group minima (as order keys): at
//            least P distinct centroids (one per group) have a <= t_q, the score v_q
//            encodes.
//   bound    E_q >= |a(q,c) - s(q,c)| for every centroid c. The reference's sequential
//            dot is within gamma_n |q||c| of the real one (n = dim + 4, u = 2^-23).
//            The split dot drops q_lo c_lo and the split remainders, at most
//            3.05 * 2^-16 |q_i c_i| per element, and accumulates 3 * 32 * ksteps exact
//            bf16 products plus the accumulator in fp32; each addition is allowed 8x
//            the fp32 unit roundoff (2^-20) whatever order or rounding the matrix
//            core uses, plus an absolute term for flushed subnormals. The shared
//            |q|^2 + |c|^2 term is rounded once more in both.
//   pass 2   every centroid with !(a > T_q), T_q = t_q + 2 E_q rounded up, is a
//            candidate. A centroid outside has s > t_q + E_q >= s of at least P
//            candidates, so P entries precede it in the exact order: the exact first
//            P are all candidates.
//   pass 3   each candidate is re-scored with the reference's sequential fp32 sums;
//            its rank is the number of candidates with a smaller (s, c) key, and the
//            P of rank < P are the probes in order, bit for bit.
// A query with more candidates than the re-score capacity, or fewer than P (only NaN
// or infinite inputs can cause that), is flagged in `fallback`; k_probe_fallback
// (coarse.hip) then ranks it from exact scores of every centroid.
#include <cstring>

#include "device_common.hpp"
#include "kernels.hpp"

using namespace ovvs_dev;

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));


constexpr int kRows = 16;                     // queries per workgroup (MFMA M dimension)
constexpr int kMaxChunks = OVVS_PROBE_MAX_GROUPS / 16;

// Launch shape and LDS carve of one probe launch.
struct ProbeShape {
  int ntile;   // 16-centroid tiles (nlist padded to 16)
  int gt;      // tiles per chunk
  int nch;     // chunks; 16 * nch group slots
  int cap;     // re-score capacity per query
  int dq;      // LDS row stride of the staged queries (dim rounded up to 4)
  int real_groups;  // groups holding at least one real centroid
  size_t lds;  // dynamic LDS bytes
};

constexpr size_t align16(size_t b) { return (b + 15) & ~static_cast<size_t>(15); }

// LDS: qs [16][dq] f32 | count [16] i32 | thr [16] f32 | qn [16] f32 | area: gmin
// [16][16*nch] u32 during passes 1-2, then slot [16][cap] u64 (candidate id, later its
// exact key).
struct Carve {
  float* qs;
  int32_t* count;
  float* thr;
  float* qn;
  uint32_t* gmin;
  uint64_t* slot;
};

__device__ __forceinline__ Carve carve(unsigned char* base, const ProbeShape& sh) {
  Carve c;
  c.qs = reinterpret_cast<float*>(base);
  unsigned char* p = base + align16(static_cast<size_t>(kRows) * sh.dq * 4);
  c.count = reinterpret_cast<int32_t*>(p);
  c.thr = reinterpret_cast<float*>(p + kRows * 4);
  c.qn = reinterpret_cast<float*>(p + 2 * kRows * 4);
  p += align16(3 * kRows * 4);
  c.gmin = reinterpret_cast<uint32_t*>(p);
  c.slot = reinterpret_cast<uint64_t*>(p);
  return c;
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// bf16 bits of x, rounded to nearest even (NaN stays NaN).
__host__ __device__ __forceinline__ uint16_t bf16_bits(uint32_t u) {
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// The split of x: hi = bf16(x), lo = bf16(x - hi).
__device__ __forceinline__ void split_bf16(float x, uint16_t& hi, uint16_t& lo) {
  hi = bf16_bits(__float_as_uint(x));
  const float r = x - __uint_as_float(static_cast<uint32_t>(hi) << 16);
  lo = bf16_bits(__float_as_uint(r));
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 w) {
  bf16x8 v;
  __builtin_memcpy(&v, &w, sizeof(v));
  return v;
}

// Approximate dot products of tile t: lane holds rows 4*(lane/16)+r, column lane%16.
// Operand lane layout of v_mfma_f32_16x16x32_bf16: lane l holds A[l%16][8(l/16)+j]
// and B[8(l/16)+j][l%16], j = 0..7, per 32-deep k-step. The centroid operands come
// from the split copy (OvvsProbeArgs::cmfma): per tile and k-step, 64 lanes x 16 B
// of high parts, then 64 lanes x 16 B of low parts.
template <int KS>
__device__ __forceinline__ f32x4 tile_dot(const bf16x8 (&ah)[KS], const bf16x8 (&al)[KS],
                                          const uint32_t* __restrict__ cm, int t) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const uint4* src =
      reinterpret_cast<const uint4*>(cm) + static_cast<int64_t>(t) * KS * 2 * 64 + lane_id();
  uint4 bh[KS], bl[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    bh[s] = src[(2 * s) * 64];
    bl[s] = src[(2 * s + 1) * 64];
  }
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const bf16x8 h = as_bf16x8(bh[s]), l = as_bf16x8(bl[s]);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[s], h, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[s], l, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[s], h, acc, 0, 0, 0);
  }
  return acc;
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

// Candidate bound T = t + 2E for one query (see the file comment), rounded up.
__device__ float candidate_bound(float t, float qn, float cn_max, int dim, int ksteps) {
  if (!(t < __builtin_inff()) || !(qn < __builtin_inff()) || !(cn_max < __builtin_inff()))
    return __builtin_inff();
  const double u = 1.1920928955078125e-7;   // 2^-23
  const double um = 9.5367431640625e-7;     // 2^-20, per matrix-core addition
  const double n = static_cast<double>(dim) + 4.0;
  const double gamma = n * u / (1.0 - n * u);
  const double m = 3.0 * 32.0 * ksteps + 3.0 * ksteps + 16.0;
  const double gm = m * um / (1.0 - m * um);
  const double emf = 3.05 * 1.52587890625e-5 + 1.02 * gm;  // 2^-16 split remainder
  const double qd = static_cast<double>(qn) * (1.0 + 4.0 * n * u);
  const double cd = static_cast<double>(cn_max) * (1.0 + 4.0 * n * u);
  const double S = sqrt(qd * cd) * (1.0 + 1e-6);
  const double E = 2.0 * (2.0 * (emf + gamma) * S + 2.0 * u * (qd + cd + 2.0 * S)) +
                   m * 1e-30 * (1.0 + sqrt(qd) + sqrt(cd));
  const double T = static_cast<double>(t) + 2.0 * E;
  float f = static_cast<float>(T);
  if (static_cast<double>(f) < T && f < __builtin_inff()) f = next_up(f);
  return f;
}

template <int KS, int NW>
__global__ __launch_bounds__(64 * NW) void k_probe_mfma(const OvvsProbeArgs p, const ProbeShape shape) {
  constexpr int kWaves = NW;
  constexpr int kThreads = 64 * NW;
  constexpr int kRowsPerWave = kRows / kWaves;  // rows each wave selects and ranks
  extern __shared__ __align__(16) unsigned char smem[];
  const Carve L = carve(smem, shape);
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t q0 = static_cast<int64_t>(blockIdx.x) * kRows;
  const int dim = p.dim, dq = shape.dq;

  // Stage the 16 query rows (zero past dim and past nq).
  for (int i = static_cast<int>(threadIdx.x); i < kRows * dq; i += kThreads) {
    const int r = i / dq, t = i - r * dq;
    const int64_t q = q0 + r;
    L.qs[i] = (q < p.nq && t < dim) ? p.queries[q * dim + t] : 0.f;
  }
  if (threadIdx.x < kRows) L.count[threadIdx.x] = 0;
  if (p.zero && blockIdx.x == 0 && threadIdx.x < 4) p.zero[threadIdx.x] = 0;
  __syncthreads();
  // Query norms: given, or the sequential sums of squares of the staged rows.
  if (threadIdx.x < kRows) {
    const int64_t q = q0 + threadIdx.x;
    float s = 0.f;
    if (p.qnorm) {
      s = q < p.nq ? p.qnorm[q] : 0.f;
    } else {
      const float* r = L.qs + threadIdx.x * dq;
      for (int t = 0; t < dim; ++t) s = s + r[t] * r[t];
      if (q < p.nq) p.qnorm_out[q] = s;
    }
    L.qn[threadIdx.x] = q < p.nq ? s : 0.f;
  }
  __syncthreads();

  bf16x8 ah[KS], al[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    uint16_t h[8], l[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = 32 * s + 8 * (lane >> 4) + j;
      split_bf16(k < dim ? L.qs[(lane & 15) * dq + k] : 0.f, h[j], l[j]);
    }
    __builtin_memcpy(&ah[s], h, sizeof(h));
    __builtin_memcpy(&al[s], l, sizeof(l));
  }
  float qn[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t row = q0 + 4 * (lane >> 4) + r;
    qn[r] = L.qn[4 * (lane >> 4) + r];
    (void)row;
  }
  const int col = lane & 15;

  // Pass 1: running minimum of a over each (chunk, column) group.
  for (int ch = wave; ch < shape.nch; ch += kWaves) {
    const int t0 = ch * shape.gt;
    const int t1 = min(t0 + shape.gt, shape.ntile);
    float m[4] = {__builtin_inff(), __builtin_inff(), __builtin_inff(), __builtin_inff()};
    for (int t = t0; t < t1; ++t) {
      const f32x4 acc = tile_dot<KS>(ah, al, p.cmfma, t);
      const int c = 16 * t + col;
      if (c < p.nlist) {
        const float cn = p.cnorm[c];
#pragma unroll
        for (int r = 0; r < 4; ++r) m[r] = __builtin_fminf(m[r], (qn[r] + cn) - 2.f * acc[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
      L.gmin[(4 * (lane >> 4) + r) * (16 * shape.nch) + ch * 16 + col] = score_key(m[r]);
  }
  __syncthreads();

  // The P-th smallest group minimum of each row, bit by bit from the top: v is the
  // smallest key with at least P group minima <= v. Each lane holds its slots; the
  // wave's rows are searched together (independent compare/count chains).
  const int ng = 16 * shape.nch;
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
    for (int b = 31; b >= 0; --b) {
      int cnt[kRowsPerWave];
#pragma unroll
      for (int rr = 0; rr < kRowsPerWave; ++rr) {
        const uint32_t probe = v[rr] | ((1u << b) - 1u);
        cnt[rr] = 0;
#pragma unroll
        for (int i = 0; i < kMaxChunks / 4; ++i) cnt[rr] += __popcll(__ballot(g[rr][i] <= probe));
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
        const float qnr = q < p.nq ? L.qn[row] : 0.f;
        L.thr[row] = candidate_bound(key_to_score(v[rr]), qnr, p.cnorm_max, dim, KS);
      }
    }
  }
  __syncthreads();

  // Pass 2: every centroid whose approximate score is not above the bound.
  float T[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) T[r] = L.thr[4 * (lane >> 4) + r];
  const int cap = shape.cap;
  for (int t = wave; t < shape.ntile; t += kWaves) {
    const f32x4 acc = tile_dot<KS>(ah, al, p.cmfma, t);
    const int c = 16 * t + col;
    if (c < p.nlist) {
      const float cn = p.cnorm[c];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float s = (qn[r] + cn) - 2.f * acc[r];
        if (!(s > T[r])) {
          const int row = 4 * (lane >> 4) + r;
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
    const float dot = (dim & 3) == 0 ? seq_dot_v4_ahead(qrow, crow, dim) : seq_dot(qrow, crow, dim);
    *s = make_key((L.qn[row] + p.cnorm[c]) - 2.f * dot, c);
  }
  wave_sync();
  for (int f = lane; f < total; f += 64) {
    int rr = 0;
#pragma unroll
    for (int j = 1; j < kRowsPerWave; ++j) rr += f >= pre[j] ? 1 : 0;
    const int row = kRowsPerWave * wave + rr;
    const uint64_t* keys = L.slot + row * cap;
    const uint64_t key = keys[f - pre[rr]];
    int rank = 0;
    for (int j = 0; j < cnt[rr]; ++j) rank += keys[j] < key ? 1 : 0;
    if (rank < p.P) p.probes[(q0 + row) * p.P + rank] = static_cast<int32_t>(key & 0xffffffffu);
    if (rank == 0 && p.order_keys) p.order_keys[q0 + row] = p.list_rank[key & 0xffffffffu] >> p.key_shift;
  }
}

// Shape of a launch, or false when the fused probe does not serve these sizes.
bool probe_shape(int32_t dim, int32_t nlist, int32_t P, ProbeShape* sh) {
  if (dim <= 0 || dim > 32 * OVVS_PROBE_MAX_KSTEPS || nlist <= 0 || nlist > (1 << 24) || P <= 0 ||
      P > OVVS_PROBE_MAX_P)
    return false;
  sh->ntile = (nlist + 15) / 16;
  sh->gt = (sh->ntile + kMaxChunks - 1) / kMaxChunks;
  sh->nch = (sh->ntile + sh->gt - 1) / sh->gt;
  int real = 0;
  for (int ch = 0; ch < sh->nch; ++ch) real += min(16, nlist - 16 * ch * sh->gt);
  sh->real_groups = real;
  if (2 * P > real) return false;
  sh->cap = P <= 64 ? 256 : OVVS_PROBE_CAP;
  sh->dq = (dim + 3) & ~3;
  const size_t area = static_cast<size_t>(kRows) *
                      (static_cast<size_t>(16 * sh->nch) * 4 > static_cast<size_t>(sh->cap) * 8
                           ? static_cast<size_t>(16 * sh->nch) * 4
                           : static_cast<size_t>(sh->cap) * 8);
  sh->lds = align16(static_cast<size_t>(kRows) * sh->dq * 4) + align16(3 * kRows * 4) + area;
  return sh->lds <= 160 * 1024;
}

template <int KS, int NW>
hipError_t launch_probe_nw(const OvvsProbeArgs& p, const ProbeShape& sh, hipStream_t stream) {
  if (sh.lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_probe_mfma<KS, NW>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(sh.lds));
    if (e != hipSuccess) return e;
  }
  const int64_t blocks = (p.nq + kRows - 1) / kRows;
  hipLaunchKernelGGL((k_probe_mfma<KS, NW>), dim3(static_cast<uint32_t>(blocks)), dim3(64 * NW),
                     sh.lds, stream, p, sh);
  return hipGetLastError();
}

// 16 waves per workgroup when the batch gives fewer workgroups than the 256 CUs
// (small batches: the latency of one workgroup is the launch), else 8.
template <int KS>
hipError_t launch_probe(const OvvsProbeArgs& p, const ProbeShape& sh, hipStream_t stream) {
  if ((p.nq + kRows - 1) / kRows < 256) return launch_probe_nw<KS, 16>(p, sh, stream);
  return launch_probe_nw<KS, 8>(p, sh, stream);
}

}  // namespace

extern "C" int ovvs_hip_probe_mfma_supported(int32_t dim, int32_t nlist, int32_t P) {
  ProbeShape sh;
  return probe_shape(dim, nlist, P, &sh) ? 1 : 0;
}

extern "C" size_t ovvs_hip_probe_cmfma_words(int32_t dim, int32_t nlist) {
  if (dim <= 0 || dim > 32 * OVVS_PROBE_MAX_KSTEPS || nlist <= 0) return 0;
  const size_t ks = static_cast<size_t>((dim + 31) / 32);
  return static_cast<size_t>((nlist + 15) / 16) * ks * 2 * 64 * 4;
}

extern "C" void ovvs_probe_pack_cmfma(const float* C, int32_t nlist, int32_t dim,
                                      uint32_t* out) {
  const int ks = (dim + 31) / 32, ntile = (nlist + 15) / 16;
  for (int t = 0; t < ntile; ++t)
    for (int s = 0; s < ks; ++s)
      for (int lane = 0; lane < 64; ++lane) {
        uint16_t hi[8], lo[8];
        for (int j = 0; j < 8; ++j) {
          const int k = 32 * s + 8 * (lane / 16) + j, c = 16 * t + lane % 16;
          const float x = (c < nlist && k < dim) ? C[static_cast<size_t>(c) * dim + k] : 0.f;
          uint32_t u;
          std::memcpy(&u, &x, 4);
          hi[j] = bf16_bits(u);
          const uint32_t hu = static_cast<uint32_t>(hi[j]) << 16;
          float h;
          std::memcpy(&h, &hu, 4);
          const float r = x - h;
          std::memcpy(&u, &r, 4);
          lo[j] = bf16_bits(u);
        }
        uint32_t* dh = out + ((static_cast<size_t>(t) * ks + s) * 2 * 64 + lane) * 4;
        uint32_t* dl = dh + 64 * 4;
        for (int w = 0; w < 4; ++w) {
          dh[w] = static_cast<uint32_t>(hi[2 * w]) | (static_cast<uint32_t>(hi[2 * w + 1]) << 16);
          dl[w] = static_cast<uint32_t>(lo[2 * w]) | (static_cast<uint32_t>(lo[2 * w + 1]) << 16);
        }
      }
}

extern "C" hipError_t ovvs_hip_probe_mfma(const OvvsProbeArgs* args, hipStream_t stream) {
  if (!args) return hipErrorInvalidValue;
  const OvvsProbeArgs& p = *args;
  if (p.nq <= 0) return hipSuccess;
  ProbeShape sh;
  if (!p.queries || (!p.qnorm && !p.qnorm_out) || !p.centroids || !p.cmfma || !p.cnorm || !p.probes ||
      !p.fallback || p.nq > 0x7fffffff || !probe_shape(p.dim, p.nlist, p.P, &sh))
    return hipErrorInvalidValue;
  switch ((p.dim + 31) / 32) {
    case 1: return launch_probe<1>(p, sh, stream);
    case 2: return launch_probe<2>(p, sh, stream);
    case 3: return launch_probe<3>(p, sh, stream);
    default: return launch_probe<4>(p, sh, stream);
  }
}
