/* ivfpq_oracle.c — CPU restatement of the ovVS IVF-PQ search semantics.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker for libovvs: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
 * and never as the thing measured or shipped. libovvs does not link it.
 *
 * It restates, in plain C with every fp32 operation rounded separately
 * (built with -ffp-contract=off, no fast-math), the CPU route of
 * ovvsIvfPqSearch (reference src/neighbors/indexes.cpp:538-1134):
 *   coarse L2 score  (q.q + c.c) - 2(q.c)         mixer.cpp:174-199, cpu_prims.cpp:48-58
 *   total order      score asc, +-0 equal, NaN last, ordinal asc   cpu_prims.cpp:24-32
 *   probe set        first P centroids under that order             indexes.cpp:605-606
 *   candidate order  probe rank, then packed list order, bitset-filtered  indexes.cpp:683-712
 *   residual LUT     T[m][j] = sum_u (r_u - B[m][j][u])^2, r = q - c  indexes.cpp:764-785
 *   ADC              a = sum_m T[m][code_m], sequential from +0       mixer.cpp:378-390
 *   shortlist        first min(R, rows) by (a, dense ordinal)         indexes.cpp:1046-1047
 *   refine           exact metric distance of each shortlisted row    indexes.cpp:1067-1079
 *   final            first min(k, kr) by (v, shortlist rank), IP sign flip,
 *                    (-1, +inf) padding                               indexes.cpp:1080-1096
 * plus the declared binary16-LUT extension (no reference counterpart):
 * T16 = f16_rne(T), accumulated in fp32, and the ScaNN-style index around the
 * search (graphs.cpp:3286-3374): column factors sqrt(var + 1e-6) of the build,
 * scaled queries, re-rank of the returned ids on the original rows.
 *
 * Pinning: every function here is checked in tests/test_oracle.py against the
 * real reference compiled from /root/reference into oracle/_ref (bit-identical
 * ids and distances on shared IPQ1 indexes), against the reference tests'
 * known-answer cases (legacy IPQ1 blob, equal-score ties, cross-list ties,
 * filters), and against closed forms (nprobe = nlist with krefine = n equals
 * exact brute force). oracle_f32_to_f16 is pinned against numpy's float16
 * conversion (an independent IEEE round-to-nearest-even implementation). The
 * ScaNN functions are pinned against the reference's own ScaNN answers
 * (tests/golden/scann_cases.*, and oracle/_ref live), closed-form column
 * statistics, and brute force at full probe and refine. */

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#if defined(__FP_FAST_FMAF) || defined(__FAST_MATH__)
#error "the oracle must be built without FMA contraction and without fast-math"
#endif

enum { OR_L2 = 0, OR_L2_SQRT = 1, OR_IP = 2, OR_COSINE = 3, OR_HAMMING = 4, OR_LP = 5 };

typedef struct oracle_index {
  int64_t n;
  int64_t dim;
  int32_t nlist;
  int32_t pq_m;
  int32_t pq_ks;
  int32_t dsub;
  int32_t metric;
  int32_t pad_;
  const float* centroids;       /* [nlist * dim] */
  const float* codebooks;       /* [pq_m * pq_ks * dsub] */
  const uint8_t* packed_codes;  /* [n * pq_m], list-major */
  const int64_t* packed_ids;    /* [n] */
  const int64_t* list_offsets;  /* [nlist + 1] */
  const float* dataset;         /* [n * dim], row = id */
} oracle_index;

/* ---- scalar kernels: left-to-right fp32 sums from +0 (internal.hpp:57-64,215-225) ---- */

static float seq_l2sq(const float* a, const float* b, int64_t d) {
  float s = 0.f;
  for (int64_t i = 0; i < d; ++i) {
    const float t = a[i] - b[i];
    s += t * t;
  }
  return s;
}

static float seq_dot(const float* a, const float* b, int64_t d) {
  float s = 0.f;
  for (int64_t i = 0; i < d; ++i) s += a[i] * b[i];
  return s;
}

static float seq_norm(const float* a, int64_t d) {
  float s = 0.f;
  for (int64_t i = 0; i < d; ++i) s += a[i] * a[i];
  return s;
}

/* std::max(a, b) for floats: returns a unless a < b (keeps NaN in a). */
static float ref_max(float a, float b) { return (a < b) ? b : a; }

/* ---- total order (cpu_prims.cpp:24-32) ---- */

typedef struct {
  float score;
  int64_t ordinal;
} scored;

static int precedes(float ls, int64_t lo, float rs, int64_t ro) {
  if (ls < rs) return 1;
  if (ls > rs) return 0;
  const int ln = isnan(ls) != 0;
  const int rn = isnan(rs) != 0;
  if (ln != rn) return !ln;
  return lo < ro;
}

static int cmp_scored(const void* a, const void* b) {
  const scored* x = (const scored*)a;
  const scored* y = (const scored*)b;
  if (precedes(x->score, x->ordinal, y->score, y->ordinal)) return -1;
  if (precedes(y->score, y->ordinal, x->score, x->ordinal)) return 1;
  return 0;
}

/* First min(k, cols) entries of scores[0..cols) under the total order, sorted.
 * Ordinals are the column indices. Returns the number written. */
int64_t oracle_topk(const float* scores, int64_t cols, int64_t k, int64_t* idx, float* val) {
  if (cols <= 0 || k <= 0) return 0;
  if (k > cols) k = cols;
  scored* all = (scored*)malloc((size_t)cols * sizeof(scored));
  if (!all) return -1;
  for (int64_t i = 0; i < cols; ++i) {
    all[i].score = scores[i];
    all[i].ordinal = i;
  }
  qsort(all, (size_t)cols, sizeof(scored), cmp_scored);
  for (int64_t i = 0; i < k; ++i) {
    if (idx) idx[i] = all[i].ordinal;
    if (val) val[i] = all[i].score;
  }
  free(all);
  return k;
}

/* ---- binary16 (declared extension; conversion semantics as internal.hpp:83-106) ---- */

/* fp32 -> binary16 bits, round to nearest even; overflow (|x| >= 65520) -> inf;
 * NaN -> quiet NaN with the sign kept; subnormal halves are produced exactly. */
uint16_t oracle_f32_to_f16(float value) {
  uint32_t bits;
  memcpy(&bits, &value, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t mag = bits & 0x7fffffffu;
  if (mag > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  const int32_t exp = (int32_t)(mag >> 23) - 127; /* unbiased */
  if (exp >= 16) return (uint16_t)(sign | 0x7c00u);
  /* Express |x| = m * 2^(e) with the full 24-bit significand. */
  uint32_t sig = (mag & 0x7fffffu) | (mag >= 0x00800000u ? 0x800000u : 0u);
  if (mag < 0x00800000u) return (uint16_t)sign; /* fp32 subnormal: far below half range */
  /* Target quantum: 2^-24 for subnormal halves (exp < -14), else 2^(exp-10). */
  int32_t shift; /* how many low bits of sig fall below the half quantum */
  if (exp < -14) {
    shift = 13 + (-14 - exp);
    if (shift > 24) return (uint16_t)sign; /* < 2^-25: rounds to zero */
  } else {
    shift = 13;
  }
  uint32_t q = sig >> shift;
  const uint32_t rem = sig & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (q & 1u))) ++q;
  uint32_t out;
  if (exp < -14) {
    out = q; /* subnormal (q may carry into the smallest normal: 0x400) */
  } else {
    /* q has 11 bits (1.mantissa); a carry to 12 bits bumps the exponent. */
    uint32_t e = (uint32_t)(exp + 15);
    if (q >= 0x800u) {
      q >>= 1;
      ++e;
    }
    if (e >= 31u) return (uint16_t)(sign | 0x7c00u);
    out = (e << 10) | (q & 0x3ffu);
  }
  return (uint16_t)(sign | out);
}

float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  float mag;
  if (e == 0) {
    mag = ldexpf((float)m, -24);
  } else if (e == 31) {
    uint32_t b = 0x7f800000u | (m << 13);
    memcpy(&mag, &b, 4);
  } else {
    mag = ldexpf((float)(m | 0x400u), (int)e - 25);
  }
  uint32_t b;
  memcpy(&b, &mag, 4);
  b |= sign;
  float out;
  memcpy(&out, &b, 4);
  return out;
}

/* ---- coarse probe (mixer.cpp:174-199 with cpu_gemm, then cpu_topk) ---- */

void oracle_coarse_scores(const float* queries, int64_t nq, const float* centroids, int32_t nlist,
                          int64_t dim, float* out) {
  float* cn = (float*)malloc((size_t)nlist * sizeof(float));
  for (int32_t c = 0; c < nlist; ++c) cn[c] = seq_norm(centroids + (int64_t)c * dim, dim);
  for (int64_t q = 0; q < nq; ++q) {
    const float* qv = queries + q * dim;
    const float qn = seq_norm(qv, dim);
    for (int32_t c = 0; c < nlist; ++c) {
      const float ip = seq_dot(qv, centroids + (int64_t)c * dim, dim);
      out[q * nlist + c] = (qn + cn[c]) - 2.f * ip;
    }
  }
  free(cn);
}

/* probes: [nq * P] centroid ids in rank order. */
int oracle_probe(const oracle_index* ix, const float* queries, int64_t nq, int32_t P,
                 int64_t* probes) {
  float* s = (float*)malloc((size_t)nq * (size_t)ix->nlist * sizeof(float));
  if (!s) return -1;
  oracle_coarse_scores(queries, nq, ix->centroids, ix->nlist, ix->dim, s);
  for (int64_t q = 0; q < nq; ++q) {
    oracle_topk(s + q * ix->nlist, ix->nlist, P, probes + q * P, NULL);
  }
  free(s);
  return 0;
}

/* ---- residual lookup table (indexes.cpp:764-785) ---- */

void oracle_lut(const oracle_index* ix, const float* query, int32_t list, int32_t lut_f16,
                float* table) {
  const int64_t dim = ix->dim;
  float* r = (float*)malloc((size_t)dim * sizeof(float));
  const float* c = ix->centroids + (int64_t)list * dim;
  for (int64_t t = 0; t < dim; ++t) r[t] = query[t] - c[t];
  for (int32_t m = 0; m < ix->pq_m; ++m) {
    const float* cb = ix->codebooks + (int64_t)m * ix->pq_ks * ix->dsub;
    for (int32_t j = 0; j < ix->pq_ks; ++j) {
      float v = seq_l2sq(r + (int64_t)m * ix->dsub, cb + (int64_t)j * ix->dsub, ix->dsub);
      if (lut_f16) v = oracle_f16_to_f32(oracle_f32_to_f16(v));
      table[(int64_t)m * ix->pq_ks + j] = v;
    }
  }
  free(r);
}

static int id_allowed(const uint8_t* bitset, int64_t id) {
  if (!bitset) return 1;
  return (bitset[id >> 3] >> (id & 7)) & 1;
}

/* Shortlist of one query: the first min(R, rows) candidates by (ADC, dense
 * ordinal). out_pos gets packed positions, out_score ADC scores, in order.
 * Returns the shortlist length, or -1 on allocation failure. total_rows (if not
 * NULL) receives the query's accepted candidate count. */
int64_t oracle_shortlist(const oracle_index* ix, const float* query, const int64_t* probes,
                         int32_t P, int32_t R, const uint8_t* bitset, int32_t lut_f16,
                         int64_t* out_pos, float* out_score, int64_t* total_rows) {
  int64_t rows = 0;
  for (int32_t p = 0; p < P; ++p) {
    const int64_t l = probes[p];
    rows += ix->list_offsets[l + 1] - ix->list_offsets[l];
  }
  scored* cand = (scored*)malloc((size_t)(rows > 0 ? rows : 1) * sizeof(scored));
  int64_t* pos = (int64_t*)malloc((size_t)(rows > 0 ? rows : 1) * sizeof(int64_t));
  float* table = (float*)malloc((size_t)ix->pq_m * (size_t)ix->pq_ks * sizeof(float));
  if (!cand || !pos || !table) {
    free(cand);
    free(pos);
    free(table);
    return -1;
  }
  int64_t dense = 0;
  for (int32_t p = 0; p < P; ++p) {
    const int64_t l = probes[p];
    const int64_t b = ix->list_offsets[l], e = ix->list_offsets[l + 1];
    if (e <= b) continue;
    oracle_lut(ix, query, (int32_t)l, lut_f16, table);
    for (int64_t at = b; at < e; ++at) {
      if (!id_allowed(bitset, ix->packed_ids[at])) continue;
      const uint8_t* code = ix->packed_codes + at * ix->pq_m;
      float a = 0.f;
      for (int32_t m = 0; m < ix->pq_m; ++m) a += table[(int64_t)m * ix->pq_ks + code[m]];
      cand[dense].score = a;
      cand[dense].ordinal = dense;
      pos[dense] = at;
      ++dense;
    }
  }
  if (total_rows) *total_rows = dense;
  qsort(cand, (size_t)dense, sizeof(scored), cmp_scored);
  const int64_t kr = dense < R ? dense : R;
  for (int64_t i = 0; i < kr; ++i) {
    out_pos[i] = pos[cand[i].ordinal];
    if (out_score) out_score[i] = cand[i].score;
  }
  free(cand);
  free(pos);
  free(table);
  return kr;
}

/* ---- exact re-rank distance (mixer.cpp:177-221, internal.hpp:240-272) ---- */

float oracle_refine_distance(int32_t metric, const float* q, const float* x, int64_t dim) {
  switch (metric) {
    case OR_L2: {
      const float qn = seq_norm(q, dim), xn = seq_norm(x, dim), ip = seq_dot(q, x, dim);
      return (qn + xn) - 2.f * ip;
    }
    case OR_IP:
      return -seq_dot(q, x, dim);
    case OR_COSINE: {
      const float qn = seq_norm(q, dim), xn = seq_norm(x, dim), ip = seq_dot(q, x, dim);
      const float a = sqrtf(ref_max(qn, 1e-12f));
      const float b = sqrtf(ref_max(xn, 1e-12f));
      return 1.f - ip / (a * b);
    }
    case OR_L2_SQRT:
      return sqrtf(seq_l2sq(q, x, dim));
    case OR_HAMMING: {
      int s = 0;
      for (int64_t i = 0; i < dim; ++i) s += (int)((uint32_t)(q[i] >= 0.f) ^ (uint32_t)(x[i] >= 0.f));
      return (float)s;
    }
    case OR_LP: {
      const float p = 2.f; /* the search passes metric_arg 2 (indexes.cpp:1076) */
      float s = 0.f;
      for (int64_t i = 0; i < dim; ++i) s += powf(fabsf(q[i] - x[i]), p);
      return powf(s, 1.f / p);
    }
    default:
      return seq_l2sq(q, x, dim);
  }
}

/* ---- full search (indexes.cpp:538-1134) ---- */

int oracle_ivfpq_search(const oracle_index* ix, const float* queries, int64_t nq, int64_t k,
                        int32_t nprobe, int32_t krefine, const uint8_t* bitset, int32_t lut_f16,
                        int64_t* neighbors, float* distances) {
  int32_t P = nprobe < ix->nlist ? nprobe : ix->nlist;
  if (P < 1) P = 1;
  const int32_t R = krefine < (int32_t)k ? (int32_t)k : krefine;
  int64_t* probes = (int64_t*)malloc((size_t)nq * (size_t)P * sizeof(int64_t));
  int64_t* spos = (int64_t*)malloc((size_t)R * sizeof(int64_t));
  float* v = (float*)malloc((size_t)R * sizeof(float));
  int64_t* fidx = (int64_t*)malloc((size_t)R * sizeof(int64_t));
  float* fval = (float*)malloc((size_t)R * sizeof(float));
  if (!probes || !spos || !v || !fidx || !fval || oracle_probe(ix, queries, nq, P, probes) != 0) {
    free(probes);
    free(spos);
    free(v);
    free(fidx);
    free(fval);
    return -1;
  }
  for (int64_t q = 0; q < nq; ++q) {
    const float* qv = queries + q * ix->dim;
    for (int64_t t = 0; t < k; ++t) {
      neighbors[q * k + t] = -1;
      distances[q * k + t] = INFINITY;
    }
    const int64_t kr =
        oracle_shortlist(ix, qv, probes + q * P, P, R, bitset, lut_f16, spos, NULL, NULL);
    if (kr < 0) return -1;
    if (kr == 0) continue;
    for (int64_t i = 0; i < kr; ++i) {
      const int64_t id = ix->packed_ids[spos[i]];
      v[i] = oracle_refine_distance(ix->metric, qv, ix->dataset + id * ix->dim, ix->dim);
    }
    const int64_t kk = oracle_topk(v, kr, k, fidx, fval);
    for (int64_t t = 0; t < kk; ++t) {
      neighbors[q * k + t] = ix->packed_ids[spos[fidx[t]]];
      distances[q * k + t] = ix->metric == OR_IP ? -fval[t] : fval[t];
    }
  }
  free(probes);
  free(spos);
  free(v);
  free(fidx);
  free(fval);
  return 0;
}

/* Exact nearest neighbours by the index metric over the whole dataset, the
 * closed form IVF-PQ reduces to when nprobe = nlist and krefine >= n. */
int oracle_brute_force(const float* dataset, int64_t n, int64_t dim, int32_t metric,
                       const float* queries, int64_t nq, int64_t k, int64_t* neighbors,
                       float* distances) {
  float* v = (float*)malloc((size_t)n * sizeof(float));
  int64_t* idx = (int64_t*)malloc((size_t)k * sizeof(int64_t));
  float* val = (float*)malloc((size_t)k * sizeof(float));
  if (!v || !idx || !val) {
    free(v);
    free(idx);
    free(val);
    return -1;
  }
  for (int64_t q = 0; q < nq; ++q) {
    const float* qv = queries + q * dim;
    for (int64_t i = 0; i < n; ++i) v[i] = oracle_refine_distance(metric, qv, dataset + i * dim, dim);
    const int64_t kk = oracle_topk(v, n, k, idx, val);
    for (int64_t t = 0; t < k; ++t) {
      neighbors[q * k + t] = t < kk ? idx[t] : -1;
      distances[q * k + t] = t < kk ? (metric == OR_IP ? -val[t] : val[t]) : INFINITY;
    }
  }
  free(v);
  free(idx);
  free(val);
  return 0;
}

/* ---- ScaNN-style index (graphs.cpp:3286-3374) ---- */

/* Column factors of the build (graphs.cpp:3291-3301): m = (sum_i x[i][d]) / n,
 * v = sum_i (x[i][d] - m)^2, aniso[d] = sqrt(v / max(n, 1) + 1e-6), every sum
 * left to right in fp32. */
void oracle_scann_aniso(const float* x, int64_t n, int64_t dim, float* aniso) {
  for (int64_t d = 0; d < dim; ++d) {
    float m = 0.f;
    for (int64_t i = 0; i < n; ++i) m += x[i * dim + d];
    m /= (float)n;
    float v = 0.f;
    for (int64_t i = 0; i < n; ++i) {
      const float t = x[i * dim + d] - m;
      v += t * t;
    }
    aniso[d] = sqrtf(v / (float)(n > 1 ? n : 1) + 1e-6f);
  }
}

/* Search (graphs.cpp:3316-3374): R = max(krefine, k); IVF-PQ search of the
 * queries scaled column-wise by aniso for R results (k = R) on `ix` (the index
 * built on the scaled rows); then per query the returned ids in [0, n), in result
 * order, re-ranked by the index metric on the original rows and queries, the first
 * min(k, count) by (distance, position) written (inner product as +ip) and the
 * rest padded with (-1, +inf). Returns 0, or -1 when the inner search fails. */
int oracle_scann_search(const oracle_index* ix, const float* rows, int64_t n, const float* aniso,
                        const float* queries, int64_t nq, int64_t k, int32_t nprobe,
                        int32_t krefine, int64_t* neighbors, float* distances) {
  const int64_t dim = ix->dim;
  const int32_t R = krefine < (int32_t)k ? (int32_t)k : krefine;
  if (nq <= 0 || R <= 0) return -1;
  float* qs = (float*)malloc((size_t)nq * (size_t)dim * sizeof(float));
  int64_t* cand = (int64_t*)malloc((size_t)nq * (size_t)R * sizeof(int64_t));
  float* cd = (float*)malloc((size_t)nq * (size_t)R * sizeof(float));
  int64_t* ids = (int64_t*)malloc((size_t)R * sizeof(int64_t));
  float* v = (float*)malloc((size_t)R * sizeof(float));
  int64_t* idx = (int64_t*)malloc((size_t)R * sizeof(int64_t));
  float* val = (float*)malloc((size_t)R * sizeof(float));
  int rc = -1;
  if (!qs || !cand || !cd || !ids || !v || !idx || !val) goto done;
  for (int64_t i = 0; i < nq; ++i)
    for (int64_t d = 0; d < dim; ++d) qs[i * dim + d] = queries[i * dim + d] * aniso[d];
  if (oracle_ivfpq_search(ix, qs, nq, R, nprobe, R, NULL, 0, cand, cd) != 0) goto done;
  for (int64_t q = 0; q < nq; ++q) {
    int64_t m = 0;
    for (int32_t t = 0; t < R; ++t) {
      const int64_t id = cand[q * R + t];
      if (id >= 0 && id < n) ids[m++] = id;
    }
    for (int64_t i = 0; i < m; ++i)
      v[i] = oracle_refine_distance(ix->metric, queries + q * dim, rows + ids[i] * dim, dim);
    const int64_t kk = oracle_topk(v, m, k, idx, val);
    if (kk < 0) goto done;
    for (int64_t t = 0; t < k; ++t) {
      neighbors[q * k + t] = t < kk ? ids[idx[t]] : -1;
      distances[q * k + t] = t < kk ? (ix->metric == OR_IP ? -val[t] : val[t]) : INFINITY;
    }
  }
  rc = 0;
done:
  free(qs);
  free(cand);
  free(cd);
  free(ids);
  free(v);
  free(idx);
  free(val);
  return rc;
}
