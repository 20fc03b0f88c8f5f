// scan_layout.cpp — the order in which the scan visits an IVF-PQ index's rows.
//
// Each list's rows are split into segments of at most `seg_rows` rows whose PQ
// reconstructions lie close together (recursive 2-means on the reconstructed
// residuals). Every segment starts at a 64-row code tile and carries the
// per-dimension range (box) of its rows' reconstructions; the box gives a lower
// bound on the ADC score of every row of the segment for any query, which lets the
// scan skip segments whose rows cannot enter a shortlist. Every row keeps its
// index within its list (the reference's packed order, src/neighbors/indexes.cpp:
// 50-57, 683-712), and the scan orders candidates by that index, so the visiting
// order changes no result. The segmentation only affects how much the scan can
// skip; any split is correct.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>
#include <thread>
#include <utility>
#include <vector>

#include "internal.hpp"

namespace {

using ovvs::ScanLayoutHost;

// IEEE binary16 helpers (bit patterns): round to nearest even, exact widening, and
// the neighbours toward -inf / +inf.
uint16_t half_rne(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return static_cast<uint16_t>(sign | 0x7e00u);  // NaN
  if (ax >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // rounds to inf
  if (ax < 0x38800000u) {
    // Subnormal (or zero) half: value = m * 2^-24, m = round(|f| * 2^24).
    if (ax < 0x33000000u) return static_cast<uint16_t>(sign);  // below half of the smallest
    const uint32_t e = ax >> 23;
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;  // 14..24 for e in [102, 112]
    uint32_t m = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1u);
    if (rem > halfway || (rem == halfway && (m & 1u))) ++m;
    return static_cast<uint16_t>(sign | m);
  }
  uint32_t h = ((ax >> 13) - (112u << 10));
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return static_cast<uint16_t>(sign | h);
}

float half_to_float(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  float v;
  if (e == 0) {
    v = std::ldexp(static_cast<float>(m), -24);
  } else if (e == 31) {
    v = m ? std::numeric_limits<float>::quiet_NaN() : std::numeric_limits<float>::infinity();
  } else {
    v = std::ldexp(static_cast<float>(m | 0x400u), static_cast<int>(e) - 25);
  }
  return sign ? -v : v;
}

uint16_t half_toward_neg(uint16_t h) {
  if (h == 0xfc00u) return h;
  if (h & 0x8000u) return static_cast<uint16_t>(h + 1u);
  return h == 0 ? static_cast<uint16_t>(0x8001u) : static_cast<uint16_t>(h - 1u);
}

uint16_t half_toward_pos(uint16_t h) {
  if (h == 0x7c00u) return h;
  if (h & 0x8000u) return h == 0x8000u ? static_cast<uint16_t>(1u) : static_cast<uint16_t>(h - 1u);
  return static_cast<uint16_t>(h + 1u);
}

}  // namespace

namespace ovvs {

// Largest binary16 value <= lo and smallest >= hi (lo, hi not NaN), packed as
// lo | hi << 16: a box that contains [lo, hi].
uint32_t pack_box_fp16(float lo, float hi) {
  uint16_t l = half_rne(lo), h = half_rne(hi);
  if (half_to_float(l) > lo) l = half_toward_neg(l);
  if (half_to_float(h) < hi) h = half_toward_pos(h);
  return static_cast<uint32_t>(l) | (static_cast<uint32_t>(h) << 16);
}

float unpack_box_fp16(uint32_t b, int hi) { return half_to_float(static_cast<uint16_t>(hi ? b >> 16 : b & 0xffffu)); }

// The range [c + lo, c + hi] in absolute coordinates, rounded outward to binary16:
// the sums are formed in double, widened by a relative 2^-40 (more than their
// rounding error), rounded outward to float and then to binary16. A non-finite
// centroid coordinate bounds nothing.
uint32_t pack_abs_box_fp16(float c, float lo, float hi) {
  constexpr float kInf = std::numeric_limits<float>::infinity();
  if (!std::isfinite(c)) return pack_box_fp16(-kInf, kInf);
  double a = static_cast<double>(c) + static_cast<double>(lo);
  double b = static_cast<double>(c) + static_cast<double>(hi);
  a -= std::fabs(a) * 0x1p-40;
  b += std::fabs(b) * 0x1p-40;
  float fa = static_cast<float>(a), fb = static_cast<float>(b);
  if (static_cast<double>(fa) > a) fa = std::nextafter(fa, -kInf);
  if (static_cast<double>(fb) < b) fb = std::nextafter(fb, kInf);
  return pack_box_fp16(fa, fb);
}

}  // namespace ovvs

namespace {

// Squared distance between two reconstruction rows (float accumulation in double).
double dist2(const float* a, const float* b, int D) {
  double s = 0.0;
  for (int d = 0; d < D; ++d) {
    const double t = static_cast<double>(a[d]) - static_cast<double>(b[d]);
    s += t * t;
  }
  return s;
}

double dist2(const float* a, const double* b, int D) {
  double s = 0.0;
  for (int d = 0; d < D; ++d) {
    const double t = static_cast<double>(a[d]) - b[d];
    s += t * t;
  }
  return s;
}

// Splits rows idx (indices into X, rows of D floats) into two non-empty groups by
// a few 2-means iterations seeded with two far-apart rows; falls back to halves
// when the rows do not separate (identical or non-finite values).
void bisect(const float* X, int D, const std::vector<int32_t>& idx, std::vector<int32_t>& left,
            std::vector<int32_t>& right) {
  const size_t n = idx.size();
  auto row = [&](int32_t i) { return X + static_cast<size_t>(i) * D; };
  int32_t a = idx[0];
  double best = -1.0;
  for (const int32_t i : idx) {
    const double d = dist2(row(i), row(idx[0]), D);
    if (d > best) {
      best = d;
      a = i;
    }
  }
  int32_t b = a;
  best = -1.0;
  for (const int32_t i : idx) {
    const double d = dist2(row(i), row(a), D);
    if (d > best) {
      best = d;
      b = i;
    }
  }
  std::vector<uint8_t> side(n, 0);
  bool separated = false;
  if (best > 0.0 && std::isfinite(best)) {
    std::vector<double> ca(row(a), row(a) + D), cb(row(b), row(b) + D);
    std::vector<double> sa(static_cast<size_t>(D)), sb(static_cast<size_t>(D));
    for (int it = 0; it < 6; ++it) {
      size_t na = 0, nb = 0;
      std::fill(sa.begin(), sa.end(), 0.0);
      std::fill(sb.begin(), sb.end(), 0.0);
      bool changed = false;
      for (size_t t = 0; t < n; ++t) {
        const float* x = row(idx[t]);
        const uint8_t s = dist2(x, cb.data(), D) < dist2(x, ca.data(), D) ? 1 : 0;
        changed |= s != side[t];
        side[t] = s;
        std::vector<double>& acc = s ? sb : sa;
        for (int d = 0; d < D; ++d) acc[static_cast<size_t>(d)] += x[d];
        (s ? nb : na) += 1;
      }
      if (na == 0 || nb == 0) break;
      separated = true;
      if (it > 0 && !changed) break;
      for (int d = 0; d < D; ++d) {
        ca[static_cast<size_t>(d)] = sa[static_cast<size_t>(d)] / static_cast<double>(na);
        cb[static_cast<size_t>(d)] = sb[static_cast<size_t>(d)] / static_cast<double>(nb);
      }
    }
  }
  left.clear();
  right.clear();
  if (separated) {
    for (size_t t = 0; t < n; ++t) (side[t] ? right : left).push_back(idx[t]);
  }
  if (left.empty() || right.empty()) {
    left.assign(idx.begin(), idx.begin() + static_cast<std::ptrdiff_t>(n / 2));
    right.assign(idx.begin() + static_cast<std::ptrdiff_t>(n / 2), idx.end());
  }
}

// Segments of one list: rows (indices into the list) of each segment in list order,
// segments in depth-first order of the bisection; groups[i] is the first segment of
// group i, a maximal subtree of the bisection holding at most group_segs segments
// (so a group is a run of consecutive segments with nearby reconstructions).
void segment_list(const float* X, int32_t n, int D, int seg_rows, int group_segs,
                  std::vector<std::vector<int32_t>>& segs, std::vector<int32_t>& groups) {
  segs.clear();
  groups.clear();
  // The bisection tree, built without recursion (a split may peel off a single row,
  // so the depth can reach the list's length). Children get larger node ids than
  // their parent; a node's segments are the consecutive run [first, first + nsegs).
  struct Node {
    int32_t left = -1, right = -1, first = 0, nsegs = 0;
  };
  std::vector<Node> nodes(1);
  std::vector<std::pair<std::vector<int32_t>, int32_t>> stack;
  stack.emplace_back(std::vector<int32_t>(static_cast<size_t>(n)), 0);
  for (int32_t i = 0; i < n; ++i) stack.back().first[static_cast<size_t>(i)] = i;
  std::vector<int32_t> left, right;
  while (!stack.empty()) {
    std::vector<int32_t> idx = std::move(stack.back().first);
    const int32_t v = stack.back().second;
    stack.pop_back();
    if (static_cast<int>(idx.size()) <= seg_rows) {
      std::sort(idx.begin(), idx.end());
      nodes[static_cast<size_t>(v)].first = static_cast<int32_t>(segs.size());
      nodes[static_cast<size_t>(v)].nsegs = 1;
      segs.push_back(std::move(idx));
      continue;
    }
    bisect(X, D, idx, left, right);
    const int32_t l = static_cast<int32_t>(nodes.size());
    nodes[static_cast<size_t>(v)].left = l;
    nodes[static_cast<size_t>(v)].right = l + 1;
    nodes.resize(nodes.size() + 2);
    stack.emplace_back(right, l + 1);  // the left subtree is taken first
    stack.emplace_back(left, l);
  }
  for (size_t v = nodes.size(); v-- > 0;) {
    Node& nd = nodes[v];
    if (nd.left < 0) continue;
    nd.first = nodes[static_cast<size_t>(nd.left)].first;
    nd.nsegs = nodes[static_cast<size_t>(nd.left)].nsegs + nodes[static_cast<size_t>(nd.right)].nsegs;
  }
  // Groups: the maximal subtrees with at most group_segs segments, in segment order.
  std::vector<int32_t> todo{0};
  while (!todo.empty()) {
    const Node& nd = nodes[static_cast<size_t>(todo.back())];
    todo.pop_back();
    if (nd.nsegs <= group_segs) {
      groups.push_back(nd.first);
      continue;
    }
    todo.push_back(nd.right);
    todo.push_back(nd.left);
  }
}

// Runs fn(c) for every list c over up to 16 host threads.
template <class Fn>
void for_each_list(int32_t nlist, Fn fn) {
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const unsigned workers = std::min<unsigned>(16u, std::min<unsigned>(hw, static_cast<unsigned>(nlist)));
  std::atomic<int32_t> next{0};
  auto run = [&]() {
    for (int32_t c = next.fetch_add(1); c < nlist; c = next.fetch_add(1)) fn(c);
  };
  std::vector<std::thread> pool;
  for (unsigned t = 1; t < workers; ++t) pool.emplace_back(run);
  run();
  for (std::thread& t : pool) t.join();
}

}  // namespace

namespace ovvs {

ovvsStatus make_scan_layout(const ovvsIvfPqIndexImpl& ix, int seg_rows, ScanLayoutHost& out) {
  constexpr int64_t kT = OVVS_CODE_TILE_ROWS, kB = OVVS_CODE_BLOCK;
  const int32_t nlist = ix.nlist, pq_m = ix.pq_m, ks = ix.pq_ks, dsub = ix.dsub;
  const int D = pq_m * dsub;
  const int64_t nblocks = (pq_m + kB - 1) / kB;
  const int64_t tile_bytes = nblocks * kT * kB;

  // Pass 1 (parallel): segments of every list.
  std::vector<std::vector<std::vector<int32_t>>> segs(static_cast<size_t>(nlist));
  std::vector<std::vector<int32_t>> grps(static_cast<size_t>(nlist));
  std::atomic<bool> failed{false};
  for_each_list(nlist, [&](int32_t c) {
    try {
      const std::vector<int64_t>& rows = ix.lists[static_cast<size_t>(c)];
      const int32_t n = static_cast<int32_t>(rows.size());
      if (n == 0) return;
      std::vector<float> X(static_cast<size_t>(n) * D);
      for (int32_t i = 0; i < n; ++i) {
        const uint8_t* code = ix.codes.data() + static_cast<size_t>(rows[static_cast<size_t>(i)]) * pq_m;
        float* x = X.data() + static_cast<size_t>(i) * D;
        for (int32_t m = 0; m < pq_m; ++m) {
          const float* cw = ix.codebooks.data() + (static_cast<size_t>(m) * ks + code[m]) * dsub;
          for (int32_t u = 0; u < dsub; ++u) x[m * dsub + u] = cw[u];
        }
      }
      segment_list(X.data(), n, D, seg_rows, OVVS_GROUP_SEGMENTS, segs[static_cast<size_t>(c)],
                   grps[static_cast<size_t>(c)]);
    } catch (...) {
      failed = true;
    }
  });
  if (failed) return OVVS_STATUS_OOM;

  // Positions and segment indices.
  out.list_seg.assign(static_cast<size_t>(nlist) + 1, 0);
  out.list_grp.assign(static_cast<size_t>(nlist) + 1, 0);
  std::vector<int64_t> list_pos(static_cast<size_t>(nlist) + 1, 0);
  int64_t nseg = 0, pos = 0, ngrp = 0;
  for (int32_t c = 0; c < nlist; ++c) {
    out.list_seg[static_cast<size_t>(c)] = static_cast<int32_t>(nseg);
    out.list_grp[static_cast<size_t>(c)] = static_cast<int32_t>(ngrp);
    ngrp += static_cast<int64_t>(grps[static_cast<size_t>(c)].size());
    list_pos[static_cast<size_t>(c)] = pos;
    for (const auto& s : segs[static_cast<size_t>(c)]) {
      pos += (static_cast<int64_t>(s.size()) + kT - 1) / kT * kT;
      ++nseg;
    }
    if (nseg > std::numeric_limits<int32_t>::max() || pos > std::numeric_limits<int32_t>::max())
      return OVVS_STATUS_DEVICE_UNAVAILABLE;
  }
  out.list_seg[static_cast<size_t>(nlist)] = static_cast<int32_t>(nseg);
  out.list_grp[static_cast<size_t>(nlist)] = static_cast<int32_t>(ngrp);
  out.grp_seg.assign(static_cast<size_t>(ngrp) + 1, static_cast<int32_t>(nseg));
  out.grp_box.assign(static_cast<size_t>(ngrp) * D, 0u);
  list_pos[static_cast<size_t>(nlist)] = pos;
  out.positions = pos;
  out.box_dims = D;
  out.seg_start.assign(static_cast<size_t>(nseg), 0);
  out.seg_len.assign(static_cast<size_t>(nseg), 0);
  out.seg_box.assign(static_cast<size_t>(nseg) * D, 0u);
  out.list_box.assign(static_cast<size_t>(nlist) * D, 0u);
  out.ids.assign(static_cast<size_t>(pos), -1);
  out.rord.assign(static_cast<size_t>(pos), -1);
  out.codes.assign(static_cast<size_t>(pos / kT) * static_cast<size_t>(tile_bytes), 0);

  // Pass 2 (parallel): rows, codes and boxes.
  for_each_list(nlist, [&](int32_t c) {
    const std::vector<int64_t>& rows = ix.lists[static_cast<size_t>(c)];
    int64_t p = list_pos[static_cast<size_t>(c)];
    int32_t sg = out.list_seg[static_cast<size_t>(c)];
    std::vector<float> lbox(static_cast<size_t>(D) * 2);
    for (int d = 0; d < D; ++d) {
      lbox[2 * d] = std::numeric_limits<float>::infinity();
      lbox[2 * d + 1] = -std::numeric_limits<float>::infinity();
    }
    std::vector<float> boxv(static_cast<size_t>(D) * 2);
    // Residual-coordinate boxes of this list's segments, for the group boxes.
    std::vector<float> seg_boxes(segs[static_cast<size_t>(c)].size() * static_cast<size_t>(D) * 2);
    const int32_t sg_first = out.list_seg[static_cast<size_t>(c)];
    for (const auto& s : segs[static_cast<size_t>(c)]) {
      out.seg_start[static_cast<size_t>(sg)] = static_cast<int32_t>(p);
      out.seg_len[static_cast<size_t>(sg)] = static_cast<int32_t>(s.size());
      float* box = boxv.data();
      for (int d = 0; d < D; ++d) {
        box[2 * d] = std::numeric_limits<float>::infinity();
        box[2 * d + 1] = -std::numeric_limits<float>::infinity();
      }
      std::vector<uint8_t> has_nan(static_cast<size_t>(D), 0);
      for (size_t t = 0; t < s.size(); ++t, ++p) {
        const int32_t r = s[t];
        const int64_t id = rows[static_cast<size_t>(r)];
        out.ids[static_cast<size_t>(p)] = id;
        out.rord[static_cast<size_t>(p)] = r;
        const uint8_t* code = ix.codes.data() + static_cast<size_t>(id) * pq_m;
        uint8_t* tile = out.codes.data() + static_cast<size_t>(p / kT) * tile_bytes + (p % kT) * kB;
        for (int32_t m = 0; m < pq_m; ++m) {
          tile[(m / kB) * (kT * kB) + (m % kB)] = code[m];
          const float* cw = ix.codebooks.data() + (static_cast<size_t>(m) * ks + code[m]) * dsub;
          for (int32_t u = 0; u < dsub; ++u) {
            const int d = m * dsub + u;
            const float v = cw[u];
            if (v != v) {
              has_nan[static_cast<size_t>(d)] = 1;
              continue;
            }
            box[2 * d] = std::min(box[2 * d], v);
            box[2 * d + 1] = std::max(box[2 * d + 1], v);
          }
        }
      }
      // A dimension with a NaN entry (or no finite entry) bounds nothing.
      uint32_t* packed = out.seg_box.data() + static_cast<size_t>(sg) * D;
      const float* cen = ix.centroids.data() + static_cast<size_t>(c) * static_cast<size_t>(ix.dim);
      for (int d = 0; d < D; ++d) {
        if (has_nan[static_cast<size_t>(d)] || !(box[2 * d] <= box[2 * d + 1])) {
          box[2 * d] = -std::numeric_limits<float>::infinity();
          box[2 * d + 1] = std::numeric_limits<float>::infinity();
        }
        lbox[2 * d] = std::min(lbox[2 * d], box[2 * d]);
        lbox[2 * d + 1] = std::max(lbox[2 * d + 1], box[2 * d + 1]);
        packed[d] = ovvs::pack_abs_box_fp16(cen[d], box[2 * d], box[2 * d + 1]);
      }
      std::copy(box, box + static_cast<size_t>(D) * 2,
                seg_boxes.begin() + static_cast<std::ptrdiff_t>(sg - sg_first) * D * 2);
      p = (p + kT - 1) / kT * kT;
      ++sg;
    }
    // Group boxes: the union of their segments' boxes.
    {
      const std::vector<int32_t>& gs = grps[static_cast<size_t>(c)];
      const float* cen = ix.centroids.data() + static_cast<size_t>(c) * static_cast<size_t>(ix.dim);
      const int32_t g_first = out.list_grp[static_cast<size_t>(c)];
      const int32_t nsl = static_cast<int32_t>(segs[static_cast<size_t>(c)].size());
      for (size_t gi = 0; gi < gs.size(); ++gi) {
        const int32_t s0 = gs[gi];
        const int32_t s1 = gi + 1 < gs.size() ? gs[gi + 1] : nsl;
        out.grp_seg[static_cast<size_t>(g_first) + gi] = sg_first + s0;
        uint32_t* gp = out.grp_box.data() + (static_cast<size_t>(g_first) + gi) * D;
        for (int d = 0; d < D; ++d) {
          float lo = std::numeric_limits<float>::infinity(), hi = -lo;
          for (int32_t k = s0; k < s1; ++k) {
            lo = std::min(lo, seg_boxes[(static_cast<size_t>(k) * D + d) * 2]);
            hi = std::max(hi, seg_boxes[(static_cast<size_t>(k) * D + d) * 2 + 1]);
          }
          gp[d] = ovvs::pack_abs_box_fp16(cen[d], lo, hi);
        }
      }
    }
    // The list's box contains every segment box (an empty list keeps an empty
    // box; the scan never evaluates it).
    uint32_t* lpacked = out.list_box.data() + static_cast<size_t>(c) * D;
    const float* cen = ix.centroids.data() + static_cast<size_t>(c) * static_cast<size_t>(ix.dim);
    for (int d = 0; d < D; ++d) {
      lpacked[d] = lbox[2 * d] <= lbox[2 * d + 1]
                       ? ovvs::pack_abs_box_fp16(cen[d], lbox[2 * d], lbox[2 * d + 1])
                       : 0x7c00fc00u;
    }
  });
  // Spatial rank of every list: the depth-first order of a recursive 2-means
  // bisection of the centroids (lists with nearby centroids get nearby ranks).
  {
    out.list_rank.assign(static_cast<size_t>(nlist), 0);
    std::vector<std::vector<int32_t>> stack;
    stack.emplace_back(static_cast<size_t>(nlist));
    for (int32_t c = 0; c < nlist; ++c) stack.back()[static_cast<size_t>(c)] = c;
    std::vector<int32_t> left, right;
    int32_t next = 0;
    while (!stack.empty()) {
      std::vector<int32_t> idx = std::move(stack.back());
      stack.pop_back();
      if (idx.size() <= 1) {
        for (const int32_t c : idx) out.list_rank[static_cast<size_t>(c)] = next++;
        continue;
      }
      bisect(ix.centroids.data(), ix.dim, idx, left, right);
      stack.push_back(right);
      stack.push_back(left);
    }
  }
  // Largest centroid coordinate magnitude (+inf if any is not finite): bounds how
  // far rounding can move a residual coordinate.
  out.cmax = 0.f;
  for (const float v : ix.centroids) {
    const float m = std::fabs(v);
    if (!(m <= out.cmax)) out.cmax = std::isfinite(m) ? m : std::numeric_limits<float>::infinity();
    if (std::isinf(out.cmax)) break;
  }
  return OVVS_STATUS_SUCCESS;
}

}  // namespace ovvs
