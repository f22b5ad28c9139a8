// The depth-first walk plan of a draft tree of at most 64 rows, built by one wave with lane u holding row u
// (shared by the GDN and Mamba2 tree walks). The rows are parent first (parent(u) < u for u > 0, row 0 the root).
//
// Children are walked in increasing (need, index), need being the stack entries a subtree's walk parks: 0 for a leaf,
// the child's for one child, else max(largest, second largest + 1) over the children (Sethi-Ullman / Strahler
// numbering; the neediest child last keeps the stack shallow). The plan gives every row its successor in that
// pre-order and how the walk reaches it, so the walk reads one lane per node.
//
// Built in parallel rather than by loops over the rows: child masks and first children by LDS atomics, depths and
// the successor's ancestor by pointer jumping over lane shuffles, needs one tree level at a time (children of the
// level below already counted into a per-row histogram), from the deepest level present. A serial row loop costs
// ~100 ns per row in one wave (a readlane, scalar branches and the vector updates per step), ~5 us for a 16-row tree;
// for the needs alone, a pass over 16 rows in decreasing index with lane-held histograms took 1.6 us against 1.3 for
// the levels.
#pragma once

#include <utility>

#include "common.h"

namespace e4walk {

// The LDS one wave uses while it builds a plan (1.8 KB), and where it hands the result to the other waves.
struct PlanScratch {
  uint64_t kids[64];  // row u: mask of u's children
  uint64_t hist[64];  // row u: byte n counts u's children of need n (needs <= 6 at 64 rows)
  int first[64];      // row u: smallest key among u's children
  int key[64];        // row u: need * 64 + u (or u when needs do not order the children)
  int plan[64];       // the packed plan (below)
  int dfs;            // the plan holds: the request is walked depth first
};

// Packed plan of row u: bits 0-6 the row walked after u (kNoNext: none), bit 7 it is u's first child (continues from
// u's registers), bit 8 it is the last child of its parent (the parked state is popped), bit 9 u has several
// children (its state is parked).
constexpr int kNoNext = 127;
constexpr int kPlanFirst = 1 << 7;
constexpr int kPlanLast = 1 << 8;
constexpr int kPlanMulti = 1 << 9;

E4_DEV int plan_next(int pl) { return (pl & kNoNext) == kNoNext ? -1 : (pl & kNoNext); }

// Orders LDS accesses of one wave against each other: the wave's LDS operations complete in issue order, so this only
// has to stop the compiler from moving them.
E4_DEV void wave_lds_order() { __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront"); }

// One rotation of the repeat check within each 16-lane row (DPP row_ror: no LDS round trip): lane u compares its slot
// with that of the lane D places along its row, whose index comes along the same rotation.
template <int D>
E4_DEV void row_repeat(int lo, int lane, int T, bool& dup) {
  const int other = __builtin_amdgcn_mov_dpp(lo, 0x120 + D, 0xF, 0xF, false);
  const int from = __builtin_amdgcn_mov_dpp(lane, 0x120 + D, 0xF, 0xF, false);
  dup = dup || (lane < T && from < T && other == lo);
}
template <int... Ds>
E4_DEV bool row_repeats(int lo, int lane, int T, std::integer_sequence<int, Ds...>) {
  bool dup = false;
  (row_repeat<Ds + 1>(lo, lane, T, dup), ...);
  return dup;
}

// Lane u: whether row u's 64-bit slot equals another row's, compared on the low words. Equal low words with different
// high words also count: a request with a duplicate keeps the index-order walk, which is exact for any slots.
// At most 16 rows all sit in the wave's first row of 16 lanes: 15 rotations within it; more rows, lane shuffles.
E4_DEV bool slot_repeats(uint64_t slot, int lane, int T) {
  const int lo = static_cast<int>(static_cast<uint32_t>(slot));
  if (T <= 16) return row_repeats(lo, lane, T, std::make_integer_sequence<int, 15>{});
  bool dup = false;
#pragma unroll 4
  for (int d = 1; d < T; ++d) {  // row u against row (u + d) mod 64: every pair of rows once per direction
    const int o = (lane + d) & 63;
    const int other = __shfl(lo, o, 64);
    dup = dup || (lane < T && o < T && other == lo);
  }
  return dup;
}

// Stack entries needed below a row from its children's histogram (Sethi-Ullman numbering).
E4_DEV int need_of(uint64_t hist) {
  if (hist == 0) return 0;
  const int m1 = (63 - __builtin_clzll(hist)) >> 3;
  const uint64_t c1 = (hist >> (8 * m1)) & 0xff;
  if (c1 >= 2) return m1 + 1;
  const uint64_t rest = hist & ~(0xffull << (8 * m1));
  if (rest == 0) return m1;  // one child
  const int m2 = (63 - __builtin_clzll(rest)) >> 3;
  return m1 > m2 + 1 ? m1 : m2 + 1;
}

// Builds the plan of a request of T <= 64 rows whose parents passed the checks (0 <= parent(u) < u for 0 < u < T).
// One whole wave calls it (every lane active); lane u returns row u's packed plan. by_need: children in (need, index)
// order, else in index order.
E4_DEV int build_plan(PlanScratch& ps, int lane, int T, int par, bool by_need) {
  const bool child = lane > 0 && lane < T;
  ps.kids[lane] = 0;
  ps.hist[lane] = 0;
  ps.first[lane] = 0x7fffffff;
  wave_lds_order();
  if (child) atomicOr(reinterpret_cast<unsigned long long*>(&ps.kids[par]), 1ull << lane);
  wave_lds_order();

  uint64_t kids;
  int first, after = -1;  // first child; the sibling walked after row u
  if (by_need) {
    // depths: d(u) += d(up(u)); up(u) = up(up(u)) until every row points at the root (six rounds reach 64 levels)
    int dep = child ? 1 : 0, up = child ? par : lane;
    for (int r = 0; r < 6 && __ballot(lane < T && up != 0) != 0; ++r) {
      const int d2 = __shfl(dep, up, 64), u2 = __shfl(up, up, 64);
      dep += d2;
      up = u2;
    }
    // the deepest level first: a row's children (one level down) have all counted themselves into its histogram
    int deepest = 0;  // the deepest level, bit by bit from ballots (depths are below 64)
#pragma unroll
    for (int b = 5; b >= 0; --b) {
      const int cand = deepest | (1 << b);
      if (__ballot(lane < T && dep >= cand) != 0) deepest = cand;
    }
    int need = 0;
    for (int level = deepest; level >= 1; --level) {
      const bool mine = child && dep == level;
      if (__ballot(mine) == 0) continue;
      if (mine) {
        need = need_of(ps.hist[lane]);
        atomicAdd(reinterpret_cast<unsigned long long*>(&ps.hist[par]), 1ull << (8 * need));
      }
      wave_lds_order();
    }
    const int key = need * 64 + lane;
    ps.key[lane] = key;
    if (child) atomicMin(&ps.first[par], key);
    wave_lds_order();

    kids = ps.kids[lane];
    const int fk = ps.first[lane];
    first = fk == 0x7fffffff ? -1 : (fk & 63);
    if (child) {  // the smallest key above u's among its parent's children
      uint64_t sib = ps.kids[par] & ~(1ull << lane);
      int best = 0x7fffffff;
      while (sib != 0) {
        const int s = __builtin_ctzll(sib);
        sib &= sib - 1;
        const int ks = ps.key[s];
        if (ks > key && ks < best) best = ks;
      }
      after = best == 0x7fffffff ? -1 : (best & 63);
    }
  } else {
    // index order: the first child is the lowest bit of the row's child mask, the next sibling the lowest bit of the
    // parent's mask above the row (2 << 63 wraps to 0: row 63 has none above it)
    kids = ps.kids[lane];
    first = kids != 0 ? __builtin_ctzll(kids) : -1;
    if (child) {
      const uint64_t above = ps.kids[par] & ~((2ull << lane) - 1ull);
      after = above != 0 ? __builtin_ctzll(above) : -1;
    }
  }
  // A row without children continues at the next sibling of its nearest ancestor-or-self that has one (the root:
  // the walk ends). Pointer jumping to the first marked ancestor-or-self, marked rows pointing at themselves.
  const bool marked = lane == 0 || lane >= T || after >= 0;
  int J = marked ? lane : par;
  for (int r = 0; r < 6; ++r) {
    const int JJ = __shfl(J, J, 64);
    if (__ballot(JJ != J) == 0) break;
    J = JJ;
  }
  const int after_J = __shfl(after, J, 64);
  const int next = first >= 0 ? first : (J == 0 ? -1 : after_J);
  const int after_next = __shfl(after, next & 63, 64);
  const bool last = first < 0 && next >= 0 && after_next < 0;
  return (next < 0 ? kNoNext : next) | (first >= 0 ? kPlanFirst : 0) | (last ? kPlanLast : 0) |
         ((kids & (kids - 1)) != 0 ? kPlanMulti : 0);
}

}  // namespace e4walk
