// Launch plan of the W4A16 prefill: which tile columns run 256-row tiles and
// which run 192-row tiles so that the last round of tiles on the CUs is not
// left part-empty.  Host-only C++ (no HIP), shared with a CPU check.
//
// Cost model: a 256 x 256 tile is one unit of CU time, a 192-row tile
// TAIL_COST_PCT / 100 of one (measured on MI355X: a round of 192-row tiles
// takes 0.86 of a round of 256-row ones).  The hardware dispatches tiles to
// CUs in order as CUs free up, i.e. a greedy list schedule: the `full` unit
// jobs first (every CU gets floor(full / cus), `full % cus` CUs one more), then
// each tail job on the least-loaded CU.  Costs are integers (percent), so the
// schedule is evaluated exactly.
#pragma once

#include <cstdint>

namespace tb {
namespace plan {

constexpr int64_t UNIT_COST = 100;
constexpr int64_t TAIL_COST_PCT = 86;

// The k-th smallest (k >= 1) element of the multiset
// {a + j c : j >= 0} (na copies) united with {b + j c : j >= 0} (nb copies),
// na >= 1, c > 0: the start time of the k-th tail job of a greedy schedule
// whose CUs start with loads a (na of them) and b (nb of them).
inline int64_t kth_start(int64_t a, int64_t na, int64_t b, int64_t nb, int64_t c, int64_t k) {
  auto count_le = [&](int64_t t) {
    int64_t n = 0;
    if (t >= a) n += na * ((t - a) / c + 1);
    if (t >= b) n += nb * ((t - b) / c + 1);
    return n;
  };
  int64_t lo = a < b || nb == 0 ? a : b, hi = a + (k - 1) * c;  // count_le(hi) >= na * k >= k
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo) / 2;
    if (count_le(mid) >= k)
      hi = mid;
    else
      lo = mid + 1;
  }
  return lo;
}

// Makespan (in percent of a unit) of `full` unit jobs then `tail` tail jobs on
// `cus` CUs under the greedy list schedule above.  O(log) per call.
inline int64_t makespan(int64_t full, int64_t tail, int64_t cus) {
  const int64_t r = full / cus, rem = full % cus;
  const int64_t top = (rem ? r + 1 : r) * UNIT_COST;
  if (tail == 0) return top;
  const int64_t start = kth_start(r * UNIT_COST, cus - rem, (r + 1) * UNIT_COST, rem, TAIL_COST_PCT, tail);
  const int64_t end = start + TAIL_COST_PCT;
  return end > top ? end : top;
}

struct PrefillPlan {
  int n_split, n_full, tail_m, tail_n, tail_blocks;
};

// Columns 0 .. n_split-1 of tiles run 256-row tiles (n_full blocks), the rest
// 192-row tiles (tail_m x tail_n of them, launched as tail_blocks, a multiple
// of 8).  A split is taken only when it shortens the makespan by 3 % or more;
// the first tile-column count (from the right) with a multiple of 8 full tiles
// that achieves the best makespan wins.
inline PrefillPlan plan_prefill(int M, int tiles_m, int tiles_n, int cus) {
  PrefillPlan p{tiles_n, tiles_m * tiles_n, 0, 0, 0};
  const int64_t tail_m = (M + 191) / 192;
  int64_t best = makespan((int64_t)tiles_m * tiles_n, 0, cus);
  for (int s = tiles_n - 1; s >= 0; --s) {
    if (((int64_t)tiles_m * s) % 8 != 0) continue;
    const int64_t t = makespan((int64_t)tiles_m * s, tail_m * (tiles_n - s), cus);
    if (t * 100 < best * 97) {
      best = t;
      p.n_split = s;
    }
  }
  if (p.n_split < tiles_n) {
    p.n_full = tiles_m * p.n_split;
    p.tail_m = (int)tail_m;
    p.tail_n = tiles_n - p.n_split;
    p.tail_blocks = (int)((tail_m * p.tail_n + 7) / 8 * 8);
  }
  return p;
}

}  // namespace plan
}  // namespace tb
