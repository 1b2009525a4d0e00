// CPU check of the W4A16 prefill launch plan (tilebench_amd/csrc/prefill_plan.h).
//
// The closed-form makespan must equal a direct simulation of the greedy list
// schedule (a min-heap of CU loads, every job placed on the least-loaded CU)
// for every (full, tail, cus) it is asked about, and the plan it picks must be
// the one the simulation-based planner picks.  Also checks the plans the GPU
// tests rely on and that planning a very large shape stays cheap.
// Build: g++ -O2 -std=c++17 -I tilebench_amd/csrc tests/native/prefill_plan_check.cpp
// With -DPLANT_OFF_BY_ONE the closed form counts one start too few and the
// check must fail.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <functional>
#include <vector>

#ifdef PLANT_OFF_BY_ONE
#include "prefill_plan.h"
namespace planted {
inline int64_t makespan(int64_t full, int64_t tail, int64_t cus) {
  return tb::plan::makespan(full, tail > 1 ? tail - 1 : tail, cus);
}
}  // namespace planted
#define MAKESPAN planted::makespan
#else
#include "prefill_plan.h"
#define MAKESPAN tb::plan::makespan
#endif

using tb::plan::TAIL_COST_PCT;
using tb::plan::UNIT_COST;

static int64_t simulate(int64_t full, int64_t tail, int64_t cus) {
  std::vector<int64_t> load((size_t)cus, 0);
  std::make_heap(load.begin(), load.end(), std::greater<int64_t>());
  auto place = [&](int64_t cost) {
    std::pop_heap(load.begin(), load.end(), std::greater<int64_t>());
    load.back() += cost;
    std::push_heap(load.begin(), load.end(), std::greater<int64_t>());
  };
  for (int64_t i = 0; i < full; ++i) place(UNIT_COST);
  for (int64_t i = 0; i < tail; ++i) place(TAIL_COST_PCT);
  return *std::max_element(load.begin(), load.end());
}

static tb::plan::PrefillPlan plan_by_simulation(int M, int tiles_m, int tiles_n, int cus) {
  tb::plan::PrefillPlan p{tiles_n, tiles_m * tiles_n, 0, 0, 0};
  const int64_t tail_m = (M + 191) / 192;
  int64_t best = simulate((int64_t)tiles_m * tiles_n, 0, cus);
  for (int s = tiles_n - 1; s >= 0; --s) {
    if (((int64_t)tiles_m * s) % 8 != 0) continue;
    const int64_t t = simulate((int64_t)tiles_m * s, tail_m * (tiles_n - s), cus);
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

int main() {
  long mismatches = 0, checked = 0;
  for (int64_t cus : {256, 304, 80, 7}) {
    for (int64_t full = 0; full <= 3 * cus + 5; full += (full < 2 * cus ? 1 : 3))
      for (int64_t tail = 0; tail <= 3 * cus + 5; tail += 1 + tail / 64) {
        ++checked;
        if (MAKESPAN(full, tail, cus) != simulate(full, tail, cus)) {
          if (mismatches < 5)
            std::printf("makespan(%lld, %lld, %lld): %lld vs simulated %lld\n", (long long)full, (long long)tail,
                        (long long)cus, (long long)MAKESPAN(full, tail, cus), (long long)simulate(full, tail, cus));
          ++mismatches;
        }
      }
  }
  long plan_mismatches = 0;
  for (int M = 17; M <= 12288; M += (M < 1024 ? 37 : 301))
    for (int N : {256, 1024, 1408, 2816, 4096, 5504, 11008, 14336}) {
      const int tm = (M + 255) / 256, tn = (N + 255) / 256;
      const auto a = tb::plan::plan_prefill(M, tm, tn, 256);
      const auto b = plan_by_simulation(M, tm, tn, 256);
      ++checked;
      if (a.n_split != b.n_split || a.n_full != b.n_full || a.tail_blocks != b.tail_blocks) ++plan_mismatches;
    }
  // plans the GPU tests and the headline rely on
  const auto c1 = tb::plan::plan_prefill(4096, 16, 43, 256);
  const bool c1_ok = c1.n_split == 32 && c1.n_full == 512 && c1.tail_m == 22 && c1.tail_n == 11;
  const auto t3 = tb::plan::plan_prefill(3000, 12, 43, 256);
  const bool t3_ok = t3.n_split == 10 && t3.tail_m == 16 && t3.tail_n == 33;
  // a very large shape plans in well under a millisecond
  const auto t0 = std::chrono::steady_clock::now();
  volatile int sink = 0;
  for (int i = 0; i < 10; ++i) sink += tb::plan::plan_prefill(65536, 256, 256, 256).n_split;
  const double us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count() / 10;
  std::printf("checked=%ld mismatches=%ld plan_mismatches=%ld config1=%d/%d/%dx%d m3000=%d/%dx%d plan_65536_us=%.1f\n",
              checked, mismatches, plan_mismatches, c1.n_full, c1.n_split, c1.tail_m, c1.tail_n, t3.n_split, t3.tail_m,
              t3.tail_n, us);
  return (mismatches == 0 && plan_mismatches == 0 && c1_ok && t3_ok && us < 1000.0) ? 0 : 1;
}
