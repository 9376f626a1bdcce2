// Checks the bound on the chunked-prefill workspace: over seeded launch
// shapes on caches of 96 to 8192 rows with 1 to 8 kv heads, every chunk size
// the planner picks (plain or balanced chunks, 32-query tiles or 16-query
// halves, either forced or the planner's choice) keeps the launch's (kv head,
// item) pairs within prefill_item_budget(cap, n_kv), which is what the
// workspace is sized for; the budget is four items per query tile of the
// cache, at most kPrefillMaxPlannedItems, and never falls as the cache
// grows.  Prints "ok <launches>" or the first failing case.
#include <cstdio>
#include <random>

#include "bnr_internal.h"

using namespace bnr;

int main() {
  const long long caps[] = {96, 512, 1000, 2048, 4096, 8192};
  const int kvs[] = {1, 2, 5, 8};
  std::mt19937 rng(20261202);
  int launches = 0;
  for (long long cap : caps) {
    for (int n_kv : kvs) {
      const long long tiles = (cap + 31) / 32;
      const long long budget = prefill_item_budget(cap, n_kv);
      const long long want = std::min(4LL * n_kv * tiles, kPrefillMaxPlannedItems);
      if (budget != want) {
        std::printf("FAIL budget %lld != %lld (cap %lld, n_kv %d)\n", budget, want, cap, n_kv);
        return 1;
      }
      if (prefill_item_budget(cap + 32, n_kv) < budget) {
        std::printf("FAIL budget falls past cap %lld (n_kv %d)\n", cap, n_kv);
        return 1;
      }
      const int reps = cap >= 4096 ? 6 : 14;
      for (int r = 0; r < reps; ++r) {
        // Token counts up to the whole cache, the start below the token count
        // (the launches that take key chunks), unaligned as often as not.
        const int n = 1 + (int)(rng() % (unsigned)cap);
        const int room = (int)cap - n;
        const int start = room > 0 ? (int)(rng() % (unsigned)(std::min(room, n) + 1)) : 0;
        for (int pref = -1; pref <= 1; ++pref) {
          const PrefillChoice pc = plan_prefill_chunk(n, start, n_kv, 256, pref, pref, cap);
          const int ct = pc.tiles, bal = pc.balanced;
          const PrefillPlan p = prefill_plan(n, start, ct);
          ++launches;
          if (ct < 1 || (bal != 0 && bal != 1) || (pref >= 0 && p.split && bal != pref) ||
              (pref >= 0 && pc.q16 != pref)) {
            std::printf("FAIL pick ct %d bal %d (cap %lld n_kv %d n %d start %d pref %d)\n", ct, bal,
                        cap, n_kv, n, start, pref);
            return 1;
          }
          if (p.split && (long long)n_kv * p.n_items > budget) {
            std::printf("FAIL %lld items > budget %lld (cap %lld n_kv %d n %d start %d ct %d)\n",
                        (long long)n_kv * p.n_items, budget, cap, n_kv, n, start, ct);
            return 1;
          }
        }
      }
    }
  }
  std::printf("ok %d\n", launches);
  return 0;
}
