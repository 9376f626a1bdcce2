// Host-only check of the split-K decode planner (bnr::plan_decode), linked
// against libbitnet_hip.so; no GPU is touched.  Prints "ok" or the first
// violated property.
//
// Properties, over 5000+ seeded launches (1..64 sequences, 1..8192 rows,
// 1..64 kv heads, the default 256-CU configuration and tuning overrides):
//  - rows_per_split == 16 * rpg * passes, 1 <= rpg <= 8, passes >= 1;
//  - split_off[b+1] - split_off[b] == ceil(len_b / rows) and max_splits is
//    the largest of them (at most kMaxSplits);
//  - the two-launch merge only with rpg 1, 2, 4 or 8;
//  - launches of at least large_wgs 64-row workgroups (batch > 1) take the
//    two-launch merge with rpg 4; a single sequence never does;
//  - a small launch fits target_wgs workgroups whenever one split per
//    (sequence, kv head) does, and its plan is the cheapest such split by
//    the planner's time estimate (exhaustive search over rpg and passes);
//  - the plans of the 2B shape (5 kv heads, one sequence) at the contexts
//    the estimate was fitted on.
#include <cstdio>
#include <cstdlib>
#include <random>

#include "bnr_internal.h"

using namespace bnr;

static int fail(const char *what, int L, int batch, int n_kv) {
  std::printf("FAIL %s (first len %d, batch %d, n_kv %d)\n", what, L, batch, n_kv);
  return 1;
}

static long long cost(int rows, int splits, int passes) {
  return 35LL * rows + 61LL * splits + 474LL * (passes - 1);
}

static int check(const DecodePlanConfig &c, const int *lens, int batch, int n_kv) {
  DecodeArgs a{};
  plan_decode(c, lens, batch, n_kv, a);
  const int L0 = lens[0];
  if (a.rpg < 1 || a.rpg > 8 || a.passes < 1) return fail("rpg/passes range", L0, batch, n_kv);
  const int rows = a.rows_per_split;
  if (rows != 16 * a.rpg * a.passes) return fail("rows = 16*rpg*passes", L0, batch, n_kv);
  if (a.batch != batch || a.split_off[0] != 0) return fail("batch / split_off[0]", L0, batch, n_kv);
  int mx = 1, max_len = 1;
  long long wgs = 0, wgs4 = 0;
  for (int b = 0; b < batch; ++b) {
    const int ns = (lens[b] + rows - 1) / rows;
    if (a.split_off[b + 1] - a.split_off[b] != ns) return fail("split counts", L0, batch, n_kv);
    mx = ns > mx ? ns : mx;
    max_len = lens[b] > max_len ? lens[b] : max_len;
    wgs += ns;
    wgs4 += (lens[b] + 63) / 64;
  }
  wgs *= n_kv;
  wgs4 *= n_kv;
  if (a.max_splits != mx || mx > kMaxSplits) return fail("max_splits", L0, batch, n_kv);
  if (!a.merge_inline && (a.rpg & (a.rpg - 1))) return fail("two-launch rpg", L0, batch, n_kv);
  const bool large = batch > 1 && wgs4 >= c.large_wgs;
  if (c.merge_mode < 0 && a.merge_inline != (large ? 0 : 1)) return fail("merge choice", L0, batch, n_kv);
  if (large && c.force_rpg == 0 && a.rpg != 4) return fail("large rpg", L0, batch, n_kv);
  if (!large && c.force_rpg == 0) {
    const bool feasible = (long long)batch * n_kv <= c.target_wgs;
    if (feasible && wgs > c.target_wgs) return fail("small launch over target", L0, batch, n_kv);
    if (feasible) {
      long long best = -1;
      for (int p = c.min_passes; p <= (max_len + 15) / 16 && p <= 4096; ++p)
        for (int r = 1; r <= 8; ++r) {
          if (!a.merge_inline && (r & (r - 1))) continue;
          const int R = 16 * r * p;
          long long w = 0;
          int sp = 0;
          for (int b = 0; b < batch; ++b) {
            const int ns = (lens[b] + R - 1) / R;
            w += ns;
            sp = ns > sp ? ns : sp;
          }
          if (w * n_kv > c.target_wgs) continue;
          const long long cst = cost(R, sp, p);
          if (best < 0 || cst < best) best = cst;
        }
      if (cost(rows, mx, a.passes) != best) return fail("not the cheapest split", L0, batch, n_kv);
    }
  }
  return 0;
}

int main() {
  const DecodePlanConfig def{256, 256, 1024, 0, 1, -1};
  // The 2B shape, one sequence: the plans the estimate picks.
  struct Want { int L, rpg, passes; };
  const Want want[] = {{512, 2, 1}, {2048, 4, 1}, {3072, 4, 1}, {4096, 6, 1}, {6144, 8, 1},
                       {8192, 6, 2}, {32768, 7, 6}};
  for (const Want &w : want) {
    DecodeArgs a{};
    plan_decode(def, &w.L, 1, 5, a);
    if (a.rpg != w.rpg || a.passes != w.passes || !a.merge_inline) {
      std::printf("FAIL plan at L=%d: rpg %d passes %d (want %d x %d)\n", w.L, a.rpg, a.passes,
                  w.rpg, w.passes);
      return 1;
    }
  }
  std::mt19937 rng(0xB17E);
  const DecodePlanConfig cfgs[] = {def,
                                   {256, 256, 1024, 0, 2, -1},   // at least two passes
                                   {256, 128, 1024, 0, 1, -1},   // a smaller target
                                   {256, 256, 1024, 0, 1, 0},    // forced two-launch merge
                                   {256, 256, 1024, 6, 1, -1},   // forced rpg
                                   {128, 128, 512, 0, 1, -1}};   // a smaller device
  int n = 0;
  for (const DecodePlanConfig &c : cfgs) {
    for (int t = 0; t < 900; ++t) {
      const int batch = t < 300 ? 1 : 1 + (int)(rng() % 64);
      const int n_kv = 1 + (int)(rng() % (t % 3 == 0 ? 64 : 8));
      int lens[kMaxBatchPerLaunch];
      for (int b = 0; b < batch; ++b) lens[b] = 1 + (int)(rng() % (t % 5 == 0 ? 8192 : 4096));
      if (check(c, lens, batch, n_kv)) return 1;
      ++n;
    }
  }
  std::printf("ok %d launches\n", n);
  return 0;
}
