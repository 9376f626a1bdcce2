// Host-only check of the split-K decode planner (bnr::plan_decode), linked
// against libbitnet_hip.so; no GPU is touched.  Prints "ok" or the first
// violated property.
//
// Properties, over 10800 seeded launches (1..64 sequences, 1..8192 rows,
// 1..64 kv heads, the default 256-CU configuration and tuning overrides):
//  - every plan: 1 <= rpg <= 8, passes >= 1, the split counts are
//    ceil(len_b / rows_per_split), max_splits is the largest (at most
//    kMaxSplits);
//  - reference merge (the default): rows_per_split fits its passes of
//    4*waves*rpg rows (small launches: 8 waves and rpg <= 3, or 4 waves and
//    rpg <= 6 -- configured, or by default for sequences of at most
//    kRefWaves4Rows rows; 4 waves and rpg <= 3 (splits of at most
//    kLargeRpg3Rows rows) or 4 for large
//    launches), at least 16 rows; the launch fits its target (one workgroup
//    per CU, eight for large launches) whenever one split per (sequence,
//    kv head) does, and no smaller split size would fit it;
//  - ticket / two-launch merges (forced): rows_per_split == 16 * rpg *
//    passes; the two-launch merge only with rpg 1, 2, 4 or 8; launches of at
//    least large_wgs 64-row workgroups (batch > 1) take it with rpg 4, a
//    single sequence never does; a small launch fits target_wgs workgroups
//    whenever one split per (sequence, kv head) does, at the cheapest such
//    split by the planner's time estimate (exhaustive search);
//  - the plans of the 2B shape (5 kv heads, one sequence) at 512..32768.
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

static long long wgs_at(const int *lens, int batch, int n_kv, int rows) {
  long long w = 0;
  for (int b = 0; b < batch; ++b) w += (lens[b] + rows - 1) / rows;
  return w * n_kv;
}

static int check(const DecodePlanConfig &c, const int *lens, int batch, int n_kv) {
  DecodeArgs a{};
  plan_decode(c, lens, batch, n_kv, a);
  const int L0 = lens[0];
  if (a.rpg < 1 || a.rpg > 8 || a.passes < 1) return fail("rpg/passes range", L0, batch, n_kv);
  const int rows = a.rows_per_split;
  if (a.batch != batch || a.split_off[0] != 0) return fail("batch / split_off[0]", L0, batch, n_kv);
  int mx = 1, max_len = 1;
  long long wgs4 = 0;
  for (int b = 0; b < batch; ++b) {
    const int ns = (lens[b] + rows - 1) / rows;
    if (a.split_off[b + 1] - a.split_off[b] != ns) return fail("split counts", L0, batch, n_kv);
    mx = ns > mx ? ns : mx;
    max_len = lens[b] > max_len ? lens[b] : max_len;
    wgs4 += (lens[b] + 63) / 64;
  }
  const long long wgs = wgs_at(lens, batch, n_kv, rows);
  wgs4 *= n_kv;
  if (a.max_splits != mx || mx > kMaxSplits) return fail("max_splits", L0, batch, n_kv);
  const bool large = batch > 1 && wgs4 >= c.large_wgs;

  if (c.merge_mode < 0 || c.merge_mode == 2) {
    if (!a.merge_ref || !a.merge_inline) return fail("reference merge chosen", L0, batch, n_kv);
    if (rows < 16) return fail("at least 16 rows", L0, batch, n_kv);
    const int small_waves =
        c.ref_waves == 4 || c.ref_waves == 8 ? c.ref_waves : (max_len <= kRefWaves4Rows ? 4 : 8);
    const int waves = large ? 4 : small_waves;
    const int nrg = 4 * waves;  // row groups of a workgroup
    if (a.ref_waves != waves) return fail("reference waves", L0, batch, n_kv);
    if (!(nrg * a.rpg * (a.passes - 1) < rows && rows <= nrg * a.rpg * a.passes))
      return fail("rows fit the passes", L0, batch, n_kv);
    if (c.force_rpg == 0 && a.rpg > (large ? 4 : waves == 8 ? 3 : 6))
      return fail("reference rpg bound", L0, batch, n_kv);
    if (c.ref_rows > 0) return 0;
    const long long target = large ? 8LL * c.target_wgs : c.target_wgs;
    const bool feasible = (long long)batch * n_kv <= target;
    if (feasible && mx < kMaxSplits) {
      if (wgs > target) return fail("reference launch over target", L0, batch, n_kv);
      // no smaller split size (at least 16 rows) fits the target
      int smallest = rows;
      for (int r = rows - 1; r >= 16; --r) {
        if (wgs_at(lens, batch, n_kv, r) > target) break;
        smallest = r;
      }
      const int r0 = smallest;
      const int rpg = a.rpg;
      // large launches: at most 3 rows per row group up to kLargeRpg3Rows rows
      if (large && c.force_rpg == 0) {
        const int cap = r0 <= kLargeRpg3Rows ? 3 : 4;
        const int want = (r0 + nrg - 1) / nrg < cap ? (r0 + nrg - 1) / nrg : cap;
        if (rpg != want) return fail("large reference rpg", L0, batch, n_kv);
      }
      // the plan is the smallest fitting size rounded up to whole passes
      const int passes = (r0 + nrg * rpg - 1) / (nrg * rpg);
      if (rows != nrg * rpg * passes && rows != r0)
        return fail("reference split is not the smallest fitting one", L0, batch, n_kv);
    }
    return 0;
  }

  if (a.merge_ref) return fail("reference merge not forced", L0, batch, n_kv);
  if (rows != 16 * a.rpg * a.passes) return fail("rows = 16*rpg*passes", L0, batch, n_kv);
  if (!a.merge_inline && (a.rpg & (a.rpg - 1))) return fail("two-launch rpg", L0, batch, n_kv);
  if (c.merge_mode == 1 && !a.merge_inline) return fail("forced ticket merge", L0, batch, n_kv);
  if (c.merge_mode == 0 && a.merge_inline) return fail("forced two-launch merge", L0, batch, n_kv);
  if (large && c.force_rpg == 0 && a.rpg != 4) return fail("large rpg", L0, batch, n_kv);
  if (!large && c.force_rpg == 0) {
    const bool feasible = (long long)batch * n_kv <= c.target_wgs;
    if (feasible && wgs > c.target_wgs) return fail("small launch over target", L0, batch, n_kv);
    if (feasible) {
      long long best = -1;
      const int p_max = (max_len + 15) / 16 > c.min_passes ? (max_len + 15) / 16 : c.min_passes;
      for (int p = c.min_passes; p <= p_max && p <= 4096; ++p)
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
  const DecodePlanConfig def{256, 256, 1024, 0, 1, -1, -1, 0, 0};
  const DecodePlanConfig ticket{256, 256, 1024, 0, 1, 1, -1, 0, 8};
  // The 2B shape, one sequence: the plans of both merges.
  struct Want { int L, rpg, passes, rows; };
  const Want want_ref[] = {{512, 1, 1, 16},   {2048, 2, 1, 64},  {4096, 3, 1, 96},
                           {8192, 3, 2, 192}, {32768, 3, 7, 672}};
  for (const Want &w : want_ref) {
    DecodeArgs a{};
    plan_decode(def, &w.L, 1, 5, a);
    if (a.rpg != w.rpg || a.passes != w.passes || a.rows_per_split != w.rows || !a.merge_ref) {
      std::printf("FAIL reference plan at L=%d: rpg %d passes %d rows %d (want %d x %d, %d)\n",
                  w.L, a.rpg, a.passes, a.rows_per_split, w.rpg, w.passes, w.rows);
      return 1;
    }
  }
  const Want want_ticket[] = {{512, 2, 1, 32},   {2048, 4, 1, 64},  {3072, 4, 1, 64},
                              {4096, 6, 1, 96},  {6144, 8, 1, 128}, {8192, 6, 2, 192},
                              {32768, 7, 6, 672}};
  for (const Want &w : want_ticket) {
    DecodeArgs a{};
    plan_decode(ticket, &w.L, 1, 5, a);
    if (a.rpg != w.rpg || a.passes != w.passes || !a.merge_inline || a.merge_ref) {
      std::printf("FAIL ticket plan at L=%d: rpg %d passes %d (want %d x %d)\n", w.L, a.rpg,
                  a.passes, w.rpg, w.passes);
      return 1;
    }
  }
  std::mt19937 rng(0xB17E);
  const DecodePlanConfig cfgs[] = {def,
                                   {256, 128, 1024, 0, 1, -1, -1, 0, 4},   // a smaller target
                                   {256, 256, 1024, 3, 1, -1, -1, 0, 4},   // forced rpg
                                   {256, 256, 1024, 0, 1, -1, -1, 200, 4}, // forced split size
                                   {128, 128, 512, 0, 1, -1, -1, 0, 4},    // a smaller device
                                   {256, 256, 1024, 0, 1, -1, -1, 0, 4},   // four waves
                                   {256, 256, 1024, 0, 1, -1, -1, 0, 8},   // eight waves
                                   ticket,
                                   {256, 256, 1024, 0, 2, 1, -1, 0, 4},    // ticket, at least two passes
                                   {256, 128, 1024, 0, 1, 1, -1, 0, 4},    // ticket, a smaller target
                                   {256, 256, 1024, 0, 1, 0, -1, 0, 4},    // forced two-launch merge
                                   {256, 256, 1024, 6, 1, 1, -1, 0, 4}};  // ticket, forced rpg
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
