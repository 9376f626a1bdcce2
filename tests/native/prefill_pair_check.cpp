// Checks the paired plans of the 16-query prefill (bnr::plan_prefill_pairs)
// over seeded launch shapes (1 to 2100 tokens, 0 to 5000 cached rows, 1 to 8
// kv heads, 80 and 256 CUs), decoding every piece word the way the kernel
// does: each 16-query unit's key tiles 0 .. nk - 1 are covered exactly once
// by its pieces, whose chunk indices run 0 .. nch - 1 in key order; a bin
// holds at most two pieces, the longer first, within tau key tiles; the
// workgroups of the 1-D grid reach every (bin, piece, kv head) once; the
// split query tiles' partial-state slots are disjoint, shared by a tile's two
// halves and within n_slots, and n_slots * n_kv fits the item budget.  Also
// pins the plan of the 30-layer stack's shape (1024 tokens, 5 kv heads, 256
// CUs: 51 bins, none slower than 56 us in the planner's CU model -- the
// chain packing's slowest takes 58.6 us there).  Prints "ok <plans>" or the
// first failing case.
#include <cstdio>
#include <random>
#include <vector>

#include "bnr_internal.h"

using namespace bnr;

namespace {

struct Piece {
  int kt0, len, qt, half, ch, nch, base;
};

Piece decode(const unsigned w[2]) {
  Piece p;
  p.kt0 = (int)(w[0] & 0xFFFFu);
  p.qt = (int)((w[0] >> 16) & 0x7FFFu);
  p.half = (int)(w[0] >> 31);
  p.len = (int)(w[1] & 255u);
  p.ch = (int)((w[1] >> 8) & 255u);
  p.nch = (int)((w[1] >> 16) & 255u);
  p.base = (int)(w[1] >> 24);
  return p;
}

bool check(int n, int start, int n_kv, int n_cu, long long budget, const PairPlan &pl,
           const char *&why) {
  const int nu = (n + 15) / 16, nqt = (n + 31) / 32;
  const int max_bins = std::min(n_cu / n_kv, kMaxPairBins);
  const long long last = (long long)start + n - 1;
  if (pl.bins < 1 || pl.bins > max_bins) return why = "bins", false;
  if (pl.n_slots < 0 || pl.n_slots > 256 || (long long)pl.n_slots * n_kv > budget)
    return why = "slots", false;
  // the kernel's grid mapping reaches each (bin, piece, kv head) once
  std::vector<int> seen((size_t)pl.bins * 2 * n_kv, 0);
  for (int i = 0; i < 2 * n_cu; ++i) {
    const int cu = i % n_cu, slot = i / n_cu;
    const int cux = n_cu % 8 == 0 ? (cu % 8) * (n_cu / 8) + cu / 8 : cu;
    const int h = cux / pl.bins, bin = cux % pl.bins;
    if (h >= n_kv) continue;
    ++seen[((size_t)bin * 2 + slot) * n_kv + h];
  }
  for (int v : seen)
    if (v != 1) return why = "grid mapping", false;
  // coverage of every unit's key tiles, chunk order
  std::vector<std::vector<Piece>> units((size_t)nu);
  long long S = 0;
  for (int b = 0; b < pl.bins; ++b) {
    int sum = 0, lens[2];
    for (int k = 0; k < 2; ++k) {
      const Piece p = decode(pl.piece[2 * b + k]);
      lens[k] = p.len;
      if (p.len == 0) {
        if (pl.piece[2 * b + k][1] != 0 || k == 0) return why = "empty slot", false;
        continue;
      }
      const int u = 2 * p.qt + p.half;
      if (p.qt >= nqt || u >= nu) return why = "unit range", false;
      units[(size_t)u].push_back(p);
      sum += p.len;
    }
    if (lens[1] > lens[0]) return why = "longer piece second", false;
    if (sum > pl.tau) return why = "bin over tau", false;
  }
  for (int b = pl.bins; b < kMaxPairBins; ++b)
    if (pl.piece[2 * b][1] || pl.piece[2 * b + 1][1]) return why = "piece past bins", false;
  std::vector<int> slot_owner(256, -1);
  for (int u = 0; u < nu; ++u) {
    const int nk = (int)(std::min<long long>(start + 16LL * u + 15, last) / 32 + 1);
    S += nk;
    std::vector<Piece> &ps = units[(size_t)u];
    if (ps.empty()) return why = "unit missing", false;
    std::vector<int> cover((size_t)nk, 0);
    for (const Piece &p : ps) {
      if (p.nch != (int)ps.size() || p.ch < 0 || p.ch >= p.nch) return why = "nch", false;
      if (p.kt0 + p.len > nk) return why = "piece past the unit's keys", false;
      for (int t = p.kt0; t < p.kt0 + p.len; ++t) ++cover[(size_t)t];
      for (const Piece &o : ps)
        if ((o.kt0 < p.kt0) != (o.ch < p.ch)) return why = "chunk order", false;
      if (p.nch > 1) {
        if (p.base + p.nch > pl.n_slots) return why = "slot past n_slots", false;
        for (int c = 0; c < p.nch; ++c) {
          int &own = slot_owner[(size_t)(p.base + c)];
          if (own >= 0 && own != p.qt) return why = "slot shared by two query tiles", false;
          own = p.qt;
        }
        // the other half of the query tile, when split, uses the same base
        const int v = u ^ 1;
        if (v < nu && !units[(size_t)v].empty() && units[(size_t)v][0].nch > 1 &&
            units[(size_t)v][0].base != p.base)
          return why = "halves' bases differ", false;
      } else if (p.base != 0) {
        return why = "base of an unsplit unit", false;
      }
    }
    for (int c : cover)
      if (c != 1) return why = "key tile coverage", false;
  }
  if (pl.tau < (int)((S + max_bins - 1) / max_bins)) return why = "tau below the mean load", false;
  return true;
}

}  // namespace

int main() {
  int plans = 0;
  {
    PairPlan pl;
    const long long budget = prefill_item_budget(1280, 5);
    if (!plan_prefill_pairs(1024, 0, 5, 256, budget, pl) || pl.bins != 51 || pl.model_us > 56.0) {
      std::printf("FAIL stack shape: bins %d model %.2f us\n", pl.bins, pl.model_us);
      return 1;
    }
    const char *why = "";
    if (!check(1024, 0, 5, 256, budget, pl, why)) {
      std::printf("FAIL stack shape: %s\n", why);
      return 1;
    }
    ++plans;
  }
  std::mt19937 rng(20261202);
  const int kvs[] = {1, 2, 3, 5, 8};
  const int cus[] = {80, 256, 100};
  for (int n_cu : cus) {
    for (int n_kv : kvs) {
      for (int r = 0; r < 160; ++r) {
        const int n = 1 + (int)(rng() % 2100u);
        const int start = r % 3 == 0 ? 0 : (int)(rng() % 5001u);
        const long long cap = start + n + (long long)(rng() % 300u);
        const long long budget = prefill_item_budget(cap, n_kv);
        PairPlan pl;
        if (!plan_prefill_pairs(n, start, n_kv, n_cu, budget, pl)) {
          // only shapes with more units than two per bin, or a bin load past 255
          const int max_bins = std::min(n_cu / n_kv, kMaxPairBins);
          const int nu = (n + 15) / 16;
          if (nu <= 2 * max_bins && (start + n) / 32 + 1 <= 255 / 2) {
            std::printf("FAIL no plan for n %d start %d n_kv %d n_cu %d\n", n, start, n_kv, n_cu);
            return 1;
          }
          continue;
        }
        const char *why = "";
        if (!check(n, start, n_kv, n_cu, budget, pl, why)) {
          std::printf("FAIL %s (n %d start %d n_kv %d n_cu %d)\n", why, n, start, n_kv, n_cu);
          return 1;
        }
        ++plans;
      }
    }
  }
  std::printf("ok %d\n", plans);
  return 0;
}
