// Checks the prefill work-item order (prefill_map / prefill_order, and
// pf_bal_map for balanced chunks) over many shapes: every (query tile,
// chunk) pair appears exactly once, nch and the partial-state slot base
// match the direct count, in the longest-first orders chunk lengths never
// increase, and a tile's balanced chunks cover its key tiles once, in order,
// with lengths differing by at most one.  Prints "ok <shapes>" or the first
// failing case.
#include <algorithm>
#include <cstdio>
#include <vector>

#include "bnr_internal.h"

using namespace bnr;

static int check(int n_tokens, int start_pos, int ct) {
  PrefillArgs a{};
  a.n_tokens = n_tokens;
  a.start_pos = start_pos;
  a.n_qtiles = (n_tokens + 31) / 32;
  a.chunk_tiles = ct;
  prefill_order(a);
  const int nqt = a.n_qtiles, last_row = start_pos + n_tokens - 1;
  std::vector<int> nt(nqt), nchs(nqt), base(nqt);
  int total = 0;
  for (int qt = 0; qt < nqt; ++qt) {
    nt[qt] = std::min(start_pos + qt * 32 + 31, last_row) / 32 + 1;
    nchs[qt] = (nt[qt] + ct - 1) / ct;
    base[qt] = total;
    total += nchs[qt];
  }
  if (total != prefill_plan(n_tokens, start_pos, ct).n_items) return 1;
  std::vector<int> seen(total, 0);
  int prev_len = 1 << 30;
  for (int y = 0; y < total; ++y) {
    int qt = -1, ch = -1, nch = -1, b = -1;
    prefill_map(a, y, qt, ch, nch, b);
    if (qt < 0 || qt >= nqt || ch < 0 || ch >= nchs[qt]) return 2;
    if (nch != nchs[qt] || b != base[qt]) return 3;
    if (seen[b + ch]++) return 4;
    const int len = std::min(nt[qt], (ch + 1) * ct) - ch * ct;
    if (a.lpt && len > prev_len) return 5;
    prev_len = len;
  }
  // balanced chunks: the same items in the order of pf_bal_map
  PrefillArgs b = a;
  b.balanced = 1;
  prefill_order(b);
  if (b.balanced != a.lpt) return 6;  // allowed exactly where the lpt order is
  if (!b.balanced) return 0;
  std::fill(seen.begin(), seen.end(), 0);
  std::vector<int> next_kt(nqt, 0);
  prev_len = 1 << 30;
  for (int y = 0; y < total; ++y) {
    int qt = -1, ch = -1, nch = -1;
    pf_bal_map(b, y, qt, ch, nch);
    if (qt < 0 || qt >= nqt || ch < 0 || ch >= nchs[qt] || nch != nchs[qt]) return 7;
    if (seen[base[qt] + ch]++) return 8;
    int kt0 = -1, len = -1;
    pf_bal_range(nt[qt], nch, ch, kt0, len);
    if (len > prev_len || len < 1 || len > ct) return 9;
    if (len < nt[qt] / nch || len > nt[qt] / nch + 1) return 10;
    // chunks of one tile appear in order within a length, so check coverage
    // from the ranges themselves: ch's range starts where ch-1's ended
    int pk = 0, pl = 0;
    if (ch > 0) pf_bal_range(nt[qt], nch, ch - 1, pk, pl);
    if (kt0 != (ch > 0 ? pk + pl : 0)) return 11;
    if (ch == nch - 1 && kt0 + len != nt[qt]) return 12;
    prev_len = len;
  }
  return 0;
}

int main() {
  int shapes = 0;
  const int ns[] = {1, 2, 31, 32, 33, 64, 100, 255, 256, 257, 1000, 1024, 2048, 2049, 4096};
  const int starts[] = {0, 1, 5, 31, 32, 33, 200, 1000, 1536, 4095};
  for (int n : ns)
    for (int st : starts)
      for (int ct : {1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 16, 24, 32, 48, 64, 100, kPrefillNoSplit}) {
        const int r = check(n, st, ct);
        ++shapes;
        if (r) {
          std::printf("fail %d: n_tokens %d start_pos %d chunk_tiles %d\n", r, n, st, ct);
          return 1;
        }
      }
  std::printf("ok %d\n", shapes);
  return 0;
}
