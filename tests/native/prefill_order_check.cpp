// Checks the prefill work-item order (prefill_map / prefill_order) over many
// shapes: every (query tile, chunk) pair appears exactly once, nch and the
// partial-state slot base match the direct count, and in the longest-first
// order chunk lengths never increase.  Prints "ok <shapes>" or the first
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
