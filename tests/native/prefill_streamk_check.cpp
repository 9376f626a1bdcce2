// Checks the stream-K prefill runs (prefill_streamk_units, sk_seg, sk_u0,
// sk_wg_of) over many launch shapes and workgroup counts, walking every run
// as the kernel does: each (kv head, query tile, key tile) unit is taken by
// exactly one segment of exactly one run; segments stay inside one query
// tile and carry its key-tile count; a query tile's parts are the runs
// sk_wg_of names, one segment each; the partial-state slots the merge
// derives (2w or 2w+1) are distinct per query tile and below 2P, and a
// whole query tile is one run's segment.  Prints "ok <cases>" or the first
// failing case.
#include <cstdio>
#include <map>
#include <set>
#include <vector>

#include "bnr_internal.h"

using namespace bnr;

static int fail(const char *what, int n, int sp, int nkv, int P) {
  std::printf("FAIL %s (n_tokens %d, start %d, n_kv %d, workgroups %d)\n", what, n, sp, nkv, P);
  return 1;
}

static int check(int n_tokens, int start_pos, int n_kv, int P) {
  PrefillArgs a{};
  a.n_tokens = n_tokens;
  a.start_pos = start_pos;
  a.n_kv = n_kv;
  a.n_qtiles = (n_tokens + 31) / 32;
  prefill_streamk_units(a);
  const int nqt = a.n_qtiles, last_row = start_pos + n_tokens - 1;
  std::vector<long long> qstart(nqt);
  std::vector<int> nk(nqt);
  long long T = 0;
  for (int qt = 0; qt < nqt; ++qt) {
    nk[qt] = std::min(start_pos + qt * 32 + 31, last_row) / 32 + 1;
    qstart[qt] = T;
    T += nk[qt];
  }
  if (a.sk_per_head != T || a.sk_units != T * n_kv) return fail("unit count", n_tokens, start_pos, n_kv, P);
  if (P > a.sk_units) P = (int)a.sk_units;
  const long long U = a.sk_units;
  std::vector<unsigned char> seen(U, 0);
  // per (kv head, query tile): runs that hold a part of it, and their slots
  std::map<std::pair<int, int>, std::vector<int>> parts, slots;
  long long prev_end = 0;
  for (int w = 0; w < P; ++w) {
    const long long u0 = sk_u0(w, U, P), u1 = sk_u0(w + 1, U, P);
    if (u0 != prev_end || u1 <= u0) return fail("runs not contiguous or empty", n_tokens, start_pos, n_kv, P);
    prev_end = u1;
    for (long long u = u0; u < u1;) {
      const SkSeg sg = sk_seg(a, u, u1);
      if (sg.h < 0 || sg.h >= n_kv || sg.qt < 0 || sg.qt >= nqt) return fail("segment out of range", n_tokens, start_pos, n_kv, P);
      if (sg.nk != nk[sg.qt]) return fail("key-tile count", n_tokens, start_pos, n_kv, P);
      if (sg.qstart != sg.h * T + qstart[sg.qt] || u != sg.qstart + sg.kt0)
        return fail("segment start", n_tokens, start_pos, n_kv, P);
      if (sg.kt0 < 0 || sg.kt1 <= sg.kt0 || sg.kt1 > sg.nk) return fail("segment tiles", n_tokens, start_pos, n_kv, P);
      if (sg.kt1 != sg.nk && u + (sg.kt1 - sg.kt0) != u1) return fail("segment ends early", n_tokens, start_pos, n_kv, P);
      for (long long x = u; x < u + (sg.kt1 - sg.kt0); ++x) {
        if (seen[x]) return fail("unit taken twice", n_tokens, start_pos, n_kv, P);
        seen[x] = 1;
      }
      const std::pair<int, int> key{sg.h, sg.qt};
      const bool whole = sg.kt0 == 0 && sg.kt1 == sg.nk;
      const int wf = sk_wg_of(sg.qstart, U, P), wl = sk_wg_of(sg.qstart + sg.nk - 1, U, P);
      if (w < wf || w > wl) return fail("run outside the tile's parts", n_tokens, start_pos, n_kv, P);
      if (whole != (wf == wl)) return fail("whole tile vs parts", n_tokens, start_pos, n_kv, P);
      if (!whole) {
        parts[key].push_back(w);
        slots[key].push_back(2 * w + (sk_u0(w, U, P) >= sg.qstart ? 0 : 1));
      }
      u += sg.kt1 - sg.kt0;
    }
  }
  if (prev_end != U) return fail("runs do not cover the units", n_tokens, start_pos, n_kv, P);
  for (long long x = 0; x < U; ++x)
    if (!seen[x]) return fail("unit not taken", n_tokens, start_pos, n_kv, P);
  std::set<int> all_slots;
  for (auto &kv : parts) {
    const auto &ws = kv.second;
    const long long qs = kv.first.first * T + qstart[kv.first.second];
    const int wf = sk_wg_of(qs, U, P), wl = sk_wg_of(qs + nk[kv.first.second] - 1, U, P);
    if ((int)ws.size() != wl - wf + 1) return fail("part count != ticket count", n_tokens, start_pos, n_kv, P);
    for (int i = 0; i < (int)ws.size(); ++i)
      if (ws[i] != wf + i) return fail("parts are not runs wf..wl", n_tokens, start_pos, n_kv, P);
    for (int sl : slots[kv.first]) {
      if (sl < 0 || sl >= 2 * P) return fail("slot out of range", n_tokens, start_pos, n_kv, P);
      if (!all_slots.insert(sl).second) return fail("slot shared", n_tokens, start_pos, n_kv, P);
    }
  }
  return 0;
}

int main() {
  const int tokens[] = {1, 2, 31, 32, 33, 64, 100, 511, 512, 1000, 1024, 2048, 3001, 4096};
  const int starts[] = {0, 1, 31, 32, 200, 1536, 3000};
  const int kvs[] = {1, 5, 8};
  const int wgs[] = {1, 7, 64, 255, 256, 512, 1000};
  int n = 0;
  for (int t : tokens)
    for (int sp : starts)
      for (int kv : kvs)
        for (int P : wgs) {
          if (check(t, sp, kv, P)) return 1;
          ++n;
        }
  std::printf("ok %d\n", n);
  return 0;
}
