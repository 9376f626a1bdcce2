// Host-side planning of chunked prefill launches: the dispatch replay that
// scores a key-chunk size, the planner that picks one per launch shape, and
// the bound on the partial-state workspace those picks can need on a cache
// of a given capacity.  Pure functions of the shape and the CU count; no
// GPU is touched, so host-only checks link them directly.
#include <algorithm>
#include <vector>

#include "bnr_internal.h"

namespace bnr {

// Fitted to graph-timed MI355X spans of 12 shapes (256 to 3072 tokens, 0 to
// 3000 cached rows) x 12 chunk sizes of the 16-query kernel, the 1024- and
// 2048-token prefills from an empty cache weighted 5x: the planner's pick is
// the best measured configuration at 7 of the 12 shapes, within 5 % at 3
// more and within 12 % at all, where the 32-query kernel alone is 2-54 %
// slower than the best at 9 of them.
double g_pf16_fixed = 0.40, g_pf16_tile = 0.52, g_pf16_merge = 0.05, g_pf16_margin = 0.99;

// Prefill key-range chunking.  The planner replays the launch's dispatch for
// each candidate chunk size and keeps the shortest span.  Workgroups go to
// the XCDs round-robin (WG i to XCD i % 8), so one XCD sees every 8th
// workgroup of the dispatch order and the XCDs finish together; the replay
// follows XCD 0 alone.  An XCD places a workgroup on a CU with a free slot
// (two per CU at this kernel's register and LDS use), an idle CU first, and
// a CU's workgroups share it: one alone runs a 32-key tile in time 1, two
// side by side each take kShared.  A workgroup's work is its key tiles plus
// a fixed cost (queries and first tile loaded, outputs stored), plus a
// partial-state store when its query tile is split; the last chunk of a
// split tile then reads the others' partials.  The items come in the
// kernel's order (prefill_map, or pf_bal_map for balanced chunks).  The constants are fitted to measured
// MI355X spans over 15 shapes x 6 chunk sizes (128 to 8192 tokens, start
// 0 to 4000; a tile of 4 heads alone on a CU takes about 4 us): they keep
// the chosen chunk size within 10 % of the best measured one (2 % median).
double prefill_span(int n_tokens, int start_pos, int n_kv, int ctiles_in, int n_cu,
                    bool balanced, bool q16) {
  constexpr double kShared = 1.9, kFixed = 1.0, kStore = 0.0, kMerge = 0.1;
  // 16-query halves (prefill16_kernel): two workgroups per item, each with
  // its own fixed cost and half-height key tiles.
  const double fixed = q16 ? g_pf16_fixed : kFixed, tile = q16 ? g_pf16_tile : 1.0,
               merge = q16 ? g_pf16_merge : kMerge;
  constexpr int kXcd = 8, kSlots = 2;
  const int ncu = std::max(1, n_cu / kXcd);
  struct Cu {
    int n = 0;           // active workgroups
    double rem[kSlots];  // remaining work of each
    double tail[kSlots]; // merge work after it (split tiles)
    double t = 0.0;      // time rem[] refers to
    unsigned ver = 0;    // bumped whenever the finish times change
  };
  struct Ev {
    double t;
    int cu;
    unsigned ver;
    bool operator<(const Ev &o) const { return t > o.t; }  // min-heap
  };
  std::vector<Cu> cus((size_t)ncu);
  std::vector<Ev> heap;
  heap.reserve(256);
  auto rate = [](int n) { return n == 1 ? 1.0 : 1.0 / kShared; };
  auto advance = [&](Cu &c, double now) {
    const double r = rate(c.n);
    for (int i = 0; i < c.n; ++i) c.rem[i] -= (now - c.t) * r;
    c.t = now;
  };
  auto schedule = [&](int cu) {
    Cu &c = cus[(size_t)cu];
    ++c.ver;
    if (c.n == 0) return;
    double r = c.rem[0];
    for (int i = 1; i < c.n; ++i) r = std::min(r, c.rem[i]);
    heap.push_back(Ev{c.t + std::max(r, 0.0) / rate(c.n), cu, c.ver});
    std::push_heap(heap.begin(), heap.end());
  };
  // Free slot on the XCD: an idle CU first, else one running a single workgroup.
  auto pick = [&]() {
    int best = -1;
    for (int i = 0; i < ncu; ++i) {
      if (cus[(size_t)i].n == 0) return i;
      if (best < 0 && cus[(size_t)i].n < kSlots) best = i;
    }
    return best;
  };

  const int last_row = start_pos + n_tokens - 1;
  PrefillArgs order{};
  order.n_tokens = n_tokens;
  order.start_pos = start_pos;
  order.n_qtiles = (n_tokens + 31) / 32;
  order.chunk_tiles = std::min(std::max(ctiles_in, 1), kPrefillNoSplit);
  order.balanced = balanced;
  prefill_order(order);
  const int ctiles = order.chunk_tiles;
  const int n_items = prefill_plan(n_tokens, start_pos, ctiles).n_items;
  double now = 0.0, span = 0.0;
  long long wg = 0;
  for (int y = 0; y < n_items; ++y) {
    int qt, ch, nch, base, t;
    if (order.balanced) {
      pf_bal_map(order, y, qt, ch, nch);
      int kt0;
      pf_bal_range(std::min(start_pos + qt * 32 + 31, last_row) / 32 + 1, nch, ch, kt0, t);
    } else {
      prefill_map(order, y, qt, ch, nch, base);
      const int nk = std::min(start_pos + qt * 32 + 31, last_row) / 32 + 1;
      t = std::min(nk, (ch + 1) * ctiles) - ch * ctiles;
    }
    {
      for (int w = 0; w < (q16 ? 2 : 1) * n_kv; ++w, ++wg) {
        if (wg % kXcd != 0) continue;
        // the second half of a last tile with at most 16 queries exits at once
        const bool idle = q16 && (w & 1) && qt * 32 + 16 >= n_tokens;
        int cu;
        while ((cu = pick()) < 0) {  // wait for a slot: run to the next finish
          std::pop_heap(heap.begin(), heap.end());
          const Ev ev = heap.back();
          heap.pop_back();
          Cu &c = cus[(size_t)ev.cu];
          if (ev.ver != c.ver) continue;
          now = ev.t;
          advance(c, now);
          for (int i = 0; i < c.n;) {
            if (c.rem[i] <= 1e-9) {
              span = std::max(span, now + c.tail[i]);
              c.rem[i] = c.rem[c.n - 1];
              c.tail[i] = c.tail[c.n - 1];
              --c.n;
            } else {
              ++i;
            }
          }
          schedule(ev.cu);
        }
        Cu &c = cus[(size_t)cu];
        advance(c, now);
        c.rem[c.n] = idle ? 0.01 : fixed + t * tile + (nch > 1 ? kStore : 0.0);
        c.tail[c.n] = !idle && nch > 1 ? (nch - 1) * merge : 0.0;
        ++c.n;
        schedule(cu);
      }
    }
  }
  for (Cu &c : cus) {  // drain
    const double r = rate(c.n);
    for (int i = 0; i < c.n; ++i) {
      // the shorter of two shared workgroups ends first, the other then runs alone
      double end;
      if (c.n == 2) {
        const double a = std::min(c.rem[0], c.rem[1]), b = std::max(c.rem[0], c.rem[1]);
        end = c.t + (c.rem[i] == a ? a / r : a / r + (b - a));
      } else {
        end = c.t + c.rem[i] / r;
      }
      span = std::max(span, end + c.tail[i]);
    }
  }
  return span;
}

constexpr int kPrefillChunkCandidates[] = {3, 4, 5, 6, 7, 8, 10, 12, 14, 16, 20, 24, 32, 48, 64};


namespace {

struct PairPiece {
  int unit, kt0, len;
};
struct PairBin {
  PairPiece p[2];
  int n, sum;
};

// Pieces of the units (nk[u] key tiles each) packed into bins of at most
// two pieces and tau key tiles.  Units shorter than thr go whole, the
// longest with the shortest while both fit, else the longest alone; the
// others form one chain, longest first, cut into bins that close when full
// or when they hold two pieces.  False when a bin would exceed max_bins or
// a whole unit tau.
bool pair_pack(const std::vector<int> &nk, int tau, int thr, int max_bins,
               std::vector<PairBin> &bins) {
  bins.clear();
  std::vector<int> small, large;
  for (int u = 0; u < (int)nk.size(); ++u) (nk[u] < thr ? small : large).push_back(u);
  std::stable_sort(small.begin(), small.end(), [&](int a, int b) { return nk[a] < nk[b]; });
  std::stable_sort(large.begin(), large.end(), [&](int a, int b) { return nk[a] > nk[b]; });
  for (int i = 0, j = (int)small.size() - 1; i <= j;) {
    const int uj = small[(size_t)j];
    if (nk[uj] > tau || (int)bins.size() >= max_bins) return false;
    PairBin b{};
    b.p[b.n++] = PairPiece{uj, 0, nk[uj]};
    b.sum = nk[uj];
    if (i < j && nk[small[(size_t)i]] + nk[uj] <= tau) {
      const int ui = small[(size_t)i++];
      b.p[b.n++] = PairPiece{ui, 0, nk[ui]};
      b.sum += nk[ui];
    }
    --j;
    bins.push_back(b);
  }
  PairBin cur{};
  for (int u : large) {
    for (int k0 = 0; k0 < nk[u];) {
      const int take = std::min(nk[u] - k0, tau - cur.sum);
      cur.p[cur.n++] = PairPiece{u, k0, take};
      cur.sum += take;
      k0 += take;
      if (cur.sum == tau || cur.n == 2) {
        if ((int)bins.size() >= max_bins) return false;
        bins.push_back(cur);
        cur = PairBin{};
      }
    }
  }
  if (cur.n) {
    if ((int)bins.size() >= max_bins) return false;
    bins.push_back(cur);
  }
  return true;
}

// Time (us) of a CU running one bin: pieces of a and b key tiles (a >= b,
// b = 0 for none) of units cut into na and nb pieces (1: unsplit; a split
// piece ends with a partial state and a ticket, the unit's last one with
// the merge).  The first-dispatched workgroup has issue priority: side by
// side it runs a tile in kTileOld, the other in kTileYoung; alone either
// runs one in kTileAlone; the second's end phase is slower while the first
// still runs.  Least-squares fit to the per-CU finish times of 46 bin
// shapes in per-workgroup timelines of paired 1024-token launches (16-query
// halves, 20/5 heads, MI355X): 0.52 us rms, 1.3 us at most.
constexpr double kStartOld = 3.272, kStartYoung = 4.6, kTileOld = 3.926, kTileYoung = 5.388,
                 kTileAlone = 2.53, kEndUnsplit = 0.85, kEndSplit = 1.808, kEndSplit3 = 2.135,
                 kEndYoungUnsplit = 4.018, kEndYoungSplit = 6.063;
double bin_time(int a, int b, int na, int nb) {
  auto end = [](int n) { return n <= 1 ? kEndUnsplit : n == 2 ? kEndSplit : kEndSplit3; };
  if (b == 0) return kStartOld + a * kTileAlone + end(na);
  const double ty = kStartYoung + b * kTileYoung, to = kStartOld + a * kTileOld;
  if (ty <= to) {
    const double done = (ty - kStartOld) / kTileOld;
    return std::max(ty + (nb <= 1 ? kEndYoungUnsplit : kEndYoungSplit),
                    ty + (a - done) * kTileAlone + end(na));
  }
  const double done = (to - kStartYoung) / kTileYoung;
  return std::max(to + end(na), to + (b - done) * kTileAlone + end(nb));
}

// The largest modelled bin time of a packing.
double packing_time(const std::vector<PairBin> &bins, int nu) {
  std::vector<int> pieces((size_t)nu, 0);
  for (const PairBin &b : bins)
    for (int k = 0; k < b.n; ++k) ++pieces[(size_t)b.p[k].unit];
  double worst = 0.0;
  for (const PairBin &b : bins) {
    if (b.n == 0) continue;
    const bool first = b.n < 2 || b.p[0].len >= b.p[1].len;
    const PairPiece &x = first ? b.p[0] : b.p[1];
    const PairPiece *y = b.n < 2 ? nullptr : first ? &b.p[1] : &b.p[0];
    worst = std::max(worst, bin_time(x.len, y ? y->len : 0, pieces[(size_t)x.unit],
                                     y ? pieces[(size_t)y->unit] : 1));
  }
  return worst;
}

// Packing for a target bin time Ts under bin_time.  Repeatedly, the
// shortest remaining unit (or remainder) that can go beside another piece is
// the bin's second piece, whole, and the first piece is the longest the
// model allows beside it (a remainder of exactly that length, else cut from
// the longest -- or, with !largest, the shortest longer -- remainder);
// once every remainder is too long to go second, bins take the most key
// tiles the model allows as two cut pieces, the first from the longest
// remainder, the second from the shortest.  False when the bins exceed
// max_bins or a piece cannot meet Ts.
bool model_pack(const std::vector<int> &nk, double Ts, int max_bins, bool largest,
                std::vector<PairBin> &bins) {
  bins.clear();
  // cut pieces counted as two-way splits (a unit cut more often is caught
  // by the caller's packing_time check)
  auto amax = [&](int b, bool sa, bool sb) {
    int a = -1;
    for (int x = std::max(b, 1); x <= 255; ++x) {
      if (bin_time(x, b, sa ? 2 : 1, sb ? 2 : 1) > Ts) break;
      a = x;
    }
    return a;
  };
  // the longest first piece beside a whole second piece of b tiles
  std::vector<int> A;
  for (int b = 0; b <= 255; ++b) {
    A.push_back(amax(b, true, false));
    if (A.back() < b) break;
  }
  int ymax = 0;
  for (int b = 1; b <= 255 && amax(b, true, true) >= b; ++b) ymax = b;
  int bal_a = amax(0, true, false), bal_b = 0;
  for (int b = 1; b <= ymax; ++b) {
    const int a = amax(b, true, true);
    if (a + b > bal_a + bal_b) {
      bal_a = a;
      bal_b = b;
    }
  }
  if (bal_a < 1) return false;
  struct Entry {
    int size, unit, kt0;
    bool whole;
  };
  std::vector<Entry> pool;
  for (int u = 0; u < (int)nk.size(); ++u) pool.push_back(Entry{nk[(size_t)u], u, 0, true});
  auto take = [](Entry &e, int n) {
    const PairPiece pc{e.unit, e.kt0, n};
    e.size -= n;
    e.kt0 += n;
    e.whole = false;
    return pc;
  };
  for (;;) {
    pool.erase(std::remove_if(pool.begin(), pool.end(), [](const Entry &e) { return e.size <= 0; }),
               pool.end());
    if (pool.empty()) return true;
    if ((int)bins.size() >= max_bins) return false;
    std::sort(pool.begin(), pool.end(), [](const Entry &x, const Entry &y) {
      return x.size != y.size ? x.size < y.size : x.unit < y.unit;
    });
    PairBin bin{};
    if (pool[0].size <= ymax) {
      const int a = pool[0].size < (int)A.size() ? A[(size_t)pool[0].size] : -1;
      if (a < pool[0].size) return false;
      const PairPiece young = take(pool[0], pool[0].size);
      size_t pick = 0;  // 0: none
      for (size_t i = 1; i < pool.size() && !pick; ++i)
        if (pool[i].size == a) pick = i;
      if (!pick) {
        for (size_t i = 1; i < pool.size(); ++i)
          if (pool[i].size > a && (!pick || (largest ? pool[i].size > pool[pick].size
                                                      : pool[i].size < pool[pick].size)))
            pick = i;
      }
      if (!pick && pool.size() > 1) pick = pool.size() - 1;  // the longest, whole
      if (pick) {
        bin.p[bin.n++] = take(pool[pick], std::min(a, pool[pick].size));
      }
      bin.p[bin.n++] = young;
    } else {
      Entry &L = pool.back();
      bin.p[bin.n++] = take(L, std::min(bal_a, L.size));
      Entry *e = nullptr;
      for (Entry &x : pool)
        if (x.size > 0 && (!e || x.size < e->size)) e = &x;
      if (e && bal_b > 0) bin.p[bin.n++] = take(*e, std::min(bal_b, e->size));
    }
    bin.sum = bin.p[0].len + (bin.n > 1 ? bin.p[1].len : 0);
    bins.push_back(bin);
  }
}

}  // namespace

// The paired plan (see PairPlan).  Two packings compete under bin_time:
// the chain packing (for each tau from the mean bin load up, every
// threshold between pairing whole units and cutting the chain is packed,
// the one with the fewest pieces kept, the first tau that fits the bins and
// the partial-state slots taken) and model_pack at the smallest target
// (0.1 us steps from the balanced bin's time) it meets.  The faster one in
// the model is encoded; `span` is prefill_span's CU model applied to its
// bins: the two pieces side by side, the longer finishing alone, plus the
// merge of a split unit.
bool plan_prefill_pairs(int n_tokens, int start_pos, int n_kv, int n_cu, long long item_budget,
                        PairPlan &p) {
  p = PairPlan{};
  if (n_tokens <= 0 || n_kv <= 0 || start_pos < 0) return false;
  const int max_bins = std::min(n_cu / n_kv, kMaxPairBins);
  const int nu = (n_tokens + 15) / 16;
  if (max_bins <= 0 || nu > 2 * max_bins) return false;
  const long long last_row = (long long)start_pos + n_tokens - 1;
  if (last_row / 32 + 1 > 65535) return false;  // kt0 + len in 16 bits
  std::vector<int> nk((size_t)nu);
  long long S = 0;
  for (int u = 0; u < nu; ++u) {
    nk[(size_t)u] = (int)(std::min<long long>(start_pos + 16LL * u + 15, last_row) / 32 + 1);
    S += nk[(size_t)u];
  }
  const int nqt = (n_tokens + 31) / 32;
  // Slots of the split query tiles (both halves share a slot index); false
  // past the budget.
  auto slots = [&](const std::vector<PairBin> &bins, std::vector<int> &nch, std::vector<int> &base,
                   int &n_slots) {
    nch.assign((size_t)nu, 0);
    for (const PairBin &b : bins)
      for (int k = 0; k < b.n; ++k) ++nch[(size_t)b.p[k].unit];
    base.assign((size_t)nqt, 0);
    n_slots = 0;
    for (int qt = 0; qt < nqt; ++qt) {
      const int m = std::max(nch[(size_t)(2 * qt)], 2 * qt + 1 < nu ? nch[(size_t)(2 * qt + 1)] : 0);
      base[(size_t)qt] = n_slots;
      if (m > 1) n_slots += m;
    }
    for (int v : nch)
      if (v > 255) return false;
    return n_slots <= 256 && (long long)n_slots * n_kv <= item_budget;
  };
  std::vector<int> nch, base;
  int n_slots = 0;
  // the chain packing
  std::vector<PairBin> bins, chain, model;
  std::vector<int> thr;
  for (int tau = (int)std::max<long long>(1, (S + max_bins - 1) / max_bins); tau <= 255; ++tau) {
    thr.assign({1, tau + 1});
    for (int v : nk)
      if (v <= tau) thr.push_back(v);
    std::sort(thr.begin(), thr.end());
    thr.erase(std::unique(thr.begin(), thr.end()), thr.end());
    int best_pieces = 1 << 30;
    std::vector<PairBin> best;
    for (int t : thr) {
      if (!pair_pack(nk, tau, t, max_bins, bins)) continue;
      int pieces = 0;
      for (const PairBin &b : bins) pieces += b.n;
      if (pieces < best_pieces) {
        best_pieces = pieces;
        best = bins;
      }
    }
    if (!best.empty() && slots(best, nch, base, n_slots)) {
      chain = best;
      break;
    }
  }
  const double t_chain = chain.empty() ? 1e300 : packing_time(chain, nu);
  // the model packing, at most as slow as the chain's: 1 us steps from
  // below the balanced bin's time to the first target met, then 0.1 us steps
  // over the last 1 us
  {
    auto attempt = [&](double ts) {
      for (int largest = 1; largest >= 0; --largest) {
        if (!model_pack(nk, ts, max_bins, largest != 0, bins)) continue;
        if (packing_time(bins, nu) > ts + 1e-9 || !slots(bins, nch, base, n_slots)) continue;
        model = bins;
        return true;
      }
      return false;
    };
    const int mean = (int)((S + max_bins - 1) / max_bins);
    const double t0 = bin_time((mean * 3 + 4) / 5, mean - (mean * 3 + 4) / 5, 2, 2) - 2.0;
    const double t_end = std::min(t_chain, t0 + 1000.0);
    double hit = -1.0;
    for (double ts = t0; ts < t_end + 1.0 && hit < 0; ts += 1.0)
      if (attempt(std::min(ts, t_end))) hit = std::min(ts, t_end);
    for (int i = 1; hit >= 0 && i < 10; ++i)
      if (!attempt(hit - 1.0 + 0.1 * i)) continue;
      else break;
  }
  const std::vector<PairBin> *pick = nullptr;
  if (!model.empty() && packing_time(model, nu) < t_chain) pick = &model;
  else if (!chain.empty()) pick = &chain;
  if (!pick) return false;
  const std::vector<PairBin> &best = *pick;
  slots(best, nch, base, n_slots);
  p.bins = (int)best.size();
  p.n_slots = n_slots;
  p.model_us = packing_time(best, nu);
  double span = 0.0;
  constexpr double kShared = 1.9;
  for (size_t b = 0; b < best.size(); ++b) {
    PairBin bin = best[b];
    if (bin.n == 2 && bin.p[1].len > bin.p[0].len) std::swap(bin.p[0], bin.p[1]);
    p.tau = std::max(p.tau, bin.p[0].len + (bin.n > 1 ? bin.p[1].len : 0));
    double w[2] = {0.0, 0.0}, tail = 0.0;
    for (int k = 0; k < bin.n; ++k) {
      const PairPiece &pc = bin.p[k];
      const int u = pc.unit, qt = u / 2, half = u & 1;
      int ch = 0;  // pieces of the unit before this one
      for (const PairBin &o : best)
        for (int j = 0; j < o.n; ++j)
          if (o.p[j].unit == u && o.p[j].kt0 < pc.kt0) ++ch;
      const int n = nch[(size_t)u];
      p.piece[2 * b + k][0] = (unsigned)pc.kt0 | (unsigned)qt << 16 | (unsigned)half << 31;
      p.piece[2 * b + k][1] = (unsigned)pc.len | (unsigned)ch << 8 | (unsigned)n << 16 |
                              (unsigned)(n > 1 ? base[(size_t)qt] : 0) << 24;
      w[k] = g_pf16_fixed + pc.len * g_pf16_tile;
      if (n > 1) tail = std::max(tail, (n - 1) * g_pf16_merge);
    }
    const double a = std::min(w[0], w[1]), c = std::max(w[0], w[1]);
    span = std::max(span, (bin.n == 2 ? a * kShared + (c - a) : c) + tail);
  }
  p.span = span;
  return true;
}

// The chunk size, balance and query height for a prefill shape.  Each
// candidate costs two dispatch replays (tens to hundreds of us each); sizes
// between the powers of two matter: they set how evenly the items fill the
// resident slots (N = 1024 runs 8 % faster at 6 tiles than at 4, 512 queries
// after 1536 cached 14 % faster at 10 than at 4 or 16).  A candidate whose
// (kv head, item) pairs would exceed prefill_item_budget(cap) is not
// considered, so the workspace sized by that budget holds every planned
// launch.
PrefillChoice plan_prefill_chunk(int n_tokens, int start_pos, int n_kv, int n_cu, int bal_pref,
                                 int q16_pref, long long cap, int pair_pref, PairPlan *pairs) {
  const long long budget = prefill_item_budget(cap, n_kv);
  // A paired launch (one dispatch round of the 16-query kernel) wherever one
  // fits: graph-timed on MI355X (20/5 heads) it matches or beats the planned
  // chunks at every shape tried -- 256 to 1536 tokens from an empty cache
  // (1024: 53.6 vs 60.0 us, 768: 35.6 vs 42.2 us) and after cached prefixes
  // (512 after 512: 45.2 vs 47.9 us, 300 after 5: 16.6 vs 17.7 us).
  if (pairs && pair_pref != 0 && q16_pref != 0 &&
      plan_prefill_pairs(n_tokens, start_pos, n_kv, n_cu, budget, *pairs))
    return PrefillChoice{kPrefillNoSplit, 0, 1, 1};
  PrefillChoice best{kPrefillNoSplit, 0, 0, 0};
  double best_span = 1e300;
  for (int q = 0; q <= 1; ++q) {
    if ((q == 0 && q16_pref == 1) || (q == 1 && q16_pref == 0)) continue;
    const double margin = q ? g_pf16_margin : 0.99;  // a switch to halves must gain this much
    const double span = prefill_span(n_tokens, start_pos, n_kv, kPrefillNoSplit, n_cu, false, q);
    if (span < best_span * margin) {
      best_span = span;
      best = PrefillChoice{kPrefillNoSplit, 0, q, 0};
    }
    for (int ct : kPrefillChunkCandidates) {
      if (prefill_plan(n_tokens, start_pos, ct).n_items * (long long)n_kv > budget) continue;
      for (int bal = 0; bal <= 1; ++bal) {
        if ((bal == 0 && bal_pref == 1) || (bal == 1 && bal_pref == 0)) continue;
        // 16-query halves with balanced chunks measured 4-12 % slower than
        // with plain ones at every shape tried: not a candidate
        if (q && bal && bal_pref != 1) continue;
        const double sp = prefill_span(n_tokens, start_pos, n_kv, ct, n_cu, bal != 0, q);
        if (sp < best_span * (q && !best.q16 ? margin : 0.99)) {
          best_span = sp;
          best = PrefillChoice{ct, bal, q, 0};
        }
      }
    }
  }
  return best;
}

// (kv head, item) pairs a planned chunked launch may use on a cache of cap
// rows: four chunks per query tile on average over the cap/32 query tiles,
// and never more than kPrefillMaxPlannedItems.  Replaying the planner over
// every 32-aligned (tokens, start) pair a cache of 2048 / 4096 / 8192 rows
// allows (5 kv heads, start below the token count: the launches that take
// key chunks), the budget lengthens the modelled span by 0.3 / 1.5 / 1.0 %
// at worst against unlimited items, 0.0 % on average.  The partial states
// cost group * 66 * 64 floats (16.9 KB per q head) each.
long long prefill_item_budget(long long cap, int n_kv) {
  const long long tiles = (std::max(cap, 1LL) + 31) / 32;
  return std::min(4LL * n_kv * tiles, kPrefillMaxPlannedItems);
}

}  // namespace bnr
