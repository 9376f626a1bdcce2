// bnr_internal.h -- launch interface between the C ABI layer (bnr_api.cpp)
// and the gfx950 kernels (bnr_kernels.hip).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <stddef.h>
#include <stdint.h>

namespace bnr {

// Head dimension of the fast kernels (BitNet b1.58 2B: 2560 / 20).
constexpr int kHeadDim = 128;
// Sequences per decode launch: per-sequence positions and split offsets
// travel in the kernel-argument segment, so no host->device copy is needed.
constexpr int kMaxBatchPerLaunch = 64;
// Upper bound on context splits per (sequence, kv head); longer contexts
// give each workgroup several passes over its rows.
constexpr int kMaxSplits = 256;
// Ticket counters are 256 bytes apart: atomics on one cache line serialise.
constexpr int kCounterStride = 64;
// Reference merge accumulators of one (sequence, kv head), in floats: the
// G*128 output sums at 0, the G weight sums at kAccL, four 64-bit masks of
// splits that took the exact path at kAccMask (G <= 4).
constexpr int kAccL = 512;
constexpr int kAccMask = 576;
constexpr int kAccStride = 640;
// A split whose largest score exceeds the reference by more than this (in
// log2 units) would overflow the reference-weighted sums: it takes the
// exact path (own running maximum, partial state for the merging
// workgroup).  Weights of at most 2^64 keep 65536 rows of |v| <= 2^40
// below FLT_MAX (2^128).
constexpr float kRefSlack = 64.0f;

// RoPE + append over n_tokens consecutive positions of one sequence.  q and
// k are rotated in place; when k_cache is non-null the rotated k rows and the
// v rows are written at rows start_pos + i of a head-major cache.
struct RopeAppendArgs {
  float *q;
  float *k;
  const float *v;
  int n_tokens, start_pos, n_heads, n_kv, head_dim;
  const float *cos_tab, *sin_tab;  // [table_len x head_dim/2]
  float *k_cache, *v_cache;
  long long kv_stride;  // elements between kv heads of the cache (cap * head_dim)
  // Host-slice calls: pinned host words; workgroup w stores seq into done[w]
  // once its outputs are visible to the host (null: no signal).
  unsigned *done;
  unsigned seq;
};
hipError_t launch_rope_append(const RopeAppendArgs &a, hipStream_t s);
// Workgroups of launch_rope_append's launch (the done[] words it sets).
long long rope_append_blocks(const RopeAppendArgs &a);

// Split-K decode attention for head_dim 128.  One workgroup owns one
// (sequence, kv head, context chunk) and serves the kv head's G query
// heads from one read of each K/V row.
struct DecodeArgs {
  const float *q;      // [b][n_kv*G][128]; raw when cos_tab != null
  const float *k_new;  // [b][n_kv][128] raw new keys (fused append) or null
  const float *v_new;  // [b][n_kv][128] new values (fused append) or null
  float *k_cache, *v_cache;
  long long q_bstride, kn_bstride, cache_bstride, out_bstride;  // elements
  long long kv_stride;                                          // elements
  float *out;
  float *q_rot, *k_rot;           // optional rotated q / k outputs
  const float *cos_tab, *sin_tab; // [table_len x 64] or null (q pre-rotated)
  float *ws_o;                    // split partials: [split][n_kv][G][128]
  float2 *ws_ml;                  // split (max, sum): [split][n_kv][G]
  unsigned *counters;             // [batch][n_kv] x kCounterStride, zero between launches
  float scale_log2;               // log2(e) / sqrt(128)
  int n_kv, group, batch;
  int rows_per_split;             // rows a workgroup owns (16*RPG*passes)
  int rpg;                        // rows per 16-lane row group and pass
  int passes;
  int merge_inline;                // 1: last-workgroup merge; 0: second kernel
  // Reference merge (merge_ref = 1, decode_ref_kernel): every split weighs
  // its rows against one reference score per q head -- the score of row
  // `position`, which every workgroup computes identically -- and adds its
  // unnormalised sums into acc with device-scope float atomics; the last
  // workgroup of a (sequence, kv head) divides.  acc: [batch][n_kv] x
  // kAccStride floats, zero between launches.
  int merge_ref;
  // With merge_ref: every split stores its (m, l, O) and the last workgroup
  // combines them in a fixed order (det_merge): outputs bit-identical from
  // run to run, at the cost measured in the design notes.
  int merge_det;
  float *acc;
  int ref_waves;  // waves per workgroup of the reference-merge kernel: 4 or 8
  int max_splits;                  // largest split count of the launch (grid x)
  // Host-slice calls (reference-merge kernel only): pinned host words; the
  // workgroup that writes the output of (sequence b, kv head h) stores seq
  // into done[b * n_kv + h] once that output is visible to the host.
  unsigned *done;
  unsigned seq;
  // Measurement builds only (compiled with BNR_TIMELINE): when
  // non-null, every workgroup of the reference-merge kernel stores
  // kTimelineStamps s_memrealtime stamps (100 MHz) at
  // timeline[linear block index * kTimelineStamps].  Ignored otherwise.
  unsigned long long *timeline;
  int positions[kMaxBatchPerLaunch];
  int split_off[kMaxBatchPerLaunch + 1];
};
// Stamps per workgroup of a timeline build: entry, loads issued, rows
// consumed, path barrier passed, combine done (sums sent), sums complete,
// ticket returned, merge done (merging workgroup only, else 0).
constexpr int kTimelineStamps = 8;
hipError_t launch_decode(const DecodeArgs &a, hipStream_t s);
// The reference-merge kernel alone (a.merge_ref; group 1, 2 or 4).
hipError_t launch_decode_ref(const DecodeArgs &a, hipStream_t s);

// Scratch of the allocation-free decode entry point (bnr_noalloc.hip), for
// at most kNoAllocMaxHeads query heads and kMaxSplits splits: the
// reference-merge accumulators and tickets (zero between launches), then the
// exact path's partial states.  About 4.15 MiB per GPU.
constexpr int kNoAllocMaxHeads = 32;
constexpr long long kNoAllocAccBytes = (long long)kNoAllocMaxHeads * kAccStride * 4;
constexpr long long kNoAllocCounterBytes = (long long)kNoAllocMaxHeads * kCounterStride * 4;
constexpr long long kNoAllocZeroBytes = kNoAllocAccBytes + kNoAllocCounterBytes;
constexpr long long kNoAllocMlBytes = (long long)kMaxSplits * kNoAllocMaxHeads * 8;
constexpr long long kNoAllocOBytes = (long long)kMaxSplits * kNoAllocMaxHeads * kHeadDim * 4;
constexpr long long kNoAllocScratchBytes = kNoAllocZeroBytes + kNoAllocMlBytes + kNoAllocOBytes;
// The scratch's address on `device` (current), set up once per device: its
// merge state zeroed by a kernel on `s`, then `s` synchronised.
hipError_t noalloc_scratch(int device, hipStream_t s, void **out);
// The scratch of `device` serves one (context, stream) pair at a time:
// true when it is free (it is then claimed) or already held by this pair.
// A context gives it up when it is destroyed.
bool noalloc_claim(int device, const void *ctx, const void *stream);
void noalloc_release(int device, const void *ctx);

// Decode planner inputs: the device and the context's tuning state.
struct DecodePlanConfig {
  int n_cu;        // CUs of the device
  int target_wgs;  // small launches: at most this many workgroups (default n_cu)
  int large_wgs;   // launches of at least this many 64-row workgroups use the two-launch merge
  int force_rpg;   // 0, or a fixed rows-per-row-group (tuning)
  int min_passes;  // at least this many passes per split (tuning, default 1)
  int merge_mode;  // -1: reference merge (default); 0: second kernel; 1: in-kernel ticket;
                   // 2: reference merge; 3: reference merge, deterministic (merge_det)
  int split_cost;  // planner cost of one split of the in-kernel merges (ns), -1: the mode's default
  int ref_rows;    // reference merge: rows per split (0: planner decides)
  int ref_waves;   // reference merge, small launches: 4 or 8 waves per workgroup, or 0:
                   // 4 up to kRefWaves4Rows rows, 8 beyond (large launches: 4)
};
// Small reference-merge launches of at most this many rows per sequence run
// 4-wave workgroups (graph-timed on MI355X, 2B shape: 4 waves 5.98 vs 6.30 us
// at 512 rows, 7.33 vs 7.48 us at 1536; 8 waves 7.42 vs 7.57 us at 2048 and
// 8.98 vs 9.23 us at 4096).
constexpr int kRefWaves4Rows = 1792;
// Large reference-merge launches: splits of at most this many rows use at
// most 3 rows per row group and pass (5 passes of a 4-wave workgroup), longer
// ones up to 4.
constexpr int kLargeRpg3Rows = 240;
// Split-K plan of one decode launch over sequences of lens[b] rows: fills
// a.rpg, a.passes, a.rows_per_split, a.batch, a.split_off, a.max_splits and
// a.merge_inline.
void plan_decode(const DecodePlanConfig &c, const int *lens, int batch, int n_kv, DecodeArgs &a);

// Any head_dim / group size: one workgroup per query head, scores staged in
// a global workspace [n_heads][L].
struct DecodeGenericArgs {
  const float *q;
  const float *k_cache, *v_cache;
  long long kv_stride;
  float *out;
  float *scores;
  int n_heads, group, head_dim, L;
  float scale;
};
hipError_t launch_decode_generic(const DecodeGenericArgs &a, hipStream_t s);

// Plain streaming read of two device ranges (16-byte multiples), for
// measurement.
hipError_t launch_stream_read(const void *a, long long a_bytes, const void *b, long long b_bytes,
                              hipStream_t s);
// The same read with `loads` (1, 2, 4, 8 or 16) 16-byte loads in flight per
// lane, workgroups of `threads` (a multiple of 64, <= 1024), non-temporal
// loads when nt.
hipError_t launch_stream_read_shape(const void *a, long long a_bytes, const void *b,
                                    long long b_bytes, int threads, int loads, bool nt,
                                    hipStream_t s);

// Bins per kv head of a paired 16-query prefill launch (PrefillArgs).
constexpr int kMaxPairBins = 64;

// Causal flash prefill (head_dim 128, fp32 MFMA): query i of the n_tokens
// (position start_pos + i) attends cache rows 0..start_pos+i.
struct PrefillArgs {
  const float *q;                    // [n_tokens][n_heads][128], rotated
  const float *k_cache, *v_cache;    // [n_kv][cap][128]
  long long kv_stride;               // cap * 128
  float *out;                        // [n_tokens][n_heads][128]
  int n_tokens, start_pos, n_heads, n_kv;
  float scale_log2;                  // log2(e) / sqrt(128)
  // Key-range split: a query tile's key tiles are processed in chunks of
  // chunk_tiles tiles by separate workgroups; the last to finish merges.
  int chunk_tiles;
  int n_qtiles;                      // ceil(n_tokens / 32)
  int n_items;                       // (query tile, chunk) items per kv head
  float *ws;                         // partial states: [n_kv][n_items][G][66][64], by (query tile, chunk)
  unsigned *counters;                // [n_kv][n_qtiles] x kCounterStride, zero between launches
  unsigned *queue;                   // persistent launch: next item, workgroups done (2 x kCounterStride), zero between launches
  // Item order (prefill_order fills these).  lpt: longest first -- every
  // full-length chunk (n_full of them per kv head), then the shorter last
  // chunks of the query tiles by decreasing length, those of length ct-1-b
  // at part_off[b] .. part_off[b+1]-1 after the full ones (ct = chunk_tiles
  // <= kMaxLptChunk).  Otherwise query tiles from the last down, the chunks
  // of one tile consecutive.
  int lpt, n_full;
  int part_off[64];
  // Balanced key chunks (balanced = 1, chunk_tiles <= kMaxLptChunk): a query
  // tile of nk key tiles keeps its nch = ceil(nk / chunk_tiles) chunks, but
  // they take nk / nch tiles each, the first nk % nch one more, and the
  // items go longest first (pf_bal_map).  bal_off[l] = items longer than l
  // key tiles (prefill_order fills it).
  int balanced;
  int bal_off[65];
  // Grid-mapped launches: q16 = 1 runs every item as two 16-query halves
  // (prefill16_kernel; grid x = 2 n_kv); counters then hold one ticket per
  // (kv head, query tile, half).
  int q16;
  // Paired launch of the 16-query kernel (pair_bins > 0, q16 = 1): a 1-D grid
  // of 2 * pair_cu workgroups.  Workgroup i runs piece i / pair_cu on CU
  // c = i % pair_cu, renumbered XCD by XCD when pair_cu % 8 == 0:
  // c' = (c % 8) (pair_cu / 8) + c / 8 (else c' = c); c' is bin c' % pair_bins
  // of kv head c' / pair_bins.  A head past n_kv or a piece of zero length
  // exits at once.  A piece is a key
  // range of one 16-query unit (pf16_pair_piece has the encoding); the plan
  // puts at most two pieces in a bin so that they share a CU: on an idle
  // device the dispatcher gives workgroups i and i + (CU count) the same CU,
  // the first one first.  n_items is then the partial-state slots per kv
  // head (base + ch of a piece; both halves of a query tile share a slot).
  int pair_bins, pair_cu;
  unsigned pair_piece[2 * kMaxPairBins][2];
  // Stream-K launch (sk_units > 0): units = (kv head, query tile, key tile)
  // tile products in that order, sk_per_head of them per kv head; the
  // launch's workgroups take equal runs of them.  ws then holds two partial
  // states per workgroup: [2 * workgroups][G][66][64].
  long long sk_units, sk_per_head;
  // Measurement builds only (compiled with BNR_TIMELINE): when non-null,
  // workgroup (x, y) of the grid-mapped kernel stores kTimelineStamps words
  // at timeline[(y * gridDim.x + x) * kTimelineStamps] (PfStamp).  Ignored
  // otherwise.
  unsigned long long *timeline;
};
// Kernel arguments are passed by value: keep them within 4 KB.
static_assert(sizeof(PrefillArgs) <= 4096, "PrefillArgs exceeds the kernel argument limit");
// Words of a prefill workgroup's timeline record: 100 MHz s_memrealtime
// stamps at entry, Q and first K/V tile in LDS, last key tile done, partial
// state stored and ticket taken (split query tiles; else = key tiles done),
// merge done (the merging chunk; else 0), output stored (else 0); then the
// hardware ids (XCC_ID << 32 | HW_ID) and the item (key tiles | nch << 16 |
// query tile << 32).
enum PfStamp { kPfEntry, kPfReady, kPfTiles, kPfTicket, kPfMerged, kPfStored, kPfHwId, kPfItem };
constexpr int kMaxLptChunk = 64;
constexpr int kPrefillNoSplit = 1 << 20;  // chunk_tiles of an unsplit launch
constexpr int kPrefillMaxTokens = 32 * 65535;  // query tiles of one tiled prefill launch

// Sum over x = 1..m of floor(x / ct), and of ceil(x / ct) (m >= 0, ct >= 1).
__host__ __device__ inline long long pf_floor_sum(int m, int ct) {
  const long long q = m / ct, r = m % ct;
  return q > 0 ? ct * (q * (q - 1) / 2) + q * (r + 1) : 0;
}
__host__ __device__ inline long long pf_ceil_sum(int m, int ct) {
  const long long q = m / ct, r = m % ct;
  return ct * (q * (q + 1) / 2) + r * (q + 1);
}

// Work item y (per kv head) of a prefill launch -> query tile qt, chunk ch
// of its nch chunks, and base = the partial-state slot of the tile's chunk
// 0 (slot of chunk ch: base + ch).  Query tile qt < nqt-1 has qt + A key
// tiles, A = ceil((start_pos + 1) / 32); the last (possibly short) tile
// last_row / 32 + 1.  The host's dispatch replay uses the same function.
__host__ __device__ inline void prefill_map(const PrefillArgs &a, int y, int &qt, int &ch,
                                            int &nch, int &base) {
  const int ct = a.chunk_tiles, nqt = a.n_qtiles;
  const int last_row = a.start_pos + a.n_tokens - 1;
  const int A = (a.start_pos + 31) / 32 + 1;
  const int nt_last = last_row / 32 + 1;
  if (!a.lpt) {
    // Tiles from the last down, chunks consecutive: the items of tiles
    // q .. nqt-2 are a difference of two ceil sums; binary search.
    const int nch_last = (nt_last + ct - 1) / ct;
    if (y < nch_last) {
      qt = nqt - 1;
      ch = y;
      nch = nch_last;
    } else {
      const long long yy = y - nch_last;
      const long long top = pf_ceil_sum(nqt - 2 + A, ct);
      int lo = 0, hi = nqt - 2;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (top - pf_ceil_sum(mid - 1 + A, ct) > yy) lo = mid;
        else hi = mid - 1;
      }
      qt = lo;
      ch = (int)(yy - (top - pf_ceil_sum(lo + A, ct)));
      nch = (lo + A + ct - 1) / ct;
    }
  } else if (y < a.n_full) {
    // Full chunks: the last tile's, then tiles nqt-2 down to 0 (floor sums).
    const int f_last = nt_last / ct;
    if (y < f_last) {
      qt = nqt - 1;
      ch = y;
      nch = (nt_last + ct - 1) / ct;
    } else {
      const long long yy = y - f_last;
      const long long top = pf_floor_sum(nqt - 2 + A, ct);
      int lo = 0, hi = nqt - 2;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (top - pf_floor_sum(mid - 1 + A, ct) > yy) lo = mid;
        else hi = mid - 1;
      }
      qt = lo;
      ch = (int)(yy - (top - pf_floor_sum(lo + A, ct)));
      nch = (lo + A + ct - 1) / ct;
    }
  } else {
    // Last chunks shorter than ct, longest first; within one length the
    // last tile first, then the others from the highest tile down.
    const int y2 = y - a.n_full;
    int b = 0;
    while (b + 1 < ct - 1 && a.part_off[b + 1] <= y2) ++b;
    const int r = ct - 1 - b;
    int k = y2 - a.part_off[b];
    if (nt_last % ct == r) {
      if (k == 0) {
        qt = nqt - 1;
        ch = nt_last / ct;
        nch = ch + 1;
        base = (int)(pf_ceil_sum(qt - 1 + A, ct) - pf_ceil_sum(A - 1, ct));
        return;
      }
      --k;
    }
    const int q0 = ((r - A) % ct + ct) % ct;  // lowest regular tile with qt + A = r (mod ct)
    const int cnt = nqt - 2 >= q0 ? (nqt - 2 - q0) / ct + 1 : 0;
    qt = q0 + (cnt - 1 - k) * ct;
    ch = (qt + A) / ct;
    nch = ch + 1;
  }
  base = (int)(pf_ceil_sum(qt - 1 + A, ct) - pf_ceil_sum(A - 1, ct));
}

// Key tiles kt0 .. kt0 + len - 1 of chunk ch of a query tile with nk key
// tiles cut into nch balanced chunks.
__host__ __device__ inline void pf_bal_range(int nk, int nch, int ch, int &kt0, int &len) {
  const int q = nk / nch, r = nk - q * nch;
  kt0 = ch * q + (ch < r ? ch : r);
  len = q + (ch < r ? 1 : 0);
}

// Work item y (per kv head) of a balanced launch -> query tile qt, chunk ch
// of its nch chunks.  Order: chunk length descending; within one length the
// last query tile first, then the others from the highest down; within a
// tile, chunks in order.  A query tile qt < nqt-1 has nk = A + qt key tiles
// (A as in prefill_map) and nch = m = ceil(nk / ct) chunks: with q = nk / m
// and r = nk % m, chunks 0 .. r-1 have q + 1 tiles and r .. m-1 have q.  So
// the tiles of block m (nch = m) with a chunk of length l are those with
// q = l (nk in [l m, l m + m - 1], its m - r chunks ch = r ..) and those
// with q = l - 1 (nk in [(l-1) m + 1, l m - 1], its r chunks ch = 0 ..): a
// block's count is two arithmetic sums, and only the block that holds item
// y is walked tile by tile.  The host's dispatch replay and the kernels use
// this same function.
__host__ __device__ inline void pf_bal_map(const PrefillArgs &a, int y, int &qt, int &ch,
                                           int &nch) {
  const int ct = a.chunk_tiles, nqt = a.n_qtiles;
  const int A = (a.start_pos + 31) / 32 + 1;
  const int nk_last = (a.start_pos + a.n_tokens - 1) / 32 + 1;
  int l = ct;
  while (l > 1 && y >= a.bal_off[l - 1]) --l;
  long long k = y - a.bal_off[l];
  {
    const int m = (nk_last + ct - 1) / ct, q = nk_last / m, r = nk_last - q * m;
    const int c = l == q + 1 ? r : (l == q ? m - r : 0);
    if (k < c) {
      qt = nqt - 1;
      nch = m;
      ch = (l == q + 1 ? 0 : r) + (int)k;
      return;
    }
    k -= c;
  }
  const int nk_hi = A + nqt - 2;  // the highest regular tile (none if nqt == 1)
  for (int m = (nk_hi + ct - 1) / ct; nqt > 1 && m >= 1; --m) {
    const int lo = (m - 1) * ct + 1 > A ? (m - 1) * ct + 1 : A;
    const int hi = m * ct < nk_hi ? m * ct : nk_hi;
    if (lo > hi) break;  // blocks below hold no regular tile
    const int a1 = lo > l * m ? lo : l * m, b1 = hi < l * m + m - 1 ? hi : l * m + m - 1;
    const int a2 = lo > (l - 1) * m + 1 ? lo : (l - 1) * m + 1, b2 = hi < l * m - 1 ? hi : l * m - 1;
    const long long n1 = b1 >= a1 ? b1 - a1 + 1 : 0, n2 = b2 >= a2 ? b2 - a2 + 1 : 0;
    const long long s1 = n1 * ((long long)m + (long long)l * m) - (a1 + (long long)b1) * n1 / 2;
    const long long s2 = (a2 + (long long)b2) * n2 / 2 - n2 * (long long)(l - 1) * m;
    if (k >= s1 + s2) {
      k -= s1 + s2;
      continue;
    }
    for (int nk = b1; nk >= a1; --nk) {  // q == l: m - r chunks of length l
      const int r = nk - l * m;
      if (k < m - r) {
        qt = nk - A;
        nch = m;
        ch = r + (int)k;
        return;
      }
      k -= m - r;
    }
    for (int nk = b2; nk >= a2; --nk) {  // q == l - 1: r chunks of length l
      const int r = nk - (l - 1) * m;
      if (k < r) {
        qt = nk - A;
        nch = m;
        ch = (int)k;
        return;
      }
      k -= r;
    }
  }
  qt = 0;  // not reached for y below the item count
  ch = 0;
  nch = 1;
}

// (query tile, chunk) items per kv head of a prefill launch, and the key
// tiles they cover in total.
struct PrefillPlan {
  int n_items;
  long long key_tiles;
  bool split;  // some query tile has more than one chunk
};
PrefillPlan prefill_plan(int n_tokens, int start_pos, int chunk_tiles);
// Fills a.lpt, a.n_full and a.part_off (and a.bal_off when a.balanced)
// from a.n_tokens, a.start_pos, a.n_qtiles and a.chunk_tiles.  Balanced
// chunks need 1 < chunk_tiles <= kMaxLptChunk; otherwise a.balanced is
// cleared.
void prefill_order(PrefillArgs &a);
// Chunk planning (bnr_prefill_plan.cpp).  prefill_span: modelled span of a
// launch at ctiles key tiles per chunk.  plan_prefill_chunk: the planner's
// key tiles per chunk (kPrefillNoSplit: none) and *balanced for one shape,
// among the candidates that fit prefill_item_budget(cap, n_kv).
double prefill_span(int n_tokens, int start_pos, int n_kv, int ctiles, int n_cu, bool balanced,
                    bool q16 = false);
// The planner's choice for one launch shape: key tiles per chunk
// (kPrefillNoSplit: none), balanced chunks, 16-query halves.
struct PrefillChoice {
  int tiles, balanced, q16;
  int pairs;  // a paired 16-query launch (PairPlan) instead of chunks
};
// bal_pref / q16_pref: -1 either, 0 never, 1 always.  pair_pref != 0 (with
// q16_pref != 0 and pairs given): a paired launch wherever one fits, its
// plan in *pairs.
struct PairPlan;
PrefillChoice plan_prefill_chunk(int n_tokens, int start_pos, int n_kv, int n_cu, int bal_pref,
                                 int q16_pref, long long cap, int pair_pref = 0,
                                 PairPlan *pairs = nullptr);

// Paired plan of a 16-query launch that fits one dispatch round: the key
// tiles of every 16-query unit (queries 16 u .. 16 u + 15 attend key tiles
// 0 .. nk(u) - 1) are cut into pieces and the pieces packed into at most
// min(n_cu / n_kv, kMaxPairBins) bins of at most two pieces each, packed so
// that the slowest CU of a model of two workgroups sharing it finishes
// early.  piece[2 b + s] is piece s of bin b (s = 0 the longer one, started
// first):
//   w0 = kt0 | qt << 16 | half << 31        (unit u = 2 qt + half)
//   w1 = len | ch << 8 | nch << 16 | base << 24
// with len = 0 for an empty slot.  The chunks of a unit are its pieces in
// key order; a query tile's split units use slots base .. base + nch - 1
// (n_slots per kv head).  tau is the largest bin's key tiles, `span` the
// modelled span in prefill_span's units, model_us the largest bin's time in
// the planner's CU model of two workgroups (us).
struct PairPlan {
  int bins = 0, tau = 0, n_slots = 0;
  double span = 0.0, model_us = 0.0;
  unsigned piece[2 * kMaxPairBins][2] = {};
};
bool plan_prefill_pairs(int n_tokens, int start_pos, int n_kv, int n_cu, long long item_budget,
                        PairPlan &p);
// Constants of the 16-query halves in the span model (fixed cost, key tile,
// merge per extra chunk; a 32-query tile alone on a CU takes 1) and the
// span ratio below which the planner switches to them.
extern double g_pf16_fixed, g_pf16_tile, g_pf16_merge, g_pf16_margin;
long long prefill_item_budget(long long cap, int n_kv);
constexpr long long kPrefillMaxPlannedItems = 8192;
// persistent_wgs > 0: that many resident workgroups take items from a.queue.
// Stream-K runs: workgroup w of P takes units [sk_u0(w), sk_u0(w + 1)), a
// sequence of segments (the key tiles of one query tile within the run).
struct SkSeg {
  int h, qt, kt0, kt1, nk;  // key tiles kt0 .. kt1-1 of query tile qt (nk tiles) of kv head h
  long long qstart;         // unit of the query tile's key tile 0
};

__host__ __device__ inline long long sk_off(long long qt, int A) {
  return A * qt + qt * (qt - 1) / 2;  // units of query tiles 0 .. qt-1 of a head
}
__host__ __device__ inline long long sk_u0(int w, long long U, int P) {
  return (long long)w * U / P;
}
__host__ __device__ inline int sk_wg_of(long long u, long long U, int P) {
  return (int)(((u + 1) * P - 1) / U);  // the run holding unit u
}

// The segment starting at unit u of a run ending at uend.
__host__ __device__ inline SkSeg sk_seg(const PrefillArgs &a, long long u, long long uend) {
  const int nqt = a.n_qtiles, A = (a.start_pos + 31) / 32 + 1;
  const int nt_last = (a.start_pos + a.n_tokens - 1) / 32 + 1;
  SkSeg sg;
  sg.h = (int)(u / a.sk_per_head);
  const long long off = u - (long long)sg.h * a.sk_per_head;
  // largest qt with sk_off(qt) <= off: the quadratic's root, then exact fix-ups
  const double b = 2.0 * A - 1.0;
  int qt = (int)((sqrt(b * b + 8.0 * (double)off) - b) * 0.5);
  qt = qt < 0 ? 0 : (qt > nqt - 1 ? nqt - 1 : qt);
  while (qt + 1 < nqt && sk_off(qt + 1, A) <= off) ++qt;
  while (qt > 0 && sk_off(qt, A) > off) --qt;
  sg.qt = qt;
  sg.nk = qt + 1 < nqt ? A + qt : nt_last;
  sg.kt0 = (int)(off - sk_off(qt, A));
  sg.kt1 = (int)(sg.kt0 + (uend - u) < sg.nk ? sg.kt0 + (uend - u) : sg.nk);
  sg.qstart = u - sg.kt0;
  return sg;
}

hipError_t launch_prefill(const PrefillArgs &a, int group, int persistent_wgs, hipStream_t s);
// Stream-K prefill over `wgs` workgroups (a.sk_units, a.sk_per_head set by
// prefill_streamk_units).
hipError_t launch_prefill_streamk(const PrefillArgs &a, int group, int wgs, hipStream_t s);
// Units of a stream-K launch: sets a.sk_per_head and a.sk_units.
void prefill_streamk_units(PrefillArgs &a);
bool prefill_supported(int group);

// W2A8 ternary GEMV: out[i] = (float)dot(W[i], act) * scale, W packed 2 bits
// per weight, ceil(in_features/4) bytes per row.
struct TernaryGemvArgs {
  const uint8_t *weight;
  const int8_t *act;
  float *out;
  long long packed_cols;
  int out_features, in_features;
  float scale;  // weight_scale * act_absmax / 127, rounded as the reference does
};
// vec: 16-byte aligned rows and activations, ceil(in_features/4) % 16 == 0.
hipError_t launch_ternary_gemv(const TernaryGemvArgs &a, bool vec, hipStream_t s);

// Several ternary matrices that share one activation vector (q/k/v, or
// gate/up) in one launch: matrix i owns workgroups wg_off[i] .. wg_off[i+1]-1.
constexpr int kMaxGemvGroup = 8;
struct TernaryGemvGroupArgs {
  const uint8_t *weight[kMaxGemvGroup];
  float *out[kMaxGemvGroup];
  float scale[kMaxGemvGroup];
  int out_features[kMaxGemvGroup];
  int wg_off[kMaxGemvGroup + 1];
  const int8_t *act;
  long long packed_cols;
  int in_features, n;
  // When non-null, act_absmax is read from device memory and scale[i] is
  // formed in the kernel as (weight_scale[i] * act_absmax) / 127.
  const float *act_absmax_dev;
  float weight_scale[kMaxGemvGroup];
};
hipError_t launch_ternary_gemv_group(const TernaryGemvGroupArgs &a, bool vec, hipStream_t s);

// Modes of the layer-glue input x.
constexpr int kGluePlain = 0;     // x = a
constexpr int kGlueResidual = 1;  // x = a + b, written to h_out
constexpr int kGlueSqrelu = 2;    // x = max(a, 0)^2 * b

// Prologue of the norm-fused GEMV: x from a (and b) per mode (kGlue*),
// y = RMSNorm(x) with gamma, int8 absmax quantisation of y in LDS.
struct GemvNormArgs {
  int mode;
  const float *a, *b, *gamma;
  float eps;
  float *h_out;  // mode residual: a + b, written by workgroup 0; must not alias a or b
  int rows;      // rows per workgroup: 16, 32 or 64 (wg_off counts workgroups of that many)
};
constexpr int kMaxNormGemvK = 8192;
hipError_t launch_ternary_gemv_norm(const TernaryGemvGroupArgs &a, const GemvNormArgs &p, bool vec,
                                    hipStream_t s);

// LM head with i8 weights: out[v] = dot(weight[v], hidden) * scales[v].
struct LmHeadArgs {
  const float *hidden;
  const int8_t *weight;   // [vocab_size x hidden_size]
  const float *scales;    // [vocab_size]
  float *out;             // [vocab_size]
  long long vocab_size;
  int hidden_size;
};
// vec: 16-byte aligned weights with hidden_size % 16 == 0, hidden 16-byte aligned.
hipError_t launch_lm_head_i8(const LmHeadArgs &a, bool vec, hipStream_t s);

// Layer glue (bnr_glue.hip).
struct NormQuantArgs {
  int mode;
  const float *a, *b;
  const float *gamma;   // RMSNorm weight, or null: no normalisation
  float eps;
  int n;
  float *h_out;         // mode kGlueResidual: a + b (may alias a)
  float *y_out;         // optional: normalised values
  int8_t *q_out;        // optional: absmax int8 quantisation of y
  float *scale_out;     // optional (with q_out): max|y| / 127
  float *act_absmax;    // optional (with q_out): scale * 127, what the projections take
  unsigned *done;       // host-slice calls: pinned host word set to seq at the end (or null)
  unsigned seq;
};
hipError_t launch_norm_quant(const NormQuantArgs &a, hipStream_t s);
// done (host-slice calls): workgroup w stores seq into done[w] at its end;
// sqrelu_blocks(n) workgroups.
hipError_t launch_sqrelu(const float *gate, const float *up, float *out, long long n, hipStream_t s,
                         unsigned *done = nullptr, unsigned seq = 0);
inline long long sqrelu_blocks(long long n) {
  const long long b = (n + 255) / 256;
  return b < 4096 ? b : 4096;
}
hipError_t launch_residual(float *h, const float *delta, long long n, hipStream_t s);

}  // namespace bnr
