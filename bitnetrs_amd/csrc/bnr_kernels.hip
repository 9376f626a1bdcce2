// bnr_kernels.hip -- gfx950 decode-side kernels of the GQA attention hot path.
//
//  rope_append_kernel  half-split RoPE of q/k + head-major KV append
//                       (rope_append_vec_kernel: four pairs per thread;
//                       rope_append_row_kernel: one token per workgroup)
//  decode_kernel<G,RPG> split-K decode attention, head_dim 128, optional
//                       fused RoPE + append, last-workgroup merge
//  decode_merge_kernel  second kernel of the two-launch merge
//  decode_generic_kernel any head_dim / group size
//
// Wave64 throughout.  The decode kernel reads each K/V row of a kv head once
// and serves the G query heads of the group from registers (the reference
// re-reads every row once per query head, bitnet-cpu/src/attention.rs:
// 170-204).  The reference-merge decode kernel is in bnr_decode_ref.hip, the
// causal prefill in bnr_prefill.hip.
#include <type_traits>

#include "bnr_device.h"
#include "bnr_internal.h"

#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

namespace bnr {
namespace {

__global__ __launch_bounds__(256) void rope_append_kernel(RopeAppendArgs a) {
  const int half = a.head_dim >> 1;
  const int slots = a.n_heads + 2 * a.n_kv;
  const long long total = (long long)a.n_tokens * slots * half;
  for (long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * blockDim.x) {
    const int i = (int)(idx % half);
    const long long rest = idx / half;
    const int slot = (int)(rest % slots);
    const int tok = (int)(rest / slots);
    const int pos = a.start_pos + tok;
    if (slot < a.n_heads + a.n_kv) {
      const bool is_q = slot < a.n_heads;
      float *x = is_q ? a.q + ((long long)tok * a.n_heads + slot) * a.head_dim
                      : a.k + ((long long)tok * a.n_kv + (slot - a.n_heads)) * a.head_dim;
      const float c = a.cos_tab[(long long)pos * half + i];
      const float s = a.sin_tab[(long long)pos * half + i];
      float lo, hi;
      rot_pair(x[i], x[i + half], c, s, lo, hi);
      x[i] = lo;
      x[i + half] = hi;
      if (!is_q && a.k_cache) {
        float *dst = a.k_cache + (slot - a.n_heads) * a.kv_stride + (long long)pos * a.head_dim;
        dst[i] = lo;
        dst[i + half] = hi;
      }
    } else if (a.v_cache) {
      const int hv = slot - a.n_heads - a.n_kv;
      const float *src = a.v + ((long long)tok * a.n_kv + hv) * a.head_dim;
      float *dst = a.v_cache + hv * a.kv_stride + (long long)pos * a.head_dim;
      dst[i] = src[i];
      dst[i + half] = src[i + half];
    }
  }
  if (a.done) signal_host(a.done + blockIdx.x, a.seq);
}

// Four consecutive pairs (i .. i+3, i+half .. i+half+3) per thread, 16-byte
// accesses: the same rotation as rope_append_kernel, element for element.
// Needs half % 4 == 0 and 16-byte aligned rows and tables.
__global__ __launch_bounds__(256) void rope_append_vec_kernel(RopeAppendArgs a) {
  const int half = a.head_dim >> 1, quads = half >> 2;
  const int slots = a.n_heads + 2 * a.n_kv;
  const long long total = (long long)a.n_tokens * slots * quads;
  for (long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * blockDim.x) {
    const int i = 4 * (int)(idx % quads);
    const long long rest = idx / quads;
    const int slot = (int)(rest % slots);
    const int tok = (int)(rest / slots);
    const int pos = a.start_pos + tok;
    if (slot < a.n_heads + a.n_kv) {
      const bool is_q = slot < a.n_heads;
      float *x = is_q ? a.q + ((long long)tok * a.n_heads + slot) * a.head_dim
                      : a.k + ((long long)tok * a.n_kv + (slot - a.n_heads)) * a.head_dim;
      const float4 c = ld4(a.cos_tab + (long long)pos * half + i);
      const float4 sn = ld4(a.sin_tab + (long long)pos * half + i);
      float4 lo, hi;
      rot4(ld4(x + i), ld4(x + i + half), c, sn, lo, hi);
      st4(x + i, lo);
      st4(x + i + half, hi);
      if (!is_q && a.k_cache) {
        float *dst = a.k_cache + (slot - a.n_heads) * a.kv_stride + (long long)pos * a.head_dim;
        st4(dst + i, lo);
        st4(dst + i + half, hi);
      }
    } else if (a.v_cache) {
      const int hv = slot - a.n_heads - a.n_kv;
      const float *src = a.v + ((long long)tok * a.n_kv + hv) * a.head_dim;
      float *dst = a.v_cache + hv * a.kv_stride + (long long)pos * a.head_dim;
      st4(dst + i, ld4(src + i));
      st4(dst + i + half, ld4(src + i + half));
    }
  }
  if (a.done) signal_host(a.done + blockIdx.x, a.seq);
}

// One token per workgroup, head_dim 128 (device calls; no host signal):
// thread t rotates quad t % 16 of heads t / 16, t / 16 + 16, ... (the q
// heads, then the k heads) with one load of its table quad, and copies the
// token's v rows a float4 at a time.  The same rotation as
// rope_append_kernel, element for element.  All of a thread's loads are
// issued before its first store (a store to q or k could otherwise alias
// the next load for the compiler).  The raw rows are read once:
// non-temporal loads (1024 tokens x 20/5 heads: 9.9 -> 8.2 us per graph
// step on MI355X).
__global__ __launch_bounds__(256) void rope_append_row_kernel(RopeAppendArgs a) {
  constexpr int half = kHeadDim / 2;
  const int tok = blockIdx.x, pos = a.start_pos + tok;
  const int t = threadIdx.x, i = 4 * (t & 15);
  const int nrot = a.n_heads + a.n_kv;
  auto row = [&](int h) {
    return h < a.n_heads ? a.q + ((long long)tok * a.n_heads + h) * kHeadDim
                         : a.k + ((long long)tok * a.n_kv + (h - a.n_heads)) * kHeadDim;
  };
  auto finish = [&](int h, float *x, float4 lo, float4 hi) {
    st4(x + i, lo);
    st4(x + i + half, hi);
    if (h >= a.n_heads && a.k_cache) {
      float *dst = a.k_cache + (h - a.n_heads) * a.kv_stride + (long long)pos * kHeadDim;
      st4(dst + i, lo);
      st4(dst + i + half, hi);
    }
  };
  // the v row first: its loads go out with the q/k loads instead of after
  // their stores (which they could alias)
  constexpr int F = kHeadDim / 4;  // float4 per row
  const bool has_v = a.v_cache && t < a.n_kv * F;
  float4 vv = make_float4(0.f, 0.f, 0.f, 0.f);
  if (has_v) vv = ld4_nt(a.v + ((long long)tok * a.n_kv + t / F) * kHeadDim + 4 * (t % F));
  const float4 c = ld4(a.cos_tab + (long long)pos * half + i);
  const float4 sn = ld4(a.sin_tab + (long long)pos * half + i);
  for (int h = t >> 4; h < nrot; h += 32) {
    // heads h and h + 16: both rows loaded, then both rotated and stored
    const int h2 = h + 16;
    float *x1 = row(h), *x2 = h2 < nrot ? row(h2) : x1;
    const float4 a_lo = ld4_nt(x1 + i), a_hi = ld4_nt(x1 + i + half);
    const float4 b_lo = ld4_nt(x2 + i), b_hi = ld4_nt(x2 + i + half);
    float4 lo, hi;
    rot4(a_lo, a_hi, c, sn, lo, hi);
    float4 lo2, hi2;
    rot4(b_lo, b_hi, c, sn, lo2, hi2);
    finish(h, x1, lo, hi);
    if (h2 < nrot) finish(h2, x2, lo2, hi2);
  }
  if (has_v) st4(a.v_cache + (t / F) * a.kv_stride + (long long)pos * kHeadDim + 4 * (t % F), vv);
  if (a.v_cache) {
    for (int f = t + 256; f < a.n_kv * F; f += 256) {  // n_kv > 8 only
      const int hv = f / F, j = 4 * (f % F);
      const float4 v = ld4_nt(a.v + ((long long)tok * a.n_kv + hv) * kHeadDim + j);
      st4(a.v_cache + hv * a.kv_stride + (long long)pos * kHeadDim + j, v);
    }
  }
}

// Merge the nsplit partial states of (sequence b, kv head h) into the
// output.  CH (<= 64) splits per round: one load round trip, then wave w
// computes the round's max and split weights of q head g = w, w+4, ... (one
// lane per split, wave reductions), and every lane forms its outputs as an
// independent weighted sum.  CH is matched to the split count so that no
// load is spent on a clamped duplicate.  AGENT: the partials were written by
// other workgroups of this launch (agent-coherent loads); otherwise by an
// earlier kernel (plain loads).  lds: at least 64*G + 3*G floats.
template <int G, bool AGENT, int CH>
__device__ __forceinline__ void merge_splits(const DecodeArgs &a, int b, int h, int nsplit,
                                             float *lds) {
  static_assert(CH % 4 == 0 && CH <= 64, "splits per round: one per lane of a wave");
  constexpr int D = kHeadDim;
  constexpr int NE = G * D;                 // output elements of this kv head
  constexpr int EPL = NE >= 512 ? 2 : 1;    // adjacent elements per lane (one 8-byte load)
  constexpr int NT = NE / EPL;              // lanes with work (<= 256)
  constexpr int GPW = (G + 3) / 4;          // q heads per wave
  float *s_w = lds;             // [G][CH] split weights of the round
  float *s_M = s_w + CH * G;    // [G] running max
  float *s_L = s_M + G;         // [G] running sum
  float *s_sc = s_L + G;        // [G] rescale of the earlier rounds
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int gs0 = a.split_off[b];
  const long long step = (long long)a.n_kv * NE;
  const float *po = a.ws_o + ((long long)gs0 * a.n_kv + h) * NE;
  if (tid < G) {
    s_M[tid] = -INFINITY;
    s_L[tid] = 0.f;
  }
  const int e0 = (tid % NT) * EPL;  // first element of this lane (lanes >= NT shadow)
  const int g0 = e0 / D;
  float Or[EPL];
#pragma unroll
  for (int k = 0; k < EPL; ++k) Or[k] = 0.f;
  for (int c0 = 0; c0 < nsplit; c0 += CH) {
    const int n = min(CH, nsplit - c0);
    // One batch of loads; split indices past the end are clamped (their
    // weight is zero), so there are no branches between loads.
    float ov[EPL][CH];
    auto load_o = [&](int u) {
      const float *pu = po + (long long)min(c0 + u, nsplit - 1) * step + e0;
      if (EPL == 2) {
        const unsigned long long r =
            AGENT ? __hip_atomic_load(reinterpret_cast<const unsigned long long *>(pu),
                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                  : *reinterpret_cast<const unsigned long long *>(pu);
        const float2 f = __builtin_bit_cast(float2, r);
        ov[0][u] = f.x;
        ov[EPL - 1][u] = f.y;
      } else {
        ov[0][u] = AGENT ? ld_agent(pu) : *pu;
      }
    };
#pragma unroll
    for (int u = 0; u < CH; ++u) load_o(u);
    float2 mlr[GPW];
    auto load_ml = [&](int r) {
      const int g = min(wv + 4 * r, G - 1);
      const float *ml = reinterpret_cast<const float *>(
          &a.ws_ml[((long long)(gs0 + min(c0 + lane, nsplit - 1)) * a.n_kv + h) * G + g]);
      mlr[r] = AGENT ? make_float2(ld_agent(ml), ld_agent(ml + 1)) : make_float2(ml[0], ml[1]);
    };
#pragma unroll
    for (int r = 0; r < GPW; ++r) load_ml(r);
    __syncthreads();  // earlier round's readers of s_w / s_sc are done
#pragma unroll
    for (int r = 0; r < GPW; ++r) {
      const int g = wv + 4 * r;
      if (g >= G) continue;
      const float m = lane < n ? mlr[r].x : -INFINITY;
      const float m_old = s_M[g];
      const float mn = fmaxf(m_old, wave_max(m));
      const float w = lane < n ? fast_exp2(m - mn) : 0.f;
      const float ls = wave_sum(w * mlr[r].y);
      if (lane < CH) s_w[g * CH + lane] = w;
      if (lane == 0) {
        const float sc = fast_exp2(m_old - mn);  // 0 on the first round
        s_sc[g] = sc;
        s_L[g] = fmaf(s_L[g], sc, ls);
        s_M[g] = mn;
      }
    }
    __syncthreads();
    const float4 *w4 = reinterpret_cast<const float4 *>(s_w + g0 * CH);
    const float sc = s_sc[g0];
#pragma unroll
    for (int k = 0; k < EPL; ++k) Or[k] *= sc;
#pragma unroll
    for (int u4 = 0; u4 < CH / 4; ++u4) {
      const float4 w = w4[u4];
#pragma unroll
      for (int k = 0; k < EPL; ++k) {
        Or[k] = fmaf(w.x, ov[k][4 * u4 + 0], Or[k]);
        Or[k] = fmaf(w.y, ov[k][4 * u4 + 1], Or[k]);
        Or[k] = fmaf(w.z, ov[k][4 * u4 + 2], Or[k]);
        Or[k] = fmaf(w.w, ov[k][4 * u4 + 3], Or[k]);
      }
    }
  }
  if (tid < NT) {
    const float inv = 1.0f / s_L[g0];
    float *o = a.out + b * a.out_bstride + (long long)h * NE + e0;
#pragma unroll
    for (int k = 0; k < EPL; ++k) o[k] = Or[k] * inv;
  }
}

// ---------------------------------------------------------------------------
// Split-K decode attention, head_dim 128.
//
// Workgroup = 256 lanes = 16 row groups of 16 lanes.  Lane j of a row group
// holds dims {4j..4j+3} and {64+4j..64+4j+3} of a row: one float4 from each
// half, so one instruction of a wave reads four 256-byte row halves, and the
// half-split RoPE pair (i, i+64) of a q/k element sits in the same lane.
//
// Row of pass p, iteration i of row group rg: t0 + p*16*RPG + i*16 + rg.
// The first pass's K/V loads are issued before anything else so that the
// kernel pays one memory round trip, not a q round trip followed by a K/V
// one.  Each row group keeps an online-softmax state (m, l, o[G][8 dims per
// lane]); the 16 states merge through LDS into one (m, l, o) per workgroup.
//
// With several splits per (sequence, kv head), each workgroup stores its
// state with agent-coherent stores, waits for them to complete and takes a
// ticket with a relaxed agent-scope atomic; the workgroup that draws the last
// ticket merges all splits (agent-coherent loads, one round trip per 64
// splits) and writes the output.  It also resets the ticket counter, so no
// memset is needed between launches.
// ---------------------------------------------------------------------------
template <int G, int RPG, bool INLINE, bool RAGGED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu((RPG == 4 && !INLINE && G <= 4) ? 3 : 1)))
void decode_kernel(DecodeArgs a) {
  constexpr int D = kHeadDim;
  __shared__ float s_o[16][G][D];
  __shared__ float s_m[G][16];
  __shared__ float s_l[G][16];
  __shared__ float s_w[G][16];
  __shared__ float s_M[G], s_L[G];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int rg = tid >> 4;
  const int j = tid & 15;

  // Grid (max splits, kv heads, sequences): every kernel argument this
  // workgroup needs is fetched in one batch (no dependent lookups); splits
  // past a shorter sequence's count exit at once.
  const int b = blockIdx.z;
  const int s = blockIdx.x;
  const int nsplit = a.split_off[b + 1] - a.split_off[b];
  if (RAGGED && s >= nsplit) return;  // only when sequences differ in split count
  const int h = blockIdx.y;
  const int pos = a.positions[b];
  const int L = pos + 1;
  const int t0 = s * a.rows_per_split;
  const int t1 = min(t0 + a.rows_per_split, L);

  float *kc = a.k_cache + b * a.cache_bstride + h * a.kv_stride;
  float *vc = a.v_cache + b * a.cache_bstride + h * a.kv_stride;

  // ---- loads of the first pass, in use order: q (+cos/sin), K rows, V rows.
  // One batch, one memory round trip; rows are consumed as they arrive.
  const float *qb = a.q + b * a.q_bstride + (long long)h * G * D;
  float4 qlo[G], qhi[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    qlo[g] = ld4(qb + g * D + 4 * j);
    qhi[g] = ld4(qb + g * D + 64 + 4 * j);
  }
  float4 cs = make_float4(1.f, 1.f, 1.f, 1.f), sn = make_float4(0.f, 0.f, 0.f, 0.f);
  const bool rope = a.cos_tab != nullptr;
  if (rope) {
    cs = ld4(a.cos_tab + (long long)pos * 64 + 4 * j);
    sn = ld4(a.sin_tab + (long long)pos * 64 + 4 * j);
  }
  // The new token's raw key and value (fused append), ahead of the K/V
  // batch: a load issued after it would hold this workgroup's first dot
  // product until the whole batch had arrived.
  const bool fused = a.k_new != nullptr;
  const bool own_pos = fused && pos >= t0 && pos < t1;
  const bool need_new = fused && (own_pos || (a.k_rot && s == 0));
  float4 nklo = make_float4(0.f, 0.f, 0.f, 0.f), nkhi = nklo, nvlo = nklo, nvhi = nklo;
  if (need_new) {
    const float *kn = a.k_new + b * a.kn_bstride + h * D;
    const float *vn = a.v_new + b * a.kn_bstride + h * D;
    nklo = ld4(kn + 4 * j);
    nkhi = ld4(kn + 64 + 4 * j);
    nvlo = ld4(vn + 4 * j);
    nvhi = ld4(vn + 64 + 4 * j);
  }
  float4 klo[RPG], khi[RPG], vlo[RPG], vhi[RPG];
  bool valid[RPG];
  auto load_pass = [&](int tp) {
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
      const int t = tp + i * 16 + rg;
      valid[i] = t < t1;
      const long long off = (long long)(valid[i] ? t : t0) * D;
      klo[i] = ld4_nt(kc + off + 4 * j);
      khi[i] = ld4_nt(kc + off + 64 + 4 * j);
    }
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
      const long long off = (long long)(valid[i] ? tp + i * 16 + rg : t0) * D;
      vlo[i] = ld4_nt(vc + off + 4 * j);
      vhi[i] = ld4_nt(vc + off + 64 + 4 * j);
    }
  };
  load_pass(t0);
  __builtin_amdgcn_sched_barrier(0);  // keep every load of the batch ahead of the math

  if (rope) {
#pragma unroll
    for (int g = 0; g < G; ++g) rot4(qlo[g], qhi[g], cs, sn, qlo[g], qhi[g]);
  }
  if (a.q_rot && s == 0 && rg == 0) {
    float *qr = a.q_rot + b * a.q_bstride + (long long)h * G * D;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      st4(qr + g * D + 4 * j, qlo[g]);
      st4(qr + g * D + 64 + 4 * j, qhi[g]);
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    qlo[g] = scale4(a.scale_log2, qlo[g]);
    qhi[g] = scale4(a.scale_log2, qhi[g]);
  }

  // ---- the new token's rotated key (fused append; without a table the row
  // is appended as given) ----
  if (need_new && rope) {
    rot4(nklo, nkhi, cs, sn, nklo, nkhi);
    if (a.k_rot && s == 0 && rg == 0) {
      float *kr = a.k_rot + b * a.kn_bstride + h * D;
      st4(kr + 4 * j, nklo);
      st4(kr + 64 + 4 * j, nkhi);
    }
  }

  // ---- online softmax over this workgroup's rows ----
  float m_run[G], l_run[G];
  float4 olo[G], ohi[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
    olo[g] = make_float4(0.f, 0.f, 0.f, 0.f);
    ohi[g] = olo[g];
  }

  for (int p = 0; p < a.passes; ++p) {
    const int tp = t0 + p * 16 * RPG;
    if (tp >= t1) break;
    if (p > 0) load_pass(tp);
    if (own_pos) {
      // The new row, also where a masked row past the split's end was
      // clamped onto it (that cache row is not written yet; its stale
      // contents would make the zero weight 0 * inf = NaN).
#pragma unroll
      for (int i = 0; i < RPG; ++i) {
        const int t = tp + i * 16 + rg;
        if ((valid[i] ? t : t0) == pos) {
          klo[i] = nklo;
          khi[i] = nkhi;
          vlo[i] = nvlo;
          vhi[i] = nvhi;
          if (valid[i]) {
            st4(kc + (long long)pos * D + 4 * j, nklo);
            st4(kc + (long long)pos * D + 64 + 4 * j, nkhi);
            st4(vc + (long long)pos * D + 4 * j, nvlo);
            st4(vc + (long long)pos * D + 64 + 4 * j, nvhi);
          }
        }
      }
    }
    // FAST: the first pass with every row of the pass valid (every split of
    // a context that is a multiple of the split size) -- no row masks and
    // no rescale of the empty running state.  Only in the in-kernel merge
    // variants: the second copy of the loop body would make the batched
    // kernel (three workgroups per CU) spill.
    auto attend = [&](auto fast) {
      constexpr bool FAST = decltype(fast)::value;
      float sc[RPG][G];
#pragma unroll
      for (int i = 0; i < RPG; ++i) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float d = row_sum16(dot8(qlo[g], qhi[g], klo[i], khi[i]));
          sc[i][g] = (FAST || valid[i]) ? d : -INFINITY;
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mp = sc[0][g];
#pragma unroll
        for (int i = 1; i < RPG; ++i) mp = fmaxf(mp, sc[i][g]);
        if (FAST) {
          float lsum = 0.f;
          float4 alo, ahi;
#pragma unroll
          for (int i = 0; i < RPG; ++i) {
            const float pr = fast_exp2(sc[i][g] - mp);
            lsum += pr;
            alo = i == 0 ? scale4(pr, vlo[0]) : axpy4(pr, vlo[i], alo);
            ahi = i == 0 ? scale4(pr, vhi[0]) : axpy4(pr, vhi[i], ahi);
          }
          m_run[g] = mp;
          l_run[g] = lsum;
          olo[g] = alo;
          ohi[g] = ahi;
          continue;
        }
        const float m_new = fmaxf(m_run[g], mp);
        if (m_new == -INFINITY) continue;  // no valid row yet in this row group
        const float alpha = fast_exp2(m_run[g] - m_new);
        float lsum = l_run[g] * alpha;
        float4 alo = scale4(alpha, olo[g]), ahi = scale4(alpha, ohi[g]);
#pragma unroll
        for (int i = 0; i < RPG; ++i) {
          const float pr = valid[i] ? fast_exp2(sc[i][g] - m_new) : 0.f;
          lsum += pr;
          alo = axpy4(pr, vlo[i], alo);
          ahi = axpy4(pr, vhi[i], ahi);
        }
        m_run[g] = m_new;
        l_run[g] = lsum;
        olo[g] = alo;
        ohi[g] = ahi;
      }
    };
    if (INLINE && p == 0 && tp + 16 * RPG <= t1)
      attend(std::true_type{});
    else
      attend(std::false_type{});
  }

  // ---- merge the 16 row-group states through LDS ----
#pragma unroll
  for (int g = 0; g < G; ++g) {
    st4(&s_o[rg][g][4 * j], olo[g]);
    st4(&s_o[rg][g][64 + 4 * j], ohi[g]);
    if (j == 0) {
      s_m[g][rg] = m_run[g];
      s_l[g][rg] = l_run[g];
    }
  }
  __syncthreads();

  // Row-group weights once per (q head, row group): lane 16g + r of wave 0
  // takes row group r of head g; a DPP row is one head.
  if (tid < 64) {
#pragma unroll
    for (int g0 = 0; g0 < G; g0 += 4) {
      const int g = g0 + (tid >> 4), r = tid & 15;
      if (g < G) {
        const float mr = s_m[g][r];
        const float M = row_max16(mr);
        const float w = fast_exp2(mr - M);  // 0 for an empty row group
        const float Ls = row_sum16(s_l[g][r] * w);
        s_w[g][r] = w;
        if (r == 0) {
          s_M[g] = M;
          s_L[g] = Ls;
        }
      }
    }
  }
  __syncthreads();

  const int gs = a.split_off[b] + s;  // global split index
  // This split's unnormalised output element e (q head e / D, dim e % D).
  auto split_out = [&](int e) {
    const int g = e / D, dim = e % D;
    float O = 0.f;
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const float4 w4 = *reinterpret_cast<const float4 *>(&s_w[g][4 * r4]);
      O = fmaf(w4.x, s_o[4 * r4][g][dim], O);
      O = fmaf(w4.y, s_o[4 * r4 + 1][g][dim], O);
      O = fmaf(w4.z, s_o[4 * r4 + 2][g][dim], O);
      O = fmaf(w4.w, s_o[4 * r4 + 3][g][dim], O);
    }
    return O;
  };
  if (nsplit == 1 || !INLINE) {
    for (int e = tid; e < G * D; e += 256) {
      const int g = e / D, dim = e % D;
      const float O = split_out(e);
      if (nsplit == 1) {
        a.out[b * a.out_bstride + ((long long)h * G + g) * D + dim] = O / s_L[g];
      } else {
        a.ws_o[((long long)gs * a.n_kv + h) * G * D + e] = O;
        if (dim == 0) a.ws_ml[((long long)gs * a.n_kv + h) * G + g] = make_float2(s_M[g], s_L[g]);
      }
    }
    return;
  }

  for (int e = tid; e < G * D; e += 256) {
    st_agent(&a.ws_o[((long long)gs * a.n_kv + h) * G * D + e], split_out(e));
    if (e % D == 0) {
      const int g = e / D;
      float *ml = reinterpret_cast<float *>(&a.ws_ml[((long long)gs * a.n_kv + h) * G + g]);
      st_agent(ml, s_M[g]);
      st_agent(ml + 1, s_L[g]);
    }
  }

  // ---- ticket: the last workgroup of this (sequence, kv head) merges ----
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have completed
  __syncthreads();
  unsigned *ctr = a.counters + (b * a.n_kv + h) * kCounterStride;
  if (tid == 0) {
    const unsigned ticket =
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (ticket == (unsigned)(nsplit - 1));
  }
  __syncthreads();
  if (!s_last) return;
  if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // One round (one load round trip) for up to 64 splits, sized so that at
  // most a quarter of the loads are clamped duplicates.
  if (nsplit <= 16)
    merge_splits<G, true, 16>(a, b, h, nsplit, &s_o[0][0][0]);
  else if (nsplit <= 32)
    merge_splits<G, true, 32>(a, b, h, nsplit, &s_o[0][0][0]);
  else if (nsplit <= 48)
    merge_splits<G, true, 48>(a, b, h, nsplit, &s_o[0][0][0]);
  else
    merge_splits<G, true, 64>(a, b, h, nsplit, &s_o[0][0][0]);
}

// Second kernel of the two-launch decode: one workgroup of 256 lanes per
// (sequence, kv head, q head) merges that q head's split partials, written by
// decode_kernel<.., false> (the kernel boundary makes them visible; plain
// loads).  Lane t loads the (max, sum) of split t; the split weights come from
// a block max; lane (d, p) = (t % 128, t / 128) accumulates the splits of
// parity p for output dim d, all loads of a round in flight together.
template <int G>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
  constexpr int D = kHeadDim, CH = 32;
  __shared__ float s_w[kMaxSplits];
  __shared__ float s_red[8];
  __shared__ float s_o[D];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int h = blockIdx.x / G, g = blockIdx.x % G, b = blockIdx.y;
  const int nsplit = a.split_off[b + 1] - a.split_off[b];
  if (nsplit == 1) return;
  const int gs0 = a.split_off[b];
  const long long step = (long long)a.n_kv * G * D;
  const float *po = a.ws_o + ((long long)gs0 * a.n_kv + h) * G * D + g * D;
  const int d = tid & (D - 1), par = tid >> 7;

  // Split partials of this lane (parity par), first round, issued with the
  // (max, sum) loads so that both arrive in one round trip.
  float ov[CH];
#pragma unroll
  for (int u = 0; u < CH; ++u) ov[u] = po[(long long)min(2 * u + par, nsplit - 1) * step + d];
  float2 ml = make_float2(-INFINITY, 0.f);
  if (tid < nsplit) ml = a.ws_ml[((long long)(gs0 + tid) * a.n_kv + h) * G + g];

  // Block max of the split maxima.
  const float wm = wave_max(ml.x);
  if (lane == 0) s_red[wv] = wm;
  __syncthreads();
  const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  const float w = tid < nsplit ? fast_exp2(ml.x - M) : 0.f;
  if (tid < nsplit) s_w[tid] = w;
  const float wl = wave_sum(w * ml.y);
  if (lane == 0) s_red[4 + wv] = wl;
  __syncthreads();
  const float Ls = (s_red[4] + s_red[5]) + (s_red[6] + s_red[7]);

  float o = 0.f;
  for (int c0 = 0; c0 < nsplit; c0 += 2 * CH) {
    if (c0 > 0) {
#pragma unroll
      for (int u = 0; u < CH; ++u)
        ov[u] = po[(long long)min(c0 + 2 * u + par, nsplit - 1) * step + d];
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int sp = c0 + 2 * u + par;
      if (sp < nsplit) o = fmaf(s_w[sp], ov[u], o);
    }
  }
  if (par == 1) s_o[d] = o;
  __syncthreads();
  if (par == 0) a.out[b * a.out_bstride + ((long long)h * G + g) * D + d] = (o + s_o[d]) / Ls;
}

// ---------------------------------------------------------------------------
// Generic decode attention (any head_dim, any group size).  Same three
// phases as attention::masked_attention (bitnet-cpu/src/attention.rs:
// 183-204): scores, softmax, weighted sum of V rows.
// ---------------------------------------------------------------------------
__device__ float block_reduce(float v, bool is_max, float *red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(v, off);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(256) void decode_generic_kernel(DecodeGenericArgs a) {
  __shared__ float red[4];
  const int h = blockIdx.x;
  const int kv = h / a.group;
  const float *qh = a.q + (long long)h * a.head_dim;
  const float *kb = a.k_cache + kv * a.kv_stride;
  const float *vb = a.v_cache + kv * a.kv_stride;
  float *sc = a.scores + (long long)h * a.L;

  float mx = -INFINITY;
  for (int t = threadIdx.x; t < a.L; t += blockDim.x) {
    const float *kr = kb + (long long)t * a.head_dim;
    float d = 0.f;
    for (int i = 0; i < a.head_dim; ++i) d = fmaf(qh[i], kr[i], d);
    d *= a.scale;
    sc[t] = d;
    mx = fmaxf(mx, d);
  }
  mx = block_reduce(mx, true, red);
  float sum = 0.f;
  for (int t = threadIdx.x; t < a.L; t += blockDim.x) {
    const float e = expf(sc[t] - mx);
    sc[t] = e;
    sum += e;
  }
  sum = block_reduce(sum, false, red);
  const float inv = 1.0f / sum;
  __syncthreads();
  for (int dim = threadIdx.x; dim < a.head_dim; dim += blockDim.x) {
    float o = 0.f;
    for (int t = 0; t < a.L; ++t) o = fmaf(sc[t] * inv, vb[(long long)t * a.head_dim + dim], o);
    a.out[(long long)h * a.head_dim + dim] = o;
  }
}

// Plain streaming read of two device ranges (the K and V caches of one
// layer), for measurement: what one launch can read of that many bytes.
// One 16-byte load per thread over a grid that covers both ranges (the
// fastest of the shapes measured on MI355X); a workgroup's loads feed a sum
// that is stored only if it equals an impossible value, so they are kept.
__global__ __launch_bounds__(512) void stream_read_kernel(const float4 *a, long long na,
                                                          const float4 *b, long long nb) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (i < na) v = a[i];
  else if (i - na < nb) v = b[i - na];
  const float sum = (v.x + v.y) + (v.z + v.w);
  if (sum == -1.2345e-30f && i < na) const_cast<float4 *>(a)[i] = v;
}

// Streaming read of two device ranges, laid end to end, in one round over
// the CUs: workgroup w reads float4 words [w NL T, (w+1) NL T) (T threads),
// each lane issuing its NL 16-byte loads (words T apart) before
// it uses any of them, so NL loads per lane are in flight at once; NT: the
// loads are non-temporal.  The sum of a lane's words is stored only if it
// equals an impossible value, so no load is removed.
template <int NL, bool NT>
__global__ __launch_bounds__(1024) void stream_read_nl_kernel(const float4 *a, long long na,
                                                              const float4 *b, long long nb) {
  const long long base = (long long)blockIdx.x * NL * blockDim.x + threadIdx.x;
  float4 v[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const long long idx = base + (long long)i * blockDim.x;
    const float4 *p = idx < na ? a + idx : (idx - na < nb ? b + (idx - na) : nullptr);
    v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (p) {
      if constexpr (NT) {
        typedef float f4v __attribute__((ext_vector_type(4)));
        const f4v w = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(p));
        v[i] = make_float4(w.x, w.y, w.z, w.w);
      } else {
        v[i] = *p;
      }
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < NL; ++i) sum += (v[i].x + v[i].y) + (v[i].z + v[i].w);
  if (sum == -1.2345e-30f && base < na) const_cast<float4 *>(a)[base] = v[0];
}

template <int G, bool INLINE, bool RAGGED>
hipError_t launch_decode_gir(const DecodeArgs &a, hipStream_t s) {
  dim3 grid(a.max_splits, a.n_kv, a.batch), block(256);
  // Every rpg 1..8 for the in-kernel merge (small launches); 1, 2, 4, 8 for
  // the two-launch merge (large launches use 4).
  switch (a.rpg) {
    case 1: decode_kernel<G, 1, INLINE, RAGGED><<<grid, block, 0, s>>>(a); break;
    case 2: decode_kernel<G, 2, INLINE, RAGGED><<<grid, block, 0, s>>>(a); break;
    case 4: decode_kernel<G, 4, INLINE, RAGGED><<<grid, block, 0, s>>>(a); break;
    case 8: decode_kernel<G, 8, INLINE, RAGGED><<<grid, block, 0, s>>>(a); break;
    default:
      if constexpr (INLINE) {
        switch (a.rpg) {
          case 3: decode_kernel<G, 3, true, RAGGED><<<grid, block, 0, s>>>(a); break;
          case 5: decode_kernel<G, 5, true, RAGGED><<<grid, block, 0, s>>>(a); break;
          case 6: decode_kernel<G, 6, true, RAGGED><<<grid, block, 0, s>>>(a); break;
          case 7: decode_kernel<G, 7, true, RAGGED><<<grid, block, 0, s>>>(a); break;
          default: return hipErrorInvalidValue;
        }
      } else {
        return hipErrorInvalidValue;
      }
  }
  if (!INLINE && a.max_splits > 1)
    decode_merge_kernel<G><<<dim3(a.n_kv * G, a.batch), block, 0, s>>>(a);
  return hipGetLastError();
}

template <int G, bool INLINE>
hipError_t launch_decode_gi(const DecodeArgs &a, hipStream_t s) {
  // Uniform split counts (always so for one sequence): no early-exit check.
  bool ragged = false;
  for (int b = 0; b < a.batch; ++b)
    ragged |= (a.split_off[b + 1] - a.split_off[b]) != a.max_splits;
  return ragged ? launch_decode_gir<G, INLINE, true>(a, s) : launch_decode_gir<G, INLINE, false>(a, s);
}

template <int G>
hipError_t launch_decode_g(const DecodeArgs &a, hipStream_t s) {
  if (G <= 4 && a.merge_ref) return launch_decode_ref(a, s);
  return a.merge_inline ? launch_decode_gi<G, true>(a, s) : launch_decode_gi<G, false>(a, s);
}
}  // namespace

namespace {
bool rope_append_vec(const RopeAppendArgs &a) {
  auto a16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
  const int half = a.head_dim / 2;
  return half % 4 == 0 && a16(a.q) && a16(a.k) && a16(a.cos_tab) && a16(a.sin_tab) &&
         (!a.v_cache || (a16(a.v) && a16(a.v_cache))) && (!a.k_cache || a16(a.k_cache)) &&
         a.kv_stride % 4 == 0;
}
}  // namespace

long long rope_append_blocks(const RopeAppendArgs &a) {
  const int half = a.head_dim / 2;
  const long long total =
      (long long)a.n_tokens * (a.n_heads + 2 * a.n_kv) * (rope_append_vec(a) ? half / 4 : half);
  return std::min<long long>((total + 255) / 256, 65536);
}

hipError_t launch_rope_append(const RopeAppendArgs &a, hipStream_t s) {
  const bool vec = rope_append_vec(a);
  if (vec && !a.done && a.head_dim == kHeadDim && a.n_tokens > 0) {
    rope_append_row_kernel<<<dim3((unsigned)a.n_tokens), dim3(256), 0, s>>>(a);
    return hipGetLastError();
  }
  const long long blocks = rope_append_blocks(a);
  if (blocks == 0) return hipSuccess;
  if (vec)
    rope_append_vec_kernel<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(a);
  else
    rope_append_kernel<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeArgs &a, hipStream_t s) {
  switch (a.group) {
    case 1: return launch_decode_g<1>(a, s);
    case 2: return launch_decode_g<2>(a, s);
    case 4: return launch_decode_g<4>(a, s);
    case 8: return launch_decode_g<8>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_stream_read(const void *a, long long a_bytes, const void *b, long long b_bytes,
                              hipStream_t s) {
  const long long na = a_bytes / 16, nb = b_bytes / 16;
  if (na + nb == 0) return hipSuccess;
  const long long wgs = (na + nb + 511) / 512;
  if (wgs > 0x7fffffffLL) return hipErrorInvalidValue;
  stream_read_kernel<<<dim3((unsigned)wgs), dim3(512), 0, s>>>(
      static_cast<const float4 *>(a), na, static_cast<const float4 *>(b), nb);
  return hipGetLastError();
}

hipError_t launch_stream_read_shape(const void *a, long long a_bytes, const void *b,
                                    long long b_bytes, int threads, int loads, bool nt,
                                    hipStream_t s) {
  const long long na = a_bytes / 16, nb = b_bytes / 16;
  if (na + nb == 0) return hipSuccess;
  if (threads < 64 || threads > 1024 || threads % 64) return hipErrorInvalidValue;
  const long long per_wg = (long long)threads * loads;
  const long long wgs = (na + nb + per_wg - 1) / per_wg;
  if (wgs > 0x7fffffffLL) return hipErrorInvalidValue;
  const float4 *pa = static_cast<const float4 *>(a), *pb = static_cast<const float4 *>(b);
  const dim3 grid((unsigned)wgs), block((unsigned)threads);
#define BNR_STREAM_CASE(NL)                                                          \
  case NL:                                                                           \
    if (nt) stream_read_nl_kernel<NL, true><<<grid, block, 0, s>>>(pa, na, pb, nb);  \
    else stream_read_nl_kernel<NL, false><<<grid, block, 0, s>>>(pa, na, pb, nb);    \
    break;
  switch (loads) {
    BNR_STREAM_CASE(1)
    BNR_STREAM_CASE(2)
    BNR_STREAM_CASE(4)
    BNR_STREAM_CASE(8)
    BNR_STREAM_CASE(16)
    default: return hipErrorInvalidValue;
  }
#undef BNR_STREAM_CASE
  return hipGetLastError();
}

hipError_t launch_decode_generic(const DecodeGenericArgs &a, hipStream_t s) {
  decode_generic_kernel<<<dim3(a.n_heads), dim3(256), 0, s>>>(a);
  return hipGetLastError();
}
}  // namespace bnr
